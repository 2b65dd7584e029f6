"""ctypes binding of libnyion_hip.so (the C ABI in include/nyion_hip.h).

The product is the HIP library; this module only passes device pointers and
sizes through the C ABI.  Tensors come from PyTorch (device memory and the
current HIP stream).  There is no fallback: if the library is missing or the
device is not a gfx950, every call raises NyionError.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libnyion_hip.so")

KV_F32 = 0
KV_Q4_20B = 1
KV_F16 = 2

MEM_HOST_PINNED = 0
MEM_DEVICE_LOCAL = 1
MEM_UNIFIED_MAPPED = 2

OK = 0
ERR_INVALID = -1
ERR_UNSUPPORTED = -2
ERR_NO_DEVICE = -3
ERR_OOM = -4
ERR_LAUNCH = -5
ERR_WORKSPACE = -6
ERR_RANGE = -7


class NyionError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"nyion error {code}: {msg}")
        self.code = code


class Allocation(C.Structure):
    _fields_ = [("ptr", C.c_void_p), ("size", C.c_size_t), ("location", C.c_int32),
                ("_pad", C.c_int32), ("device_handle", C.c_uint64)]


vp, i32, u32, i64, f32, sz = C.c_void_p, C.c_int, C.c_uint32, C.c_int64, C.c_float, C.c_size_t


class SystemSnapshot(C.Structure):
    _fields_ = [("seq_len", C.c_int64), ("dspark_accept_rate", C.c_double),
                ("is_prefill", C.c_int32), ("predictive_throttle", C.c_int32)]


class FuguConfig(C.Structure):
    _fields_ = [("sparse_attention_threshold", C.c_int64), ("sparse_window", C.c_int32),
                ("sparse_random_samples", C.c_int32), ("n_heads", C.c_int32),
                ("head_dim", C.c_int32)]


class AttentionStrategy(C.Structure):
    _fields_ = [("kind", C.c_int32), ("window", C.c_int32), ("num_random", C.c_int32),
                ("sentinel_stride", C.c_int32), ("num_dspark", C.c_int32), ("_pad", C.c_int32)]


ATTN_FULL, ATTN_SPARSE, ATTN_SPARSE_DSPARK = 0, 1, 2

# name -> (restype, argtypes); the full list of symbols the header declares.
SIGNATURES = {
    "nyion_last_error": (C.c_char_p, []),
    "nyion_init": (i32, [i32]),
    "nyion_device_count": (i32, []),
    "nyion_sync": (i32, []),
    "nyion_version": (C.c_char_p, []),
    "nyion_take_status": (i32, [vp]),
    "nyion_attention_node_scratch_bytes": (sz, [u32, u32, u32, u32]),
    "nyion_attention_node": (i32, [vp, vp, vp, vp, vp, u32, u32, u32, u32, u32, i32, vp]),
    "gpu_attention_device": (i32, [vp, vp, vp, vp, i32, i32, i32, i32, i32]),
    "gpu_attention_streamed": (i32, [vp, vp, vp, vp, i32, i32, i32, i32, i32, vp]),
    "nyion_paged_decode_workspace_size": (sz, [i32, i32, i32, i32, i32, i32, i32]),
    "nyion_paged_decode_attention": (i32, [vp, vp, vp, vp, i32, vp, vp, i32, i32, i32, i32, i32,
                                           i32, i32, i32, i32, i32, f32, vp, vp, sz, vp]),
    "nyion_paged_decode_attention_noalloc": (i32, [vp, vp, vp, vp, i32, vp, vp, i32, i32, i32, i32,
                                                   i32, i32, i32, i32, i32, i32, f32, vp, vp]),
    "nyion_paged_decode_attention_tracked": (i32, [vp, vp, vp, vp, i32, vp, vp, i32, i32, i32, i32,
                                                   i32, i32, i32, i32, i32, i32, f32, vp, vp, sz,
                                                   vp, i32, vp, i32, vp]),
    "nyion_paged_decode_attention_scores": (i32, [vp, vp, vp, vp, i32, vp, vp, i32, i32, i32, i32,
                                                  i32, i32, i32, i32, i32, i32, f32, vp, vp, sz,
                                                  vp, i32, vp]),
    "nyion_paged_decode_importance": (i32, [vp, vp, i32, i32, i32, i32, i32, vp, i32, vp, i32, vp]),
    "nyion_paged_decode_attention_tracked_pipelined": (i32, [vp, vp, vp, vp, i32, vp, vp, i32, i32,
                                                             i32, i32, i32, i32, i32, i32, i32, i32,
                                                             f32, vp, vp, sz, vp, i32, vp, vp, i32,
                                                             vp]),
    "nyion_paged_decode_positions_workspace_size": (sz, [i32, i32, i32, i32, i32]),
    "nyion_paged_decode_attention_positions": (i32, [vp, vp, vp, vp, i32, vp, vp, i32, i32, i32,
                                                     i32, i32, i32, i32, i32, f32, vp, vp, sz,
                                                     vp]),
    "nyion_decode_workspace_init": (i32, [vp, sz, vp]),
    "nyion_layer_state_create": (vp, [i32, i32, i32, i32, i32]),
    "nyion_layer_state_upload_kv": (i32, [vp, i32, vp, vp, i32]),
    "nyion_layer_state_attention": (i32, [vp, i32, vp, vp, i32, i32]),
    "nyion_layer_state_sync": (i32, [vp]),
    "nyion_layer_state_destroy": (None, [vp]),
    "nyion_fugu_config_default": (i32, [i32, i32, C.POINTER(FuguConfig)]),
    "nyion_fugu_decide_attention": (i32, [C.POINTER(SystemSnapshot), C.POINTER(FuguConfig),
                                          C.POINTER(AttentionStrategy)]),
    "nyion_fugu_positions": (i32, [vp, vp, i32, i32, i32, vp, i32, i32, vp, i32, vp, vp]),
    "nyion_set_decode_partition_tokens": (i32, [i32]),
    "nyion_get_decode_partition_tokens": (i32, [i32, i32, i32, i32]),
    "nyion_prefill_attention_bf16": (i32, [vp, vp, vp, i32, i32, i32, i32, i32, f32, vp, vp, vp,
                                           vp, i32, i32, i32, i32, vp]),
    "nyion_prefill_attention_bf16_ctx": (i32, [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32,
                                               f32, vp, vp, vp, vp, i32, i32, i32, i32, vp]),
    "nyion_kv_write": (i32, [vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, vp, vp, vp]),
    "nyion_kv_append_batch": (i32, [vp, vp, vp, i32, vp, i32, i32, i32, i32, i32, i32, vp, vp,
                                    vp]),
    "nyion_kv_gather": (i32, [vp, vp, i32, i32, i32, i32, i32, i32, vp, vp]),
    "nyion_kv_gather_bf16": (i32, [vp, vp, i32, i32, i32, i32, i32, i32, vp, vp]),
    "sparse_attention_q4": (None, [C.c_uint64] * 5 + [i32] * 5),
    "nyion_zone_page_id": (i64, [i64]),
    "nyion_zone_page_tokens": (i32, [i64]),
    "nyion_zone_kv_write": (i32, [vp, vp, i64, vp, i32, i32, i32, i32, i32, i32, i32, i32, vp,
                                  vp, vp]),
    "nyion_zone_kv_gather": (i32, [vp, i64, vp, i32, i32, i32, i32, i32, i32, i32, vp, vp]),
    "nyion_zone_decode_attention": (i32, [vp, vp, vp, i64, vp, i32, i32, i32, vp, vp, i32, i32,
                                          i32, i32, i32, i32, i32, i32, f32, vp, vp, sz, vp]),
    "nyion_attention_sparse_q4_workspace_size": (sz, [i32, i32, i32, i32, i32, i32]),
    "nyion_attention_sparse_q4": (i32, [vp, vp, vp, i64, vp, i32, i32, i32, vp, vp, i32, i32, i32,
                                        i32, i32, i32, i32, vp, vp, sz, vp]),
    "nyion_page_policy_create": (vp, [i32, i32, i32]),
    "nyion_page_policy_destroy": (None, [vp]),
    "nyion_page_policy_ensure": (i32, [vp, i32, i32, vp, i32, C.POINTER(C.c_int)]),
    "nyion_page_policy_record": (i32, [vp, i32, C.c_double]),
    "nyion_page_policy_reset": (i32, [vp]),
    "nyion_page_policy_state": (i32, [vp, i32, C.POINTER(C.c_int), C.POINTER(C.c_double)]),
    "nyion_page_policy_lru": (i32, [vp, vp, i32]),
    "nyion_kv_pool_create": (vp, [i32, i32, i32, i32, i32, i32, i32, i32]),
    "nyion_kv_pool_destroy": (None, [vp]),
    "nyion_kv_pool_layer": (i32, [vp, i32, C.POINTER(C.c_void_p), C.POINTER(C.c_void_p)]),
    "nyion_kv_pool_table": (vp, [vp]),
    "nyion_kv_pool_policy": (vp, [vp]),
    "nyion_kv_pool_ensure": (i32, [vp, i32, i32, vp]),
    "nyion_kv_pool_record_importance": (i32, [vp, vp, i32, C.c_double]),
    "nyion_kv_pool_stats": (i32, [vp, C.POINTER(C.c_int64), C.POINTER(C.c_int64),
                                  C.POINTER(C.c_int64), C.POINTER(C.c_int64)]),
    "nyion_kv_pool_cold_slot": (vp, [vp, i32]),
    "nyion_gemv_q4k": (i32, [vp, vp, vp, i32, i32, vp]),
    "nyion_gemv_q4k_multi": (i32, [vp, vp, vp, vp, i32, i32, vp]),
    "nyion_gemv_q4k_batched": (i32, [vp, vp, i64, vp, i64, i32, i32, i32, vp]),
    "nyion_gemv_q6k": (i32, [vp, vp, vp, i32, i32, vp]),
    "nyion_gemv_q6k_batched": (i32, [vp, vp, i64, vp, i64, i32, i32, i32, vp]),
    "nyion_gemv_specs": (i32, [vp, i32, vp]),
    "gpu_graph_create_attention": (vp, [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32]),
    "gpu_graph_replay_attention": (i32, [vp, vp]),
    "gpu_graph_destroy": (None, [vp]),
    "gpu_attention_streamed_half": (i32, [vp, vp, vp, vp, i32, i32, i32, i32, i32, vp]),
    "gpu_graph_create_attention_half": (vp, [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32]),
    "nyion_rope_lut_init": (i32, [vp, i32, i32, vp]),
    "nyion_rope_kv_append": (i32, [vp, vp, vp, vp, i32, vp, i32, i32, i32, i32, vp, vp, vp, i32,
                                   i32, i32, i32, vp]),
    "nyion_q4_dequant": (i32, [vp, i64, i32, vp, vp]),
    "nyion_q4_quantize": (i32, [vp, i64, i32, vp, vp]),
    "nyion_hma_create": (vp, [sz, sz]),
    "nyion_hma_alloc": (i32, [vp, sz, i32, C.POINTER(Allocation)]),
    "nyion_hma_free": (i32, [vp, C.POINTER(Allocation)]),
    "nyion_hma_upload": (i32, [vp, C.POINTER(Allocation), vp, sz]),
    "nyion_hma_download": (i32, [vp, vp, C.POINTER(Allocation), sz]),
    "nyion_hma_reset": (i32, [vp]),
    "nyion_hma_stats": (i32, [vp, i32, C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]),
    "nyion_hma_has_device": (i32, [vp]),
    "nyion_hma_destroy": (None, [vp]),
    "mojo_softmax_padic": (None, [vp, vp, i32, f32]),
    "mojo_stokes_init": (vp, [i32]),
    "mojo_stokes_append": (None, [vp, i32, vp, vp, f32]),
    "mojo_stokes_free": (None, [vp]),
    "nyion_softmax_padic_dev": (i32, [vp, vp, i32, f32, vp]),
    "nyion_stokes_count": (i32, [vp]),
    "nyion_stokes_read": (i32, [vp, vp, vp, vp]),
}

_lib = None


def load():
    """Load the library (raises NyionError if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise NyionError(ERR_NO_DEVICE, f"{LIB_PATH} not built (run __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    return load().nyion_last_error().decode()


def check(rc: int, what: str = "") -> None:
    if rc != OK:
        raise NyionError(rc, f"{what}: {last_error()}")


# ----------------------------------------------------------------------------
# torch helpers
# ----------------------------------------------------------------------------

def _torch():
    import torch
    return torch


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def stream_handle(stream=None) -> int | None:
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def init(device: int = 0) -> None:
    check(load().nyion_init(device), "nyion_init")


def take_status(stream=None) -> tuple[int, str]:
    """Waits for `stream`, takes the device's range-status word: (0, "") or
    (ERR_RANGE, message)."""
    rc = load().nyion_take_status(stream_handle(stream))
    if rc not in (OK, ERR_RANGE):
        check(rc, "nyion_take_status")
    return rc, ("" if rc == OK else last_error())


def node_scratch_bytes(n_heads, n_kv_heads, seq_len, head_dim) -> int:
    return int(load().nyion_attention_node_scratch_bytes(n_heads, n_kv_heads, seq_len, head_dim))


# ----------------------------------------------------------------------------
# decode
# ----------------------------------------------------------------------------

def attention_node(q, k, v, out, n_heads, n_kv_heads, seq_len, head_dim, kv_stride,
                   kv_dtype=KV_F32, scores=None, stream=None):
    rc = load().nyion_attention_node(ptr(q), ptr(k), ptr(v), ptr(scores), ptr(out), n_heads,
                                     n_kv_heads, seq_len, head_dim, kv_stride, kv_dtype,
                                     stream_handle(stream))
    check(rc, "nyion_attention_node")


def decode_workspace_size(batch, n_heads, n_kv_heads, head_dim, max_ctx, window=0,
                          global_stride=0) -> int:
    return int(load().nyion_paged_decode_workspace_size(batch, n_heads, n_kv_heads, head_dim,
                                                         max_ctx, window, global_stride))


def alloc_workspace(nbytes: int, device="cuda"):
    """Decode workspace: zero-filled (the split-K arrival counters start at 0
    and every call leaves them at 0)."""
    torch = _torch()
    if nbytes <= 0:
        return None
    return torch.zeros(nbytes, dtype=torch.uint8, device=device)


def paged_decode(q, k_pool, v_pool, block_tables, ctx_lens, out, n_heads, n_kv_heads, head_dim,
                 block_tokens, kv_dtype=KV_F32, window=0, global_stride=0, max_ctx=None,
                 q_pos=None, scale=0.0, workspace=None, stream=None):
    """q [B][Hq][D] f32, pools [num_blocks][Hkv][block_tokens][row], block_tables [B][max_blocks]
    int32, ctx_lens [B] int32.  All device tensors."""
    B = q.shape[0]
    max_blocks = block_tables.shape[1]
    num_blocks = k_pool.shape[0]
    if max_ctx is None:
        max_ctx = int(ctx_lens.max().item())
    need = decode_workspace_size(B, n_heads, n_kv_heads, head_dim, max_ctx, window, global_stride)
    if workspace is None and need:
        workspace = alloc_workspace(need, q.device)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    rc = load().nyion_paged_decode_attention(
        ptr(q), ptr(k_pool), ptr(v_pool), ptr(block_tables), max_blocks, ptr(ctx_lens),
        ptr(q_pos), B, n_heads, n_kv_heads, head_dim, block_tokens, num_blocks, kv_dtype, window,
        global_stride, max_ctx, scale, ptr(out), ptr(workspace), ws_bytes, stream_handle(stream))
    check(rc, "nyion_paged_decode_attention")
    return workspace


def prepare_paged_decode(q, k_pool, v_pool, block_tables, ctx_lens, out, n_heads, n_kv_heads,
                         head_dim, block_tokens, max_ctx, kv_dtype=KV_F32, window=0,
                         global_stride=0, q_pos=None, scale=0.0, workspace=None, stream=None):
    """paged_decode with every argument resolved once: returns a no-argument
    callable that only crosses the C ABI (what a compiled caller pays), for
    loops that launch many decode calls."""
    B = q.shape[0]
    need = decode_workspace_size(B, n_heads, n_kv_heads, head_dim, max_ctx, window, global_stride)
    if workspace is None and need:
        workspace = alloc_workspace(need, q.device)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    fn = load().nyion_paged_decode_attention
    args = (ptr(q), ptr(k_pool), ptr(v_pool), ptr(block_tables), block_tables.shape[1],
            ptr(ctx_lens), ptr(q_pos), B, n_heads, n_kv_heads, head_dim, block_tokens,
            k_pool.shape[0], kv_dtype, window, global_stride, max_ctx, scale, ptr(out),
            ptr(workspace), ws_bytes, stream_handle(stream))
    keep = (q, k_pool, v_pool, block_tables, ctx_lens, out, q_pos, workspace)

    def call():
        rc = fn(*args)
        if rc != 0:
            check(rc, "nyion_paged_decode_attention")

    call.keep = keep
    return call


def paged_decode_tracked(q, k_pool, v_pool, block_tables, ctx_lens, out, importance, n_heads,
                         n_kv_heads, head_dim, block_tokens, kv_dtype=KV_F32, window=0,
                         global_stride=0, max_ctx=None, q_pos=None, scale=0.0, workspace=None,
                         scores=None, stream=None):
    """paged_decode plus importance [B][>= max_ctx] f64 (accumulated), the tracked
    form of the executor's Full decode call.  scores: optional f32 scratch
    [B][Hq][>= max_ctx + 2]."""
    torch = _torch()
    B = q.shape[0]
    if max_ctx is None:
        max_ctx = int(ctx_lens.max().item())
    need = decode_workspace_size(B, n_heads, n_kv_heads, head_dim, max_ctx, window, global_stride)
    if workspace is None and need:
        workspace = alloc_workspace(need, q.device)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    if scores is None:
        scores = torch.empty((B, n_heads, max_ctx + 2), dtype=torch.float32, device=q.device)
    rc = load().nyion_paged_decode_attention_tracked(
        ptr(q), ptr(k_pool), ptr(v_pool), ptr(block_tables), block_tables.shape[1], ptr(ctx_lens),
        ptr(q_pos), B, n_heads, n_kv_heads, head_dim, block_tokens, k_pool.shape[0], kv_dtype,
        window, global_stride, max_ctx, scale, ptr(out), ptr(workspace), ws_bytes, ptr(scores),
        scores.shape[-1], ptr(importance), importance.shape[-1], stream_handle(stream))
    check(rc, "nyion_paged_decode_attention_tracked")
    return workspace


def paged_decode_scores(q, k_pool, v_pool, block_tables, ctx_lens, out, scores, n_heads,
                        n_kv_heads, head_dim, block_tokens, kv_dtype=KV_F32, window=0,
                        global_stride=0, max_ctx=None, q_pos=None, scale=0.0, workspace=None,
                        stream=None):
    """The tracked decode's first launch: paged_decode plus the scores (and each
    row's max and denominator) in scores [B][Hq][>= max_ctx + 2] f32."""
    B = q.shape[0]
    if max_ctx is None:
        max_ctx = int(ctx_lens.max().item())
    need = decode_workspace_size(B, n_heads, n_kv_heads, head_dim, max_ctx, window, global_stride)
    if workspace is None and need:
        workspace = alloc_workspace(need, q.device)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    rc = load().nyion_paged_decode_attention_scores(
        ptr(q), ptr(k_pool), ptr(v_pool), ptr(block_tables), block_tables.shape[1], ptr(ctx_lens),
        ptr(q_pos), B, n_heads, n_kv_heads, head_dim, block_tokens, k_pool.shape[0], kv_dtype,
        window, global_stride, max_ctx, scale, ptr(out), ptr(workspace), ws_bytes, ptr(scores),
        scores.shape[-1], stream_handle(stream))
    check(rc, "nyion_paged_decode_attention_scores")
    return workspace


def paged_decode_tracked_pipelined(q, k_pool, v_pool, block_tables, ctx_lens, out, scores,
                                   prev_scores, prev_importance, n_heads, n_kv_heads, head_dim,
                                   block_tokens, kv_dtype=KV_F32, window=0, global_stride=0,
                                   max_ctx=None, q_pos=None, scale=0.0, workspace=None,
                                   stream=None):
    """One launch: this call's decode with its scores (as paged_decode_scores)
    and the importance sum of prev_scores (the previous call's, same
    sequences and lengths) into prev_importance; prev_scores None for the
    first call of a chain."""
    B = q.shape[0]
    if max_ctx is None:
        max_ctx = int(ctx_lens.max().item())
    need = decode_workspace_size(B, n_heads, n_kv_heads, head_dim, max_ctx, window, global_stride)
    if workspace is None and need:
        workspace = alloc_workspace(need, q.device)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    imp_stride = 0 if prev_importance is None else prev_importance.shape[-1]
    rc = load().nyion_paged_decode_attention_tracked_pipelined(
        ptr(q), ptr(k_pool), ptr(v_pool), ptr(block_tables), block_tables.shape[1], ptr(ctx_lens),
        ptr(q_pos), B, n_heads, n_kv_heads, head_dim, block_tokens, k_pool.shape[0], kv_dtype,
        window, global_stride, max_ctx, scale, ptr(out), ptr(workspace), ws_bytes, ptr(scores),
        scores.shape[-1], ptr(prev_scores), ptr(prev_importance), imp_stride,
        stream_handle(stream))
    check(rc, "nyion_paged_decode_attention_tracked_pipelined")
    return workspace


def paged_decode_importance(ctx_lens, scores, importance, n_heads, window=0, global_stride=0,
                            max_ctx=None, q_pos=None, stream=None):
    """The tracked decode's second launch: importance [B][>= max_ctx] f64 +=
    the normalised probabilities summed over heads, from scores as
    paged_decode_scores left them."""
    B = scores.shape[0]
    if max_ctx is None:
        max_ctx = int(ctx_lens.max().item())
    rc = load().nyion_paged_decode_importance(
        ptr(ctx_lens), ptr(q_pos), B, n_heads, window, global_stride, max_ctx, ptr(scores),
        scores.shape[-1], ptr(importance), importance.shape[-1], stream_handle(stream))
    check(rc, "nyion_paged_decode_importance")


def paged_decode_positions(q, k_pool, v_pool, block_tables, positions, n_positions, out, n_heads,
                           n_kv_heads, head_dim, block_tokens, kv_dtype=KV_F32, scale=0.0,
                           workspace=None, stream=None):
    B = q.shape[0]
    max_pos = positions.shape[1]
    need = int(load().nyion_paged_decode_positions_workspace_size(B, n_heads, n_kv_heads, head_dim,
                                                                  max_pos))
    if workspace is None and need:
        workspace = alloc_workspace(need, q.device)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    rc = load().nyion_paged_decode_attention_positions(
        ptr(q), ptr(k_pool), ptr(v_pool), ptr(block_tables), block_tables.shape[1], ptr(positions),
        ptr(n_positions), max_pos, B, n_heads, n_kv_heads, head_dim, block_tokens,
        k_pool.shape[0], kv_dtype, scale, ptr(out), ptr(workspace), ws_bytes,
        stream_handle(stream))
    check(rc, "nyion_paged_decode_attention_positions")
    return workspace


def fugu_decide_attention(seq_len, n_heads, head_dim, is_prefill=False, predictive_throttle=False,
                          dspark_accept_rate=0.0, cfg=None) -> AttentionStrategy:
    """FuguOrchestrator::decide_attention (host; no device needed)."""
    if cfg is None:
        cfg = FuguConfig()
        check(load().nyion_fugu_config_default(n_heads, head_dim, C.byref(cfg)), "fugu config")
    snap = SystemSnapshot(seq_len, dspark_accept_rate, int(is_prefill), int(predictive_throttle))
    out = AttentionStrategy()
    check(load().nyion_fugu_decide_attention(C.byref(snap), C.byref(cfg), C.byref(out)),
          "fugu decide")
    return out


def fugu_positions(ctx_lens, window, sentinel_stride, dspark, positions, n_positions, q_pos=None,
                   stream=None):
    """Device attention_fugu position sets: dspark [B][n] int32 -> positions [B][max], n_positions [B]."""
    B = ctx_lens.shape[0]
    nd = 0 if dspark is None else dspark.shape[1]
    rc = load().nyion_fugu_positions(ptr(ctx_lens), ptr(q_pos), B, window, sentinel_stride,
                                     ptr(dspark), nd, nd, ptr(positions), positions.shape[1],
                                     ptr(n_positions), stream_handle(stream))
    check(rc, "nyion_fugu_positions")


class LayerState:
    """PerLayerGpuState: per-layer sliding-window rings on the device, host q/k/v/out."""

    def __init__(self, window, n_heads, n_kv_heads, head_dim, n_layers):
        self.h = load().nyion_layer_state_create(window, n_heads, n_kv_heads, head_dim, n_layers)
        if not self.h:
            raise NyionError(-1, last_error())

    def upload_kv(self, layer, k, v, pos):
        import numpy as np
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        check(load().nyion_layer_state_upload_kv(self.h, layer, k.ctypes.data, v.ctypes.data, pos),
              "layer_state_upload_kv")

    def attention(self, layer, q, pos, seq_len):
        import numpy as np
        q = np.ascontiguousarray(q, np.float32)
        out = np.empty_like(q)
        check(load().nyion_layer_state_attention(self.h, layer, q.ctypes.data, out.ctypes.data,
                                                 pos, seq_len), "layer_state_attention")
        return out

    def close(self):
        if self.h:
            load().nyion_layer_state_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def set_partition_tokens(tokens: int) -> None:
    check(load().nyion_set_decode_partition_tokens(tokens), "set_partition_tokens")


def partition_tokens(batch, n_kv_heads, head_dim, max_len) -> int:
    return int(load().nyion_get_decode_partition_tokens(batch, n_kv_heads, head_dim, max_len))


# ----------------------------------------------------------------------------
# prefill
# ----------------------------------------------------------------------------

def prefill_bf16(q, k, v, out, n_heads, n_kv_heads, head_dim, causal=True, scale=0.0,
                 k_pool=None, v_pool=None, block_table=None, block_tokens=16,
                 kv_dtype=KV_F32, start_pos=0, stream=None):
    """q [N][Hq][D], k/v [N][Hkv][D] bf16 (torch.bfloat16); out [N][Hq][D] f32."""
    n = q.shape[0]
    num_blocks = 0 if k_pool is None else k_pool.shape[0]
    rc = load().nyion_prefill_attention_bf16(
        ptr(q), ptr(k), ptr(v), n, n_heads, n_kv_heads, head_dim, 1 if causal else 0, scale,
        ptr(out), ptr(k_pool), ptr(v_pool), ptr(block_table), block_tokens, num_blocks, kv_dtype,
        start_pos, stream_handle(stream))
    check(rc, "nyion_prefill_attention_bf16")


def prefill_bf16_ctx(q, k, v, k_hist, v_hist, out, n_heads, n_kv_heads, head_dim, causal=True,
                     scale=0.0, k_pool=None, v_pool=None, block_table=None, block_tokens=16,
                     kv_dtype=KV_F32, start_pos=None, stream=None):
    """Chunk after a cached prefix: k_hist/v_hist [n_hist][Hkv][D] bf16 (or None for
    n_hist = 0); the KV write defaults to start_pos = n_hist."""
    n = q.shape[0]
    n_hist = 0 if k_hist is None else k_hist.shape[0]
    if start_pos is None:
        start_pos = n_hist
    num_blocks = 0 if k_pool is None else k_pool.shape[0]
    rc = load().nyion_prefill_attention_bf16_ctx(
        ptr(q), ptr(k), ptr(v), ptr(k_hist), ptr(v_hist), n_hist, n, n_heads, n_kv_heads,
        head_dim, 1 if causal else 0, scale, ptr(out), ptr(k_pool), ptr(v_pool), ptr(block_table),
        block_tokens, num_blocks, kv_dtype, start_pos, stream_handle(stream))
    check(rc, "nyion_prefill_attention_bf16_ctx")


# ----------------------------------------------------------------------------
# KV cache
# ----------------------------------------------------------------------------

def kv_write(k_pool, v_pool, block_table, block_tokens, n_kv_heads, head_dim, kv_dtype,
             start_pos, k, v, stream=None):
    rc = load().nyion_kv_write(ptr(k_pool), ptr(v_pool), ptr(block_table), block_tokens,
                               k_pool.shape[0], n_kv_heads, head_dim, kv_dtype, start_pos,
                               k.shape[0], ptr(k), ptr(v), stream_handle(stream))
    check(rc, "nyion_kv_write")


def kv_append_batch(k_pool, v_pool, block_tables, positions, block_tokens, n_kv_heads, head_dim,
                    kv_dtype, k, v, stream=None):
    rc = load().nyion_kv_append_batch(ptr(k_pool), ptr(v_pool), ptr(block_tables),
                                      block_tables.shape[1], ptr(positions), positions.shape[0],
                                      block_tokens, k_pool.shape[0], n_kv_heads, head_dim,
                                      kv_dtype, ptr(k), ptr(v), stream_handle(stream))
    check(rc, "nyion_kv_append_batch")


def rope_lut(head_dim, max_ctx, device="cuda", stream=None):
    """Device RoPE table [max_ctx][head_dim/2][2] f32 (init_rope_lut)."""
    torch = _torch()
    lut = torch.empty((max_ctx, head_dim // 2, 2), dtype=torch.float32, device=device)
    check(load().nyion_rope_lut_init(ptr(lut), head_dim, max_ctx, stream_handle(stream)),
          "nyion_rope_lut_init")
    return lut


def rope_kv_append(q, k, v, lut, positions, k_pool, v_pool, block_tables, n_heads, n_kv_heads,
                   head_dim, block_tokens, kv_dtype=KV_F32, stream=None):
    """RoPE on q (in place) and k, then k/v of each sequence into the pools."""
    rc = load().nyion_rope_kv_append(
        ptr(q), ptr(k), ptr(v), ptr(lut), lut.shape[0], ptr(positions), q.shape[0], n_heads,
        n_kv_heads, head_dim, ptr(k_pool), ptr(v_pool), ptr(block_tables), block_tables.shape[1],
        block_tokens, k_pool.shape[0], kv_dtype, stream_handle(stream))
    check(rc, "nyion_rope_kv_append")


def kv_gather(pool, block_table, block_tokens, n_kv_heads, head_dim, kv_dtype, n_tokens, out,
              stream=None):
    rc = load().nyion_kv_gather(ptr(pool), ptr(block_table), block_tokens, pool.shape[0],
                                n_kv_heads, head_dim, kv_dtype, n_tokens, ptr(out),
                                stream_handle(stream))
    check(rc, "nyion_kv_gather")


# Reference-shaped zone pools (PagedKVCache geometry): pools are 1-D device
# tensors of pool units (f32 / float16 elements, uint8 bytes for Q4-20B);
# page_base [n_pages] (or [B][n_pages] for decode) int64 offsets in units.

def zone_page_id(pos: int) -> int:
    return int(load().nyion_zone_page_id(pos))


def zone_page_tokens(pos: int) -> int:
    return int(load().nyion_zone_page_tokens(pos))


def zone_kv_write(k_pool, v_pool, page_base, n_layers, layer, n_kv_heads, head_dim, kv_dtype,
                  start_pos, k, v, stream=None):
    rc = load().nyion_zone_kv_write(ptr(k_pool), ptr(v_pool), k_pool.numel(), ptr(page_base),
                                    page_base.shape[-1], n_layers, layer, n_kv_heads, head_dim,
                                    kv_dtype, start_pos, k.shape[0], ptr(k), ptr(v),
                                    stream_handle(stream))
    check(rc, "nyion_zone_kv_write")


def zone_kv_gather(pool, page_base, n_layers, layer, n_kv_heads, head_dim, kv_dtype, n_tokens,
                   out, stream=None):
    rc = load().nyion_zone_kv_gather(ptr(pool), pool.numel(), ptr(page_base), page_base.shape[-1],
                                     n_layers, layer, n_kv_heads, head_dim, kv_dtype, n_tokens,
                                     ptr(out), stream_handle(stream))
    check(rc, "nyion_zone_kv_gather")


def zone_decode(q, k_pool, v_pool, page_bases, n_layers, layer, ctx_lens, out, n_heads,
                n_kv_heads, head_dim, kv_dtype=KV_F32, window=0, global_stride=0, max_ctx=None,
                q_pos=None, scale=0.0, workspace=None, stream=None):
    """q [B][Hq][D] f32, page_bases [B][max_pages] int64, ctx_lens [B] int32."""
    B = q.shape[0]
    if max_ctx is None:
        max_ctx = int(ctx_lens.max().item())
    need = decode_workspace_size(B, n_heads, n_kv_heads, head_dim, max_ctx, window, global_stride)
    if workspace is None and need:
        workspace = alloc_workspace(need, q.device)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    rc = load().nyion_zone_decode_attention(
        ptr(q), ptr(k_pool), ptr(v_pool), k_pool.numel(), ptr(page_bases), page_bases.shape[1],
        n_layers, layer, ptr(ctx_lens), ptr(q_pos), B, n_heads, n_kv_heads, head_dim, kv_dtype,
        window, global_stride, max_ctx, scale, ptr(out), ptr(workspace), ws_bytes,
        stream_handle(stream))
    check(rc, "nyion_zone_decode_attention")
    return workspace


def attention_sparse_q4(q, k_pool, v_pool, page_bases, n_layers, layer, ctx_lens, out, n_heads,
                        n_kv_heads, head_dim, window, global_stride, max_ctx=None, q_pos=None,
                        workspace=None, stream=None):
    """ops::attention_sparse_q4 over zone pools of Q4-20B rows (uint8 tensors);
    q [B][Hq][D] f32, page_bases [B][max_pages] int64, ctx_lens [B] int32."""
    B = q.shape[0]
    if max_ctx is None:
        max_ctx = int(ctx_lens.max().item())
    need = load().nyion_attention_sparse_q4_workspace_size(B, n_heads, n_kv_heads, head_dim, window,
                                                           max_ctx)
    if workspace is None and need:
        workspace = alloc_workspace(need, q.device)  # zero-filled: the arrival counters
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    rc = load().nyion_attention_sparse_q4(
        ptr(q), ptr(k_pool), ptr(v_pool), k_pool.numel(), ptr(page_bases), page_bases.shape[1],
        n_layers, layer, ptr(ctx_lens), ptr(q_pos), B, n_heads, n_kv_heads, head_dim, window,
        global_stride, max_ctx, ptr(out), ptr(workspace), ws_bytes, stream_handle(stream))
    check(rc, "nyion_attention_sparse_q4")
    return workspace


def prepare_attention_sparse_q4(q, k_pool, v_pool, page_bases, n_layers, layer, ctx_lens, out,
                                n_heads, n_kv_heads, head_dim, window, global_stride, max_ctx,
                                q_pos=None, workspace=None, stream=None):
    """attention_sparse_q4 with every argument resolved once: a no-argument
    callable that only crosses the C ABI."""
    B = q.shape[0]
    need = load().nyion_attention_sparse_q4_workspace_size(B, n_heads, n_kv_heads, head_dim, window,
                                                           max_ctx)
    if workspace is None and need:
        workspace = alloc_workspace(need, q.device)  # zero-filled: the arrival counters
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    fn = load().nyion_attention_sparse_q4
    args = (ptr(q), ptr(k_pool), ptr(v_pool), k_pool.numel(), ptr(page_bases),
            page_bases.shape[1], n_layers, layer, ptr(ctx_lens), ptr(q_pos), B, n_heads,
            n_kv_heads, head_dim, window, global_stride, max_ctx, ptr(out), ptr(workspace),
            ws_bytes, stream_handle(stream))
    keep = (q, k_pool, v_pool, page_bases, ctx_lens, out, q_pos, workspace)

    def call():
        rc = fn(*args)
        if rc != 0:
            check(rc, "nyion_attention_sparse_q4")

    call.keep = keep
    return call


def sparse_attention_q4(q, k_q4, v_q4, positions, n_heads, head_dim, window=0, global_stride=0):
    """The Mojo FFI symbol on host numpy arrays (f32 q, f32-word K/V rows,
    int32 positions); returns out [n_heads][head_dim] f32."""
    import numpy as np
    q = np.ascontiguousarray(q, dtype=np.float32)
    k_q4 = np.ascontiguousarray(k_q4, dtype=np.float32)
    v_q4 = np.ascontiguousarray(v_q4, dtype=np.float32)
    pos = np.ascontiguousarray(positions, dtype=np.int32)
    out = np.full((n_heads, head_dim), np.nan, np.float32)
    load().sparse_attention_q4(q.ctypes.data, k_q4.ctypes.data, v_q4.ctypes.data, pos.ctypes.data,
                               out.ctypes.data, n_heads, head_dim, len(pos), window, global_stride)
    if out.size and np.isnan(out).all() and last_error():  # the symbol returns nothing
        raise NyionError(ERR_INVALID, f"sparse_attention_q4: {last_error()}")
    return out


def q4_dequant(inp, n_rows, head_dim, out, stream=None):
    check(load().nyion_q4_dequant(ptr(inp), n_rows, head_dim, ptr(out), stream_handle(stream)),
          "nyion_q4_dequant")


def q4_quantize(inp, n_rows, head_dim, out, stream=None):
    check(load().nyion_q4_quantize(ptr(inp), n_rows, head_dim, ptr(out), stream_handle(stream)),
          "nyion_q4_quantize")


# ----------------------------------------------------------------------------
# swamp-kernels C-ABI
# ----------------------------------------------------------------------------

def softmax_padic_dev(logits, probs, temperature=1.0, stream=None):
    check(load().nyion_softmax_padic_dev(ptr(logits), ptr(probs), logits.numel(),
                                         float(temperature), stream_handle(stream)),
          "nyion_softmax_padic_dev")


def kv_gather_bf16(pool, block_table, block_tokens, n_kv_heads, head_dim, kv_dtype, n_tokens,
                   out, stream=None):
    """Tokens [0, n_tokens) of a paged pool as [n_tokens][Hkv][D] bf16 in `out`."""
    rc = load().nyion_kv_gather_bf16(ptr(pool), ptr(block_table), block_tokens, pool.shape[0],
                                     n_kv_heads, head_dim, kv_dtype, n_tokens, ptr(out),
                                     stream_handle(stream))
    check(rc, "nyion_kv_gather_bf16")


# ----------------------------------------------------------------------------
# Q4_K weight GEMV
# ----------------------------------------------------------------------------

Q4K_BLOCK = 256
Q4K_BYTES = 144


def gemv_q4k(w, x, out, n_rows, n_cols, stream=None):
    """w: device uint8 [n_rows][n_cols/256*144]; x [n_cols] f32; out [n_rows] f32."""
    check(load().nyion_gemv_q4k(ptr(w), ptr(x), ptr(out), n_rows, n_cols, stream_handle(stream)),
          "nyion_gemv_q4k")


def gemv_q4k_multi(ws, x, outs, n_cols, stream=None):
    """Several Q4_K matrices sharing x: ws, outs lists of device tensors."""
    n = len(ws)
    wa = (C.c_void_p * n)(*[w.data_ptr() for w in ws])
    oa = (C.c_void_p * n)(*[o.data_ptr() for o in outs])
    rows = (C.c_int32 * n)(*[int(o.shape[-1]) for o in outs])
    check(load().nyion_gemv_q4k_multi(wa, ptr(x), oa, rows, n, n_cols, stream_handle(stream)),
          "nyion_gemv_q4k_multi")


def gemv_q4k_batched(w, x, out, n_rows, n_cols, stream=None):
    """x [batch][>= n_cols] f32, out [batch][>= n_rows] f32 (row-major, strided)."""
    check(load().nyion_gemv_q4k_batched(ptr(w), ptr(x), x.stride(0), ptr(out), out.stride(0),
                                        n_rows, n_cols, x.shape[0], stream_handle(stream)),
          "nyion_gemv_q4k_batched")


# ----------------------------------------------------------------------------
# Q6_K weight GEMV and mixed Q4_K / Q6_K lists
# ----------------------------------------------------------------------------

Q6K_BYTES = 210


def gemv_q6k(w, x, out, n_rows, n_cols, stream=None):
    """w: device uint8 [n_rows][n_cols/256*210] (2-byte aligned); x [n_cols] f32; out [n_rows] f32."""
    check(load().nyion_gemv_q6k(ptr(w), ptr(x), ptr(out), n_rows, n_cols, stream_handle(stream)),
          "nyion_gemv_q6k")


def gemv_q6k_batched(w, x, out, n_rows, n_cols, stream=None):
    """x [batch][>= n_cols] f32, out [batch][>= n_rows] f32 (row-major, strided)."""
    check(load().nyion_gemv_q6k_batched(ptr(w), ptr(x), x.stride(0), ptr(out), out.stride(0),
                                        n_rows, n_cols, x.shape[0], stream_handle(stream)),
          "nyion_gemv_q6k_batched")


class GemvSpec(C.Structure):
    """nyion_gemv_spec: (w, x, out, n_rows, n_cols, block_bytes 144 | 210)."""
    _fields_ = [("w", C.c_void_p), ("x", C.c_void_p), ("out", C.c_void_p), ("n_rows", C.c_int32),
                ("n_cols", C.c_int32), ("block_bytes", C.c_int32), ("reserved", C.c_int32)]


def gemv_specs(specs, stream=None):
    """specs: list of (w, x, out, n_rows, n_cols, block_bytes) with device tensors."""
    n = len(specs)
    arr = (GemvSpec * max(n, 1))()
    for i, (w, x, out, nr, nc, bb) in enumerate(specs):
        arr[i] = GemvSpec(ptr(w), ptr(x), ptr(out), nr, nc, bb, 0)
    check(load().nyion_gemv_specs(arr, n, stream_handle(stream)), "nyion_gemv_specs")


# ----------------------------------------------------------------------------
# paged KV pool with host spill
# ----------------------------------------------------------------------------

PAGE_CREATE, PAGE_EVICT, PAGE_RELOAD = 0, 1, 2
PAGE_UNMAPPED, PAGE_HOT, PAGE_COLD = 0, 1, 2


class PageEvent(C.Structure):
    _fields_ = [("kind", C.c_int32), ("page", C.c_int32), ("block", C.c_int32),
                ("slot", C.c_int32)]


def _policy_state(h, page):
    where, imp = C.c_int(0), C.c_double(0.0)
    st = load().nyion_page_policy_state(h, page, C.byref(where), C.byref(imp))
    return st, where.value, imp.value


def _policy_lru(h, cap):
    buf = (C.c_int * max(cap, 1))()
    n = load().nyion_page_policy_lru(h, buf, cap)
    return list(buf[:max(n, 0)])


class PagePolicy:
    """Host page policy (no device needed)."""

    def __init__(self, hot_limit, cold_slots, max_pages):
        self.h = load().nyion_page_policy_create(hot_limit, cold_slots, max_pages)
        if not self.h:
            raise NyionError(ERR_INVALID, last_error())
        self.max_pages = max_pages

    def ensure(self, first, last=None):
        last = first if last is None else last
        # creating pages up to `last` can evict once per page; reloads in range
        cap = 2 * (last + 1) + 4 * (last - first + 1) + 16
        buf = (PageEvent * cap)()
        n = C.c_int(0)
        rc = load().nyion_page_policy_ensure(self.h, first, last, buf, cap, C.byref(n))
        events = [(e.kind, e.page, e.block, e.slot) for e in buf[:min(n.value, cap)]]
        return rc, events

    def record(self, page, weight):
        check(load().nyion_page_policy_record(self.h, page, weight), "page_policy_record")

    def reset(self):
        check(load().nyion_page_policy_reset(self.h), "page_policy_reset")

    def state(self, page):
        return _policy_state(self.h, page)

    def lru(self):
        return _policy_lru(self.h, self.max_pages)

    def close(self):
        if getattr(self, "h", None):
            load().nyion_page_policy_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter shutdown: the library may be gone
            pass


class KvPool:
    """Device-resident paged KV cache of one sequence with a pinned-host cold tier."""

    def __init__(self, n_layers, n_kv_heads, head_dim, block_tokens, kv_dtype, hot_blocks,
                 cold_slots, max_pages):
        self.h = load().nyion_kv_pool_create(n_layers, n_kv_heads, head_dim, block_tokens,
                                             kv_dtype, hot_blocks, cold_slots, max_pages)
        if not self.h:
            raise NyionError(ERR_INVALID, last_error())
        self.n_layers, self.n_kv_heads, self.head_dim = n_layers, n_kv_heads, head_dim
        self.block_tokens, self.kv_dtype = block_tokens, kv_dtype
        self.hot_blocks, self.cold_slots, self.max_pages = hot_blocks, cold_slots, max_pages

    def layer(self, layer):
        k, v = C.c_void_p(), C.c_void_p()
        check(load().nyion_kv_pool_layer(self.h, layer, C.byref(k), C.byref(v)), "kv_pool_layer")
        return k.value, v.value

    def table(self):
        return load().nyion_kv_pool_table(self.h)

    def ensure(self, first, last=None, stream=None):
        last = first if last is None else last
        check(load().nyion_kv_pool_ensure(self.h, first, last, stream_handle(stream)),
              "kv_pool_ensure")

    def record_importance(self, importance, threshold=0.001):
        import numpy as np
        imp = np.ascontiguousarray(importance, dtype=np.float64)
        check(load().nyion_kv_pool_record_importance(self.h, imp.ctypes.data, imp.size, threshold),
              "kv_pool_record_importance")

    def stats(self):
        v = [C.c_int64(0) for _ in range(4)]
        check(load().nyion_kv_pool_stats(self.h, *[C.byref(x) for x in v]), "kv_pool_stats")
        return dict(zip(("hot", "cold", "evictions", "reloads"), [x.value for x in v]))

    def state(self, page):
        return _policy_state(load().nyion_kv_pool_policy(self.h), page)

    def lru(self):
        return _policy_lru(load().nyion_kv_pool_policy(self.h), self.max_pages)

    def cold_slot_ptr(self, slot):
        return load().nyion_kv_pool_cold_slot(self.h, slot)

    def close(self):
        if getattr(self, "h", None):
            load().nyion_kv_pool_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter shutdown: the library may be gone
            pass


# ----------------------------------------------------------------------------
# HMA arena
# ----------------------------------------------------------------------------

class Hma:
    """The HeterogeneousMemoryAllocator arena (nyion_hma_*).  alloc returns an
    Allocation; upload/download take bytes-like host data."""

    def __init__(self, device_bytes: int, host_bytes: int):
        self.h = load().nyion_hma_create(device_bytes, host_bytes)
        if not self.h:
            raise NyionError(ERR_OOM, f"nyion_hma_create: {last_error()}")

    @property
    def has_device(self) -> bool:
        return bool(load().nyion_hma_has_device(self.h))

    def alloc(self, size: int, location: int) -> Allocation:
        a = Allocation()
        check(load().nyion_hma_alloc(self.h, size, location, C.byref(a)), "nyion_hma_alloc")
        return a

    def try_alloc(self, size: int, location: int):
        """(rc, Allocation) without raising."""
        a = Allocation()
        return load().nyion_hma_alloc(self.h, size, location, C.byref(a)), a

    def free(self, a: Allocation) -> int:
        return load().nyion_hma_free(self.h, C.byref(a))

    def upload(self, a: Allocation, data: bytes) -> int:
        buf = C.create_string_buffer(bytes(data), len(data))
        return load().nyion_hma_upload(self.h, C.byref(a), buf, len(data))

    def download(self, a: Allocation, nbytes: int):
        """(rc, bytes)"""
        buf = C.create_string_buffer(nbytes)
        rc = load().nyion_hma_download(self.h, buf, C.byref(a), nbytes)
        return rc, buf.raw

    def reset(self) -> int:
        return load().nyion_hma_reset(self.h)

    def stats(self, location: int):
        used, cap = C.c_size_t(), C.c_size_t()
        check(load().nyion_hma_stats(self.h, location, C.byref(used), C.byref(cap)),
              "nyion_hma_stats")
        return used.value, cap.value

    def close(self):
        if self.h:
            load().nyion_hma_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
