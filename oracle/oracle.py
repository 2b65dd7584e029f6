"""ctypes front-end of the CPU oracle (oracle/nyion_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the reference result.  The product library never
imports it.

The oracle restates the reference's CPU attention (swamp-engine/src/ops.rs),
its Q4-20B codec and zone page arithmetic (swamp-engine/src/cache.rs) and the
swamp-kernels C-ABI (swamp-kernels/src/lib.rs).  Each C function cites the
lines it follows.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libnyion_oracle.so")

KV_F32 = 0
KV_Q4 = 1
KV_F16 = 2
CONTIGUOUS = 1 << 40  # block_tokens larger than any position


class KVLayout(C.Structure):
    _fields_ = [
        ("k_base", C.c_void_p),
        ("v_base", C.c_void_p),
        ("table", C.c_void_p),
        ("block_tokens", C.c_int64),
        ("block_stride", C.c_int64),
        ("head_stride", C.c_int64),
        ("token_stride", C.c_int64),
        ("dtype", C.c_int32),
        ("_pad", C.c_int32),
    ]


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        f32p = C.POINTER(C.c_float)
        i32p = C.POINTER(C.c_int32)
        L.orc_rope_lut.argtypes = [C.c_int, C.c_int, C.c_void_p]
        L.orc_apply_rope.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int,
                                     C.c_int, C.c_void_p]
        L.orc_q4k_unpack_scales.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p]
        L.orc_q4k_dequant_block.argtypes = [C.c_void_p, C.c_void_p]
        L.orc_q6k_scale_to_f32.restype = C.c_float
        L.orc_q6k_scale_to_f32.argtypes = [C.c_uint16]
        L.orc_q6k_dequant_block.argtypes = [C.c_void_p, C.c_void_p]
        L.orc_gemv_q6k.restype = C.c_int
        L.orc_gemv_q6k.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int]
        L.orc_mojo_sparse_attention_q4.restype = None
        L.orc_mojo_sparse_attention_q4.argtypes = [C.c_void_p] * 5 + [C.c_int] * 3
        L.orc_gemv_q4k.restype = C.c_int
        L.orc_gemv_q4k.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int]
        L.orc_dot_avx512_order.restype = C.c_float
        L.orc_dot_avx512_order.argtypes = [C.c_void_p, C.c_void_p, C.c_int]
        L.orc_weighted_sum.argtypes = [C.c_void_p, C.c_void_p, C.c_float, C.c_int]
        L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_f32_to_f16.argtypes = [C.c_float]
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_q4_row_bytes.restype = C.c_int
        L.orc_q4_row_bytes.argtypes = [C.c_int]
        L.orc_q4_quantize_row.argtypes = [C.c_void_p, C.c_int, C.c_void_p]
        L.orc_q4_dequant_row.argtypes = [C.c_void_p, C.c_int, C.c_void_p]
        L.orc_q4_quantize_rows.argtypes = [C.c_void_p, C.c_int64, C.c_int, C.c_void_p]
        L.orc_q4_dequant_rows.argtypes = [C.c_void_p, C.c_int64, C.c_int, C.c_void_p]
        for name in ("orc_zone_index", "orc_zone_block_size", "orc_zone_slot_in_page",
                     "orc_zone_page_start", "orc_zone_total_pages"):
            getattr(L, name).restype = C.c_int64
            getattr(L, name).argtypes = [C.c_int64]
        L.orc_zone_page_id.restype = C.c_int64
        L.orc_zone_page_id.argtypes = [C.c_int64, C.c_int64]
        L.orc_zone_f32_offset.restype = C.c_int64
        L.orc_zone_f32_offset.argtypes = [C.c_int64] * 5
        L.orc_zone_q4_offset.restype = C.c_int64
        L.orc_zone_q4_offset.argtypes = [C.c_int64] * 5
        L.orc_sparse_positions.restype = C.c_int
        L.orc_sparse_positions.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_int]
        L.orc_fugu_positions.restype = C.c_int
        L.orc_fugu_positions.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_int,
                                         C.c_void_p, C.c_int]
        L.orc_attention.restype = C.c_int
        L.orc_attention.argtypes = [C.c_void_p, C.c_void_p, C.POINTER(KVLayout), C.c_int, C.c_int,
                                    C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_int]
        L.orc_attention_positions.restype = C.c_int
        L.orc_attention_positions.argtypes = [C.c_void_p, C.c_void_p, C.POINTER(KVLayout),
                                              C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int,
                                              C.c_void_p, C.c_int]
        L.orc_q4_a5_row.restype = None
        L.orc_q4_a5_row.argtypes = [C.c_void_p, C.c_int, C.c_void_p]
        L.orc_sparse_q4_positions.restype = C.c_int
        L.orc_sparse_q4_positions.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p,
                                              C.c_int]
        L.orc_attention_sparse_q4.restype = C.c_int
        L.orc_attention_sparse_q4.argtypes = [C.c_void_p, C.c_void_p, C.POINTER(KVLayout), C.c_int,
                                              C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                              C.c_int]
        L.orc_attention_rows.restype = C.c_int
        L.orc_attention_rows.argtypes = [C.c_void_p, C.c_void_p, C.c_int64, C.c_int64,
                                         C.POINTER(KVLayout), C.c_void_p, C.c_int, C.c_int,
                                         C.c_int, C.c_int, C.c_int]
        L.orc_exp_q16_16.restype = C.c_int32
        L.orc_exp_q16_16.argtypes = [C.c_int32]
        L.orc_softmax_padic.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_float]
        L.orc_stokes_init.restype = C.c_void_p
        L.orc_stokes_init.argtypes = [C.c_int]
        L.orc_stokes_append.restype = C.c_int
        L.orc_stokes_append.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_float]
        L.orc_stokes_free.argtypes = [C.c_void_p]
        L.orc_stokes_count.restype = C.c_int
        L.orc_stokes_count.argtypes = [C.c_void_p]
        L.orc_stokes_read.restype = C.c_int
        L.orc_stokes_read.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]
        L.orc_max_threads.restype = C.c_int
        _ = (f32p, i32p)
        _lib = L
    return _lib


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


# ----------------------------------------------------------------------------
# layouts
# ----------------------------------------------------------------------------

def paged_layout(k_pool: np.ndarray, v_pool: np.ndarray, table: np.ndarray | None,
                 block_tokens: int, n_kv_heads: int, head_dim: int, dtype: int = KV_F32):
    """Pool [num_blocks][Hkv][block_tokens][row] with row = D f32, D binary16 or Q4 bytes."""
    row = q4_row_bytes(head_dim) if dtype == KV_Q4 else head_dim
    lay = KVLayout(k_pool.ctypes.data, v_pool.ctypes.data,
                   None if table is None else table.ctypes.data, block_tokens,
                   n_kv_heads * block_tokens * row, block_tokens * row, row, dtype, 0)
    lay._keep = (k_pool, v_pool, table)
    return lay


def contiguous_layout(k: np.ndarray, v: np.ndarray, kv_stride: int, head_dim: int,
                      dtype: int = KV_F32):
    """[Hkv][kv_stride][row] (the Attention node / gpu_attention_device layout)."""
    row = q4_row_bytes(head_dim) if dtype == KV_Q4 else head_dim
    lay = KVLayout(k.ctypes.data, v.ctypes.data, None, CONTIGUOUS, 0, kv_stride * row, row,
                   dtype, 0)
    lay._keep = (k, v)
    return lay


def token_major_layout(k: np.ndarray, v: np.ndarray, n_kv_heads: int, head_dim: int):
    """[N][Hkv][D] f32 (the per-token K/V the QKV projection produces)."""
    lay = KVLayout(k.ctypes.data, v.ctypes.data, None, CONTIGUOUS, 0, head_dim,
                   n_kv_heads * head_dim, KV_F32, 0)
    lay._keep = (k, v)
    return lay


# ----------------------------------------------------------------------------
# attention
# ----------------------------------------------------------------------------

def attention(q: np.ndarray, layout: KVLayout, seq_len: int, q_pos: int, n_heads: int,
              n_kv_heads: int, head_dim: int, importance: bool = False, threads: int = 1):
    q = np.ascontiguousarray(q, dtype=np.float32)
    out = np.empty(n_heads * head_dim, dtype=np.float32)
    imp = np.zeros(seq_len, dtype=np.float64) if importance else None
    rc = lib().orc_attention(out.ctypes.data, q.ctypes.data, C.byref(layout), seq_len, q_pos,
                             n_heads, n_kv_heads, head_dim, _ptr(imp), threads)
    if rc != 0:
        raise ValueError(f"orc_attention failed rc={rc}")
    return (out, imp) if importance else out


def attention_positions(q: np.ndarray, layout: KVLayout, positions: np.ndarray, n_heads: int,
                        n_kv_heads: int, head_dim: int, threads: int = 1,
                        importance: bool = False):
    """Softmax over exactly `positions`.  importance=True also returns the f64
    sum over heads of each listed position's probability (same order as
    `positions`)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    pos = np.ascontiguousarray(positions, dtype=np.int32)
    out = np.empty(n_heads * head_dim, dtype=np.float32)
    imp = np.zeros(len(pos), dtype=np.float64) if importance else None
    rc = lib().orc_attention_positions(out.ctypes.data, q.ctypes.data, C.byref(layout),
                                       pos.ctypes.data, len(pos), n_heads, n_kv_heads, head_dim,
                                       _ptr(imp), threads)
    if rc != 0:
        raise ValueError(f"orc_attention_positions failed rc={rc}")
    return (out, imp) if importance else out


def q4_a5_row(row: np.ndarray, head_dim: int) -> np.ndarray:
    """One Q4-20B row decoded as attention_sparse_q4 reads it (ops.rs:640-662)."""
    row = np.ascontiguousarray(row, dtype=np.uint8)
    out = np.empty(head_dim, dtype=np.float32)
    lib().orc_q4_a5_row(row.ctypes.data, head_dim, out.ctypes.data)
    return out


def attention_sparse_q4(q: np.ndarray, layout: KVLayout, seq_len: int, q_pos: int, n_heads: int,
                        n_kv_heads: int, head_dim: int, window: int, global_stride: int,
                        threads: int = 1) -> np.ndarray:
    """ops::attention_sparse_q4 (ops.rs:597-723) over a Q4-20B layout."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    out = np.empty(n_heads * head_dim, dtype=np.float32)
    rc = lib().orc_attention_sparse_q4(out.ctypes.data, q.ctypes.data, C.byref(layout), seq_len,
                                       q_pos, n_heads, n_kv_heads, head_dim, window,
                                       global_stride, threads)
    if rc != 0:
        raise ValueError(f"orc_attention_sparse_q4 failed rc={rc}")
    return out


def attention_rows(q: np.ndarray, layout: KVLayout, rows, n_heads: int, n_kv_heads: int,
                   head_dim: int, threads: int = 1, out: np.ndarray | None = None):
    """q: [N][Hq*D] f32.  Returns out [N][Hq*D] with only `rows` filled."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    n = q.shape[0]
    rows = np.ascontiguousarray(rows, dtype=np.int32)
    if out is None:
        out = np.zeros((n, n_heads * head_dim), dtype=np.float32)
    rc = lib().orc_attention_rows(out.ctypes.data, q.ctypes.data, n_heads * head_dim,
                                  n_heads * head_dim, C.byref(layout), rows.ctypes.data,
                                  len(rows), n_heads, n_kv_heads, head_dim, threads)
    if rc != 0:
        raise ValueError(f"orc_attention_rows failed rc={rc}")
    return out


def sparse_positions(seq_len: int, q_pos: int, window: int, global_stride: int) -> np.ndarray:
    cap = window + 130
    buf = np.empty(cap, dtype=np.int32)
    n = lib().orc_sparse_positions(seq_len, q_pos, window, global_stride, buf.ctypes.data, cap)
    if n < 0:
        raise ValueError(f"orc_sparse_positions rc={n}")
    return buf[:n].copy()


def fugu_positions(seq_len: int, q_pos: int, window: int, sentinel_stride: int,
                   dspark) -> np.ndarray:
    ds = np.ascontiguousarray(dspark, dtype=np.int32)
    cap = window + 130 + len(ds)
    buf = np.empty(cap, dtype=np.int32)
    n = lib().orc_fugu_positions(seq_len, q_pos, window, sentinel_stride, ds.ctypes.data, len(ds),
                                 buf.ctypes.data, cap)
    if n < 0:
        raise ValueError(f"orc_fugu_positions rc={n}")
    return buf[:n].copy()


# ----------------------------------------------------------------------------
# Q4 codec
# ----------------------------------------------------------------------------

def q4_row_bytes(head_dim: int) -> int:
    return ((head_dim + 31) // 32) * 20


def rope_lut(head_dim: int, max_ctx: int) -> np.ndarray:
    """init_rope_lut: [max_ctx][head_dim/2][2] f32 (cos, sin)."""
    out = np.empty((max_ctx, head_dim // 2, 2), dtype=np.float32)
    lib().orc_rope_lut(head_dim, max_ctx, out.ctypes.data)
    return out


def apply_rope(q: np.ndarray, k: np.ndarray, pos: int, max_ctx: int, lut: np.ndarray):
    """apply_rope_ufc on copies of one token's q [Hq][D], k [Hkv][D]."""
    q = np.array(q, dtype=np.float32, copy=True, order="C")
    k = np.array(k, dtype=np.float32, copy=True, order="C")
    lut = np.ascontiguousarray(lut, dtype=np.float32)
    lib().orc_apply_rope(q.ctypes.data, k.ctypes.data, pos, q.shape[0], k.shape[0], q.shape[1],
                         max_ctx, lut.ctypes.data)
    return q, k


def q4_quantize_rows(x: np.ndarray) -> np.ndarray:
    """x [..., D] f32 -> [..., row_bytes] u8 (one Q4-20B row per leading index)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    d = x.shape[-1]
    rb = q4_row_bytes(d)
    flat = x.reshape(-1, d)
    out = np.zeros((flat.shape[0], rb), dtype=np.uint8)
    lib().orc_q4_quantize_rows(flat.ctypes.data, flat.shape[0], d, out.ctypes.data)
    return out.reshape(x.shape[:-1] + (rb,))


def q4_dequant_rows(b: np.ndarray, head_dim: int) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint8)
    rb = q4_row_bytes(head_dim)
    flat = b.reshape(-1, rb)
    out = np.empty((flat.shape[0], head_dim), dtype=np.float32)
    lib().orc_q4_dequant_rows(flat.ctypes.data, flat.shape[0], head_dim, out.ctypes.data)
    return out.reshape(b.shape[:-1] + (head_dim,))


def f32_to_f16_bits(x: float) -> int:
    return int(lib().orc_f32_to_f16(float(x)))


def f16_bits_to_f32(h: int) -> float:
    return float(lib().orc_f16_to_f32(int(h)))


# ----------------------------------------------------------------------------
# swamp-kernels C-ABI
# ----------------------------------------------------------------------------

def softmax_padic(logits, temperature: float = 1.0) -> np.ndarray:
    x = np.ascontiguousarray(logits, dtype=np.float32)
    out = np.zeros_like(x)
    lib().orc_softmax_padic(x.ctypes.data, out.ctypes.data, len(x), float(temperature))
    return out


def exp_q16_16(x: int) -> int:
    return int(lib().orc_exp_q16_16(int(x)))


def max_threads() -> int:
    return int(lib().orc_max_threads())


# ----------------------------------------------------------------------------
# Q4_K weights (swamp-kernels/src/fused_gemv_q4k.rs)
# ----------------------------------------------------------------------------

Q4K_BLOCK = 256
Q4K_BYTES = 144


def q4k_unpack_scales(sc: np.ndarray):
    sc = np.ascontiguousarray(sc, dtype=np.uint8)
    scales = np.zeros(8, np.uint8)
    mins = np.zeros(8, np.uint8)
    lib().orc_q4k_unpack_scales(sc.ctypes.data, scales.ctypes.data, mins.ctypes.data)
    return scales, mins


def q4k_dequant(w: np.ndarray, n_rows: int, n_cols: int) -> np.ndarray:
    """Q4_K bytes [n_rows][n_cols/256 * 144] -> f32 [n_rows][n_cols]."""
    w = np.ascontiguousarray(w, dtype=np.uint8).reshape(-1, Q4K_BYTES)
    out = np.empty((w.shape[0], Q4K_BLOCK), np.float32)
    for i in range(w.shape[0]):
        lib().orc_q4k_dequant_block(w[i].ctypes.data, out[i].ctypes.data)
    return out.reshape(n_rows, n_cols)


def gemv_q4k(w: np.ndarray, x: np.ndarray, n_rows: int, n_cols: int) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert w.size == n_rows * (n_cols // Q4K_BLOCK) * Q4K_BYTES and x.size >= n_cols
    out = np.empty(n_rows, np.float32)
    if lib().orc_gemv_q4k(w.ctypes.data, x.ctypes.data, out.ctypes.data, n_rows, n_cols) != 0:
        raise ValueError("orc_gemv_q4k: n_cols must be a positive multiple of 256")
    return out


# ----------------------------------------------------------------------------
# Q6_K weights (swamp-kernels/src/fused_gemv_q6k.rs)
# ----------------------------------------------------------------------------

Q6K_BYTES = 210


def q6k_scale_to_f32(bits: int) -> float:
    return float(lib().orc_q6k_scale_to_f32(int(bits)))


def q6k_dequant(w: np.ndarray, n_rows: int, n_cols: int) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8).reshape(-1, Q6K_BYTES)
    out = np.empty((w.shape[0], Q4K_BLOCK), np.float32)
    for i in range(w.shape[0]):
        lib().orc_q6k_dequant_block(w[i].ctypes.data, out[i].ctypes.data)
    return out.reshape(n_rows, n_cols)


def gemv_q6k(w: np.ndarray, x: np.ndarray, n_rows: int, n_cols: int) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert w.size == n_rows * (n_cols // Q4K_BLOCK) * Q6K_BYTES and x.size >= n_cols
    out = np.empty(n_rows, np.float32)
    if lib().orc_gemv_q6k(w.ctypes.data, x.ctypes.data, out.ctypes.data, n_rows, n_cols) != 0:
        raise ValueError("orc_gemv_q6k: n_cols must be a positive multiple of 256")
    return out


def mojo_q4_rows(x: np.ndarray) -> np.ndarray:
    """f32 rows [n][head_dim] -> the Mojo kernel's row format [n][blocks*20]
    f32 words (attention.mojo:8-33): per 32-element block word 0 d, word 1
    dmin, words 2.. the 16 nibble bytes as float values, quantised with the
    Q4-20B rules (cache.rs:637-663; d and dmin as the f16 values stored)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n, hd = x.shape
    b = q4_quantize_rows(x)
    blocks = (hd + 31) // 32
    g = b.reshape(n, blocks, 20)
    d = g[:, :, 0:2].copy().view(np.float16).astype(np.float32)[:, :, 0]
    dmin = g[:, :, 2:4].copy().view(np.float16).astype(np.float32)[:, :, 0]
    out = np.zeros((n, blocks, 20), np.float32)
    out[:, :, 0] = d
    out[:, :, 1] = dmin
    out[:, :, 2:18] = g[:, :, 4:20].astype(np.float32)
    return out.reshape(n, blocks * 20)


def mojo_sparse_attention_q4(q: np.ndarray, k_q4: np.ndarray, v_q4: np.ndarray,
                             positions: np.ndarray, n_heads: int, head_dim: int) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.float32)
    k_q4 = np.ascontiguousarray(k_q4, dtype=np.float32)
    v_q4 = np.ascontiguousarray(v_q4, dtype=np.float32)
    pos = np.ascontiguousarray(positions, dtype=np.int32)
    out = np.zeros(n_heads * head_dim, np.float32)
    lib().orc_mojo_sparse_attention_q4(q.ctypes.data, k_q4.ctypes.data, v_q4.ctypes.data,
                                       pos.ctypes.data, out.ctypes.data, n_heads, head_dim, len(pos))
    return out.reshape(n_heads, head_dim)
