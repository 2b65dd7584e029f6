"""Binary16 KV caches on the GPU (gpu): paged decode (block walk and, for
pages under 16 tokens, per-row gather), tracked decode with importance,
position lists, window decode, the attention node and the project ABI's f16 names (gpu_attention_streamed_half,
gpu_graph_create_attention_half, fused_attention.cu:534-545, 672-717)
against the oracle on the same binary16 rows; the KV writer's rounding, the
gathers' widening and the RoPE epilogue bit-exactly.

Attention tolerance: max-abs-err <= 2e-3 and rel-err (max|diff| / max|ref|)
<= 1e-3, the same as for f32 caches.  The kernel multiplies the binary16
rows as stored, with q split into binary16 high and low parts (scores at f32
accuracy) and the softmax weights rounded to binary16 (relative error <=
2^-12 each), so besides the summation order only that rounding separates it
from the oracle."""
import numpy as np
import pytest
import torch

import oracle
import workloads as W

pytestmark = pytest.mark.gpu

F16 = 2  # NYION_KV_F16
ATOL, RTOL = 2e-3, 1e-3


def to_dev(x):
    x = np.ascontiguousarray(x)
    if x.dtype == np.uint16:
        return torch.from_numpy(x.view(np.int16)).cuda()
    return torch.from_numpy(x).cuda()


def assert_close(got, ref, what):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert np.all(np.isfinite(got)), what
    err = np.max(np.abs(got - ref))
    rel = err / max(np.max(np.abs(ref)), 1e-30)
    assert err <= ATOL and rel <= RTOL, f"{what}: max-abs {err:.3e} rel {rel:.3e}"


def run_paged(gpu, pb, **kw):
    q, kp, vp = to_dev(pb.q), to_dev(pb.k_pool), to_dev(pb.v_pool)
    tab, ctx = to_dev(pb.tables), to_dev(pb.ctx_lens)
    out = torch.full_like(q, float("nan"))
    gpu.paged_decode(q, kp, vp, tab, ctx, out, pb.n_heads, pb.n_kv_heads, pb.head_dim,
                     pb.block_tokens, kv_dtype=F16, max_ctx=int(pb.ctx_lens.max()), **kw)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("ctx,hq,hkv,hd,bt", [
    ([1, 17, 300, 4096], 32, 4, 64, 16),
    ([5000, 33], 32, 8, 128, 16),
    ([129, 1024, 2], 16, 16, 64, 32),
    ([777], 8, 1, 128, 64)])
def test_paged_decode_f16(gpu, ctx, hq, hkv, hd, bt):
    pb = W.paged_batch(ctx, n_heads=hq, n_kv_heads=hkv, head_dim=hd, block_tokens=bt, seed=len(ctx),
                       kv_dtype=oracle.KV_F16)
    assert_close(run_paged(gpu, pb), W.reference_decode(pb, threads=8), f"f16 decode {ctx}")


@pytest.mark.parametrize("bt", [4, 8])
def test_paged_decode_f16_small_pages(gpu, bt):
    """Pages under 16 tokens take the per-row gather path."""
    pb = W.paged_batch([1, 17, 300, 777], block_tokens=bt, seed=bt, kv_dtype=oracle.KV_F16)
    assert_close(run_paged(gpu, pb), W.reference_decode(pb), f"f16 block_tokens {bt}")


def test_tracked_f16(gpu):
    """ops::attention_tracked on binary16 rows: outputs and importance[t] =
    sum_h p_h[t] against the oracle on the same rows."""
    pb = W.paged_batch([300, 4096, 2000], seed=21, kv_dtype=oracle.KV_F16)
    q_pos = [250, 4095, 1500]
    q, kp, vp = to_dev(pb.q), to_dev(pb.k_pool), to_dev(pb.v_pool)
    tab, ctx = to_dev(pb.tables), to_dev(pb.ctx_lens)
    out = torch.full_like(q, float("nan"))
    imp = torch.zeros((pb.batch, 4096 + 2), dtype=torch.float64, device="cuda")
    gpu.paged_decode_tracked(q, kp, vp, tab, ctx, out, imp, pb.n_heads, pb.n_kv_heads, pb.head_dim,
                             pb.block_tokens, kv_dtype=F16,
                             q_pos=to_dev(np.asarray(q_pos, np.int32)))
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), W.reference_decode(pb, q_pos=q_pos), "f16 tracked out")
    got = imp.cpu().numpy()
    for b in range(pb.batch):
        L = int(pb.ctx_lens[b])
        _, ref_imp = oracle.attention(pb.q[b].reshape(-1), pb.layout(b), L, q_pos[b], pb.n_heads,
                                      pb.n_kv_heads, pb.head_dim, importance=True)
        W.assert_importance(got[b, :L], ref_imp, f"f16 importance b={b}")
        assert np.all(got[b, q_pos[b] + 1:] == 0.0), f"f16 importance past valid_end b={b}"


def test_positions_f16(gpu):
    """Explicit position lists (the Fugu set) over binary16 rows."""
    pb = W.paged_batch([6000, 2500], seed=23, kv_dtype=oracle.KV_F16)
    sets = [oracle.fugu_positions(6000, 5999, 256, 64, [5, 77, 5990, 3000, 4]),
            oracle.fugu_positions(2500, 2499, 1024, 0, [17, 18, 2499])]
    pos = np.zeros((2, max(len(x) for x in sets)), np.int32)
    npos = np.array([len(x) for x in sets], np.int32)
    for b, x in enumerate(sets):
        pos[b, :len(x)] = x
    out = torch.full((2, 32, 64), float("nan"), device="cuda")
    gpu.paged_decode_positions(to_dev(pb.q), to_dev(pb.k_pool), to_dev(pb.v_pool), to_dev(pb.tables),
                               to_dev(pos), to_dev(npos), out, 32, 4, 64, 16, kv_dtype=F16)
    torch.cuda.synchronize()
    ref = np.stack([oracle.attention_positions(pb.q[b], pb.layout(b), sets[b], 32, 4, 64).reshape(
        32, 64) for b in range(2)])
    assert_close(out.cpu().numpy(), ref, "f16 positions")


@pytest.mark.parametrize("stride", [0, 64])
def test_window_decode_f16(gpu, stride):
    pb = W.paged_batch([9000, 4200], seed=7, kv_dtype=oracle.KV_F16)
    got = run_paged(gpu, pb, window=1024, global_stride=stride)
    ref = W.reference_decode(pb, window=1024, global_stride=stride, threads=8)
    assert_close(got, ref, f"f16 window stride {stride}")


def test_node_and_project_half_names(gpu):
    rng = np.random.default_rng(12)
    S, stride = 2000, 2048
    q = rng.standard_normal((32, 64), dtype=np.float32)
    k = rng.standard_normal((4, stride, 64), dtype=np.float32).astype(np.float16)
    v = rng.standard_normal((4, stride, 64), dtype=np.float32).astype(np.float16)
    kb, vb = k.view(np.uint16), v.view(np.uint16)
    ref = oracle.attention(q.reshape(-1), oracle.contiguous_layout(kb, vb, stride, 64, oracle.KV_F16),
                           S, S - 1, 32, 4, 64).reshape(32, 64)
    dq, dk, dv = to_dev(q), to_dev(kb), to_dev(vb)
    out = torch.full_like(dq, float("nan"))
    gpu.attention_node(dq, dk, dv, out, 32, 4, S, 64, stride, kv_dtype=F16)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), ref, "f16 node")
    L = gpu.load()
    out2 = torch.full_like(dq, float("nan"))
    assert L.gpu_attention_streamed_half(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), out2.data_ptr(),
                                         32, 4, S, 64, stride, None) == 0
    torch.cuda.synchronize()
    scores = torch.empty(32 * stride, device="cuda")
    eager = torch.empty_like(dq)
    gpu.attention_node(dq, dk, dv, eager, 32, 4, S, 64, stride, kv_dtype=F16, scores=scores)
    torch.cuda.synchronize()
    # the project name runs the node with its stream's split-K buffer
    assert torch.equal(out2, eager)
    assert_close(out2.cpu().numpy(), ref, "gpu_attention_streamed_half")
    out3 = torch.full_like(dq, float("nan"))
    g = L.gpu_graph_create_attention_half(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                                          scores.data_ptr(), out3.data_ptr(), 32, 4, S, 64, stride)
    assert g, gpu.last_error()
    try:
        for rep in range(3):
            out3.fill_(float("nan"))
            torch.cuda.synchronize()
            assert L.gpu_graph_replay_attention(g, torch.cuda.current_stream().cuda_stream) == 0
            torch.cuda.synchronize()
            assert torch.equal(out3, eager), rep
    finally:
        L.gpu_graph_destroy(g)
    assert_close(out3.cpu().numpy(), ref, "f16 graph")


def test_kv_write_f16_rounds_to_nearest_even(gpu):
    """f32 rows -> binary16 bits equal to numpy's conversion, including
    subnormals, signed zero and overflow to infinity."""
    rng = np.random.default_rng(3)
    hkv, hd, bt, n = 4, 64, 16, 300
    k = rng.standard_normal((n, hkv, hd), dtype=np.float32)
    v = (rng.standard_normal((n, hkv, hd)) * 1e-6).astype(np.float32)  # subnormal binary16
    k[0, 0, :8] = [65504.0, 65520.0, 70000.0, -1e9, -0.0, 0.0, 5.96e-8, 2.98e-8]
    k[1, 1, :4] = [1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, 2049.0, 2051.0]  # ties
    nblk = (n + bt - 1) // bt
    table = rng.permutation(nblk + 3)[:nblk].astype(np.int32)
    kp = torch.zeros((nblk + 3, hkv, bt, hd), dtype=torch.int16, device="cuda")
    vp = torch.zeros_like(kp)
    gpu.kv_write(kp, vp, to_dev(table), bt, hkv, hd, F16, 0, to_dev(k), to_dev(v))
    torch.cuda.synchronize()
    kh = kp.cpu().numpy().view(np.uint16)
    vh = vp.cpu().numpy().view(np.uint16)
    t = np.arange(n)
    got_k = kh[table[t // bt], :, t % bt]
    got_v = vh[table[t // bt], :, t % bt]
    assert np.array_equal(got_k, k.astype(np.float16).view(np.uint16))
    assert np.array_equal(got_v, v.astype(np.float16).view(np.uint16))


def test_kv_gather_f16_widens_exactly(gpu):
    pb = W.paged_batch([500], n_kv_heads=4, head_dim=64, seed=5, kv_dtype=oracle.KV_F16)
    n = 500
    kp, tab = to_dev(pb.k_pool), to_dev(pb.tables[0])
    out = torch.empty((4, n, 64), device="cuda")
    gpu.kv_gather(kp, tab, 16, 4, 64, F16, n, out)
    hb = torch.empty((n, 4, 64), dtype=torch.bfloat16, device="cuda")
    gpu.kv_gather_bf16(kp, tab, 16, 4, 64, F16, n, hb)
    torch.cuda.synchronize()
    t = np.arange(n)
    rows = pb.k_pool[pb.tables[0][t // 16], :, t % 16].view(np.float16).astype(np.float32)  # [n][hkv][D]
    assert np.array_equal(out.cpu().numpy(), rows.transpose(1, 0, 2))
    want_bf16 = W.bf16_bits(rows)
    assert np.array_equal(hb.view(torch.int16).cpu().numpy().view(np.uint16), want_bf16)


def test_rope_kv_append_f16(gpu):
    """The rotated k and the v of each sequence, stored as binary16: numpy's
    rounding of the f32 path's bit-exact rows."""
    rng = np.random.default_rng(8)
    B, hq, hkv, hd, bt, max_ctx = 4, 16, 4, 64, 16, 600
    pos = np.array([0, 31, 599, 800], np.int32)
    tables = rng.permutation(B * 64).astype(np.int32).reshape(B, 64)
    q = rng.standard_normal((B, hq, hd), dtype=np.float32)
    k = rng.standard_normal((B, hkv, hd), dtype=np.float32)
    v = rng.standard_normal((B, hkv, hd), dtype=np.float32)
    lut_ref = oracle.rope_lut(hd, max_ctx)
    lut = gpu.rope_lut(hd, max_ctx)
    kp = torch.zeros((B * 64, hkv, bt, hd), dtype=torch.int16, device="cuda")
    vp = torch.zeros_like(kp)
    dq = to_dev(q)
    gpu.rope_kv_append(dq, to_dev(k), to_dev(v), lut, to_dev(pos), kp, vp, to_dev(tables),
                       hq, hkv, hd, bt, F16)
    torch.cuda.synchronize()
    got_q = dq.cpu().numpy()
    kh, vh = kp.cpu().numpy().view(np.uint16), vp.cpu().numpy().view(np.uint16)
    for b in range(B):
        rq, rk = oracle.apply_rope(q[b], k[b], int(pos[b]), max_ctx, lut_ref)
        assert np.array_equal(got_q[b].view(np.uint32), rq.view(np.uint32)), f"q b={b}"
        blk, slot = tables[b, pos[b] // bt], pos[b] % bt
        assert np.array_equal(kh[blk, :, slot], rk.astype(np.float16).view(np.uint16)), f"k b={b}"
        assert np.array_equal(vh[blk, :, slot], v[b].astype(np.float16).view(np.uint16)), f"v b={b}"
