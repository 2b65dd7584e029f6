"""Seeded random sweep of paged decode against the oracle (gpu).

Each case draws a configuration the fixed-shape tests leave out: KV format
(f32, binary16, Q4-20B), head_dim 64 or 128, kv heads and GQA group (up to
32 q heads per kv head), page size 4..64 tokens (the per-row gather path
below 16), batch 1..6 with context lengths 1..3000, and full, sliding-window
or window-plus-strided-globals position sets (ops::attention and
ops::attention_sparse, swamp-engine/src/ops.rs:170-278, 85-168), with and
without explicit q positions.  Tolerance as for every attention output:
max-abs-err <= 2e-3 and max|diff| / max|ref| <= 1e-3."""
import numpy as np
import pytest
import torch

import oracle
import workloads as W

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-3
N_CASES = 64


def to_dev(x):
    x = np.ascontiguousarray(x)
    if x.dtype == np.uint16:
        return torch.from_numpy(x.view(np.int16)).cuda()
    return torch.from_numpy(x).cuda()


def draw(seed):
    rng = np.random.default_rng(1000 + seed)
    kv = [oracle.KV_F32, oracle.KV_F16, oracle.KV_Q4][seed % 3]
    hd = int(rng.choice([64, 128]))
    hkv = int(rng.choice([1, 2, 4, 8]))
    group = int(rng.choice([1, 2, 4, 8, 16, 32]))
    while hkv * group > 64:
        group //= 2
    bt = int(rng.choice([4, 8, 16, 32, 64]))
    batch = int(rng.integers(1, 7))
    ctx = [int(x) for x in rng.integers(1, 3001, size=batch)]
    mode = ["full", "window", "globals"][int(rng.integers(0, 3))]
    window = int(rng.choice([16, 100, 512, 1024])) if mode != "full" else 0
    stride = int(rng.choice([16, 64])) if mode == "globals" else 0
    q_pos = [int(rng.integers(0, c)) for c in ctx] if rng.random() < 0.4 else None
    return dict(kv=kv, hd=hd, hkv=hkv, hq=hkv * group, bt=bt, ctx=ctx, window=window,
                stride=stride, q_pos=q_pos)


@pytest.mark.parametrize("seed", range(N_CASES))
def test_random_decode(gpu, seed):
    c = draw(seed)
    print(f"case {seed}: {c}", flush=True)
    pb = W.paged_batch(c["ctx"], n_heads=c["hq"], n_kv_heads=c["hkv"], head_dim=c["hd"],
                       block_tokens=c["bt"], seed=seed, kv_dtype=c["kv"])
    q = to_dev(pb.q)
    kp, vp = to_dev(pb.k_pool), to_dev(pb.v_pool)
    tab, ctx = to_dev(pb.tables), to_dev(pb.ctx_lens)
    qp = None if c["q_pos"] is None else to_dev(np.asarray(c["q_pos"], np.int32))
    out = torch.full_like(q, float("nan"))
    gpu.paged_decode(q, kp, vp, tab, ctx, out, pb.n_heads, pb.n_kv_heads, pb.head_dim,
                     pb.block_tokens, kv_dtype=pb.kv_dtype, window=c["window"],
                     global_stride=c["stride"], max_ctx=int(pb.ctx_lens.max()), q_pos=qp)
    torch.cuda.synchronize()
    got = out.cpu().numpy().astype(np.float64)
    ref = W.reference_decode(pb, window=c["window"], global_stride=c["stride"], q_pos=c["q_pos"],
                             threads=8).astype(np.float64)
    assert np.all(np.isfinite(got)), c
    err = np.max(np.abs(got - ref))
    rel = err / max(np.max(np.abs(ref)), 1e-30)
    assert err <= ATOL and rel <= RTOL, f"{c}: max-abs {err:.3e} rel {rel:.3e}"


@pytest.mark.parametrize("seed", range(16))
def test_random_tracked_pipelined(gpu, seed):
    """Random configurations (the draws above) through two layers of the
    pipelined tracked decode (layer 1's launch also sums layer 0's
    importance; layer 1's own sum is the standalone call): outputs,
    importance and scores equal two tracked calls bit for bit."""
    c = draw(500 + seed)
    print(f"case {seed}: {c}", flush=True)
    pbs = [W.paged_batch(c["ctx"], n_heads=c["hq"], n_kv_heads=c["hkv"], head_dim=c["hd"],
                         block_tokens=c["bt"], seed=600 + 2 * seed + i, kv_dtype=c["kv"])
           for i in range(2)]
    ctx = to_dev(pbs[0].ctx_lens)
    qp = None if c["q_pos"] is None else to_dev(np.asarray(c["q_pos"], np.int32))
    max_ctx = int(pbs[0].ctx_lens.max())
    B, H = pbs[0].batch, pbs[0].n_heads
    kw = dict(kv_dtype=c["kv"], window=c["window"], global_stride=c["stride"], max_ctx=max_ctx,
              q_pos=qp)
    dev = [(to_dev(pb.q), to_dev(pb.k_pool), to_dev(pb.v_pool), to_dev(pb.tables)) for pb in pbs]
    init = np.random.default_rng(700 + seed).random((2, B, max_ctx + 1))
    ref = []
    for i, (q, kp, vp, tab) in enumerate(dev):
        out = torch.full_like(q, float("nan"))
        imp = torch.from_numpy(init[i].copy()).cuda()
        sc = torch.full((B, H, max_ctx + 2), float("nan"), device="cuda")
        gpu.paged_decode_tracked(q, kp, vp, tab, ctx, out, imp, H, c["hkv"], c["hd"], c["bt"],
                                 scores=sc, **kw)
        ref.append([x.cpu().numpy() for x in (out, imp, sc)])
    outs = [torch.full_like(d[0], float("nan")) for d in dev]
    imps = [torch.from_numpy(init[i].copy()).cuda() for i in range(2)]
    scs = [torch.full((B, H, max_ctx + 2), float("nan"), device="cuda") for _ in range(2)]
    for i, (q, kp, vp, tab) in enumerate(dev):
        gpu.paged_decode_tracked_pipelined(q, kp, vp, tab, ctx, outs[i], scs[i],
                                           scs[0] if i else None, imps[0] if i else None, H,
                                           c["hkv"], c["hd"], c["bt"], **kw)
    gpu.paged_decode_importance(ctx, scs[1], imps[1], H, window=c["window"],
                                global_stride=c["stride"], max_ctx=max_ctx, q_pos=qp)
    torch.cuda.synchronize()
    for i in range(2):
        assert np.array_equal(outs[i].cpu().numpy(), ref[i][0]), f"{c}: layer {i} output"
        assert np.array_equal(imps[i].cpu().numpy(), ref[i][1]), f"{c}: layer {i} importance"
        assert np.array_equal(scs[i].cpu().numpy(), ref[i][2], equal_nan=True), f"{c}: layer {i} scores"
    # and the tracked calls' importance against the oracle, per position
    for i, pb in enumerate(pbs):
        for b in range(B):
            L = int(pb.ctx_lens[b])
            qpb = L - 1 if c["q_pos"] is None else c["q_pos"][b]
            got = ref[i][1][b] - init[i][b]
            if c["window"] > 0:
                want = W.window_importance(pb, b, qpb, c["window"], c["stride"], got.shape[0])
            else:
                _, imp = oracle.attention(pb.q[b].reshape(-1), pb.layout(b), L, qpb, H, c["hkv"],
                                          c["hd"], importance=True)
                want = np.zeros(got.shape[0])
                want[:L] = imp
            W.assert_importance(got, want, f"{c}: layer {i} importance b={b}")


@pytest.mark.parametrize("seed", range(32))
def test_random_decode_partitioned(gpu, seed):
    """The draws above on the aligned walks (pages of 16..256 tokens) with
    the tiles per workgroup overridden (64..2048 tokens): where the direct
    partition's piece and wave boundaries fall against the window start,
    the globals and the page edges moves with every case."""
    c = draw(3000 + seed)
    rng = np.random.default_rng(4000 + seed)
    c["bt"] = int(rng.choice([16, 32, 64, 128, 256]))
    tokens = int(rng.choice([64, 128, 256, 512, 1024, 2048]))
    print(f"case {seed}: {c} partition {tokens}", flush=True)
    pb = W.paged_batch(c["ctx"], n_heads=c["hq"], n_kv_heads=c["hkv"], head_dim=c["hd"],
                       block_tokens=c["bt"], seed=seed, kv_dtype=c["kv"])
    q = to_dev(pb.q)
    kp, vp = to_dev(pb.k_pool), to_dev(pb.v_pool)
    tab, ctx = to_dev(pb.tables), to_dev(pb.ctx_lens)
    qp = None if c["q_pos"] is None else to_dev(np.asarray(c["q_pos"], np.int32))
    out = torch.full_like(q, float("nan"))
    try:
        gpu.set_partition_tokens(tokens)
        gpu.paged_decode(q, kp, vp, tab, ctx, out, pb.n_heads, pb.n_kv_heads, pb.head_dim,
                         pb.block_tokens, kv_dtype=pb.kv_dtype, window=c["window"],
                         global_stride=c["stride"], max_ctx=int(pb.ctx_lens.max()), q_pos=qp)
        torch.cuda.synchronize()
    finally:
        gpu.set_partition_tokens(0)
    got = out.cpu().numpy().astype(np.float64)
    ref = W.reference_decode(pb, window=c["window"], global_stride=c["stride"], q_pos=c["q_pos"],
                             threads=8).astype(np.float64)
    assert np.all(np.isfinite(got)), c
    err = np.max(np.abs(got - ref))
    rel = err / max(np.max(np.abs(ref)), 1e-30)
    assert err <= ATOL and rel <= RTOL, f"{c} partition {tokens}: max-abs {err:.3e} rel {rel:.3e}"
