"""Decode attention on the GPU against the oracle (gpu).

Tolerance: max-abs-err <= 2e-3 and rel-err <= 1e-3, where rel-err
is max|gpu - ref| / max|ref| over the compared tensor (fp32 accumulation on
both sides).
"""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle
import workloads as W

pytestmark = pytest.mark.gpu

ATOL = 2e-3
RTOL = 1e-3


def assert_close(got, ref, what=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = np.max(np.abs(got - ref))
    rel = err / max(np.max(np.abs(ref)), 1e-30)
    assert err <= ATOL and rel <= RTOL, f"{what}: max-abs {err:.3e} rel {rel:.3e}"
    return err, rel


def to_dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def run_paged(gpu, pb, window=0, global_stride=0, q_pos=None, max_ctx=None):
    q = to_dev(pb.q)
    kp, vp = to_dev(pb.k_pool), to_dev(pb.v_pool)
    tab, ctx = to_dev(pb.tables), to_dev(pb.ctx_lens)
    qp = None if q_pos is None else to_dev(np.asarray(q_pos, np.int32))
    out = torch.full_like(q, float("nan"))
    gpu.paged_decode(q, kp, vp, tab, ctx, out, pb.n_heads, pb.n_kv_heads, pb.head_dim,
                     pb.block_tokens, kv_dtype=pb.kv_dtype, window=window,
                     global_stride=global_stride, max_ctx=max_ctx, q_pos=qp)
    torch.cuda.synchronize()
    return out.cpu().numpy()


# ---------------------------------------------------------------- node form

def test_attention_node_c1(gpu):
    q, k, v = W.c1_contiguous(seed=0)
    ref = oracle.attention(q.reshape(-1), oracle.contiguous_layout(k, v, 128, 64), 128, 127, 32,
                           4, 64).reshape(32, 64)
    dq, dk, dv = to_dev(q), to_dev(k), to_dev(v)
    out = torch.full_like(dq, float("nan"))
    gpu.attention_node(dq, dk, dv, out, 32, 4, 128, 64, 128)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), ref, "128-position node")
    # with the node's scores buffer as split-K workspace
    scores = torch.empty(32 * 128, dtype=torch.float32, device="cuda")
    out2 = torch.full_like(dq, float("nan"))
    gpu.attention_node(dq, dk, dv, out2, 32, 4, 128, 64, 128, scores=scores)
    torch.cuda.synchronize()
    assert_close(out2.cpu().numpy(), ref, "128-position node + scores")


@pytest.mark.parametrize("with_scores", [False, True])
def test_graph_attention_replays_equal_eager(gpu, with_scores):
    """gpu_graph_create_attention / replay / destroy (fused_attention.cu:595-663):
    every replay equals the eager node bit for bit, with eager work and
    synchronisations between replays; with the scores scratch the split-K
    counters are cleared inside the graph by a kernel, not a memset."""
    rng = np.random.default_rng(31)
    S, stride = 3000, 3072
    q = rng.standard_normal((32, 64), dtype=np.float32)
    k = rng.standard_normal((4, stride, 64), dtype=np.float32)
    v = rng.standard_normal((4, stride, 64), dtype=np.float32)
    dq, dk, dv = to_dev(q), to_dev(k), to_dev(v)
    scores = torch.empty(32 * stride, dtype=torch.float32, device="cuda") if with_scores else None
    eager = torch.empty_like(dq)
    gpu.attention_node(dq, dk, dv, eager, 32, 4, S, 64, stride, scores=scores)
    torch.cuda.synchronize()
    ref = oracle.attention(q.reshape(-1), oracle.contiguous_layout(k, v, stride, 64), S, S - 1, 32,
                           4, 64).reshape(32, 64)
    assert_close(eager.cpu().numpy(), ref, "eager node")
    L = gpu.load()
    out = torch.full_like(dq, float("nan"))
    g = L.gpu_graph_create_attention(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                                     scores.data_ptr() if with_scores else None, out.data_ptr(),
                                     32, 4, S, 64, stride)
    assert g, gpu.last_error()
    try:
        stream = torch.cuda.current_stream().cuda_stream
        for rep in range(4):
            out.fill_(float("nan"))
            other = torch.empty_like(dq)
            gpu.attention_node(dq, dk, dv, other, 32, 4, S // 2, 64, stride, scores=scores)
            torch.cuda.synchronize()
            assert L.gpu_graph_replay_attention(g, stream) == 0, gpu.last_error()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), rep
    finally:
        L.gpu_graph_destroy(g)
    assert L.gpu_graph_replay_attention(None, None) == -1


def test_attention_node_stride_and_project_names(gpu):
    rng = np.random.default_rng(21)
    S, stride = 1000, 1536
    q = rng.standard_normal((32, 64), dtype=np.float32)
    k = rng.standard_normal((4, stride, 64), dtype=np.float32)
    v = rng.standard_normal((4, stride, 64), dtype=np.float32)
    ref = oracle.attention(q.reshape(-1), oracle.contiguous_layout(k, v, stride, 64), S, S - 1,
                           32, 4, 64).reshape(32, 64)
    dq, dk, dv = to_dev(q), to_dev(k), to_dev(v)
    out = torch.full_like(dq, float("nan"))
    L = gpu.load()
    assert L.gpu_attention_device(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), out.data_ptr(), 32,
                                  4, S, 64, stride) == 0
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), ref, "gpu_attention_device")
    out.fill_(float("nan"))
    scores = torch.empty(32 * stride, dtype=torch.float32, device="cuda")
    gpu.attention_node(dq, dk, dv, out, 32, 4, S, 64, stride, scores=scores)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), ref, "node stride")


def test_project_names_streams_and_growth(gpu):
    """gpu_attention_streamed on two streams at once (each stream has its own
    split-K buffer), then a longer context on one of them (its buffer is
    replaced after the stream's queued work), and gpu_attention_device: each
    output equals the node's with a caller scores buffer bit for bit, and
    the oracle at tolerance."""
    L = gpu.load()
    rng = np.random.default_rng(23)
    cases = []
    for S in (3000, 4096, 20000):
        q = rng.standard_normal((32, 64), dtype=np.float32)
        k = rng.standard_normal((4, S, 64), dtype=np.float32)
        v = rng.standard_normal((4, S, 64), dtype=np.float32)
        cases.append((S, q, k, v, to_dev(q), to_dev(k), to_dev(v)))
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs = [torch.full((32, 64), float("nan"), device="cuda") for _ in range(4)]
    torch.cuda.synchronize()
    for i, (st, (S, _, _, _, dq, dk, dv)) in enumerate(((s1, cases[0]), (s2, cases[1]), (s1, cases[2]))):
        for _ in range(3):
            assert L.gpu_attention_streamed(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                                            outs[i].data_ptr(), 32, 4, S, 64, S,
                                            C.c_void_p(st.cuda_stream)) == 0
    S, q, k, v, dq, dk, dv = cases[1]
    assert L.gpu_attention_device(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), outs[3].data_ptr(),
                                  32, 4, S, 64, S) == 0
    torch.cuda.synchronize()
    for i, ci in enumerate((0, 1, 2, 1)):
        S, q, k, v, dq, dk, dv = cases[ci]
        node = torch.full((32, 64), float("nan"), device="cuda")
        scores = torch.empty(32 * S, dtype=torch.float32, device="cuda")
        gpu.attention_node(dq, dk, dv, node, 32, 4, S, 64, S, scores=scores)
        torch.cuda.synchronize()
        assert torch.equal(outs[i], node), f"case {i}"
        ref = oracle.attention(q.reshape(-1), oracle.contiguous_layout(k, v, S, 64), S, S - 1, 32, 4,
                               64).reshape(32, 64)
        assert_close(outs[i].cpu().numpy(), ref, f"project name case {i}")


# ---------------------------------------------------------------- paged full causal

def test_paged_c2_layer(gpu):
    """One TinyLlama decode layer: ctx 4096 in 16-token blocks, shuffled table."""
    pb = W.paged_batch([4096], seed=2)
    assert_close(run_paged(gpu, pb), W.reference_decode(pb), "ctx 4096 layer")


@pytest.mark.parametrize("lens", [[1], [15, 16, 17], [1, 2, 31, 32, 33, 500, 1023, 1024, 1025]])
def test_paged_edge_lengths(gpu, lens):
    pb = W.paged_batch(lens, seed=len(lens))
    assert_close(run_paged(gpu, pb), W.reference_decode(pb), f"lens {lens}")


@pytest.mark.parametrize("bt,kv", [(4, oracle.KV_F32), (8, oracle.KV_F32), (32, oracle.KV_F32),
                                   (64, oracle.KV_F32), (256, oracle.KV_F32), (8, oracle.KV_Q4),
                                   (64, oracle.KV_Q4)])
def test_paged_block_sizes(gpu, bt, kv):
    """Pages of 4 and 8 tokens take the per-row gather path, 16 and up the
    aligned block walk (runs of a tile inside one block)."""
    pb = W.paged_batch([1, 17, 100, 300, 777], block_tokens=bt, seed=bt + kv, kv_dtype=kv)
    assert_close(run_paged(gpu, pb), W.reference_decode(pb), f"block_tokens {bt} kv {kv}")


@pytest.mark.parametrize("bt", [8, 32])
def test_window_small_and_large_blocks(gpu, bt):
    pb = W.paged_batch([70, 300, 1000], block_tokens=bt, seed=bt)
    assert_close(run_paged(gpu, pb, window=64, global_stride=16),
                 W.reference_decode(pb, window=64, global_stride=16), f"window bt {bt}")


def test_paged_batch_beyond_one_launch(gpu):
    """2100 sequences: more than one launch's 2048 (the host splits the batch)."""
    lens = np.random.default_rng(9).integers(1, 48, 2100)
    pb = W.paged_batch(lens, n_heads=8, n_kv_heads=2, seed=9)
    assert_close(run_paged(gpu, pb), W.reference_decode(pb), "2100 sequences")


@pytest.mark.parametrize("ctx,max_ctx,q_pos", [(1000, 4096, None), (4096, 4096, 100), (1, 64, None),
                                              (3000, 3001, 0)])
def test_single_sequence_host_bound(gpu, ctx, max_ctx, q_pos):
    """One sequence: the split follows max_ctx, the actual length masks the
    tail (pieces past it attend to nothing), and q_pos limits the range."""
    pb = W.paged_batch([ctx], seed=ctx, spare_blocks=(max_ctx - ctx + 15) // 16)
    nblk = (max_ctx + 15) // 16
    if pb.tables.shape[1] < nblk:  # table rows for the whole host bound
        extra = np.arange(pb.tables.shape[1], nblk, dtype=np.int32) % pb.k_pool.shape[0]
        pb.tables = np.concatenate([pb.tables, extra[None, :]], axis=1)
    qp = None if q_pos is None else [q_pos]
    for p in (64, 0):
        try:
            gpu.set_partition_tokens(p)
            got = run_paged(gpu, pb, q_pos=qp, max_ctx=max_ctx)
        finally:
            gpu.set_partition_tokens(0)
        assert_close(got, W.reference_decode(pb, q_pos=qp), f"ctx {ctx} max {max_ctx} part {p}")


def test_single_sequence_empty_is_zero(gpu):
    """ctx_len 0 (nothing to attend to) writes zeros, with or without the
    split-K merge."""
    pb = W.paged_batch([64], seed=1)
    q = to_dev(pb.q)
    kp, vp, tab = to_dev(pb.k_pool), to_dev(pb.v_pool), to_dev(pb.tables)
    ctx = torch.zeros(1, dtype=torch.int32, device="cuda")
    for p in (64, 0):
        out = torch.full_like(q, float("nan"))
        try:
            gpu.set_partition_tokens(p)
            gpu.paged_decode(q, kp, vp, tab, ctx, out, pb.n_heads, pb.n_kv_heads, pb.head_dim,
                             pb.block_tokens, max_ctx=64)
        finally:
            gpu.set_partition_tokens(0)
        torch.cuda.synchronize()
        assert torch.all(out == 0).item()


def test_paged_variable_batch_and_partitions(gpu):
    lens = W.c3_lengths(seed=3, batch=24, lo=1, hi=3000)
    pb = W.paged_batch(lens, seed=3, spare_blocks=7)
    ref = W.reference_decode(pb, threads=8)
    try:
        for p in (64, 128, 1024, 4096, 0):
            gpu.set_partition_tokens(p)
            assert_close(run_paged(gpu, pb), ref, f"partition {p}")
    finally:
        gpu.set_partition_tokens(0)


def test_paged_q_pos(gpu):
    pb = W.paged_batch([300, 1000, 64], seed=4)
    q_pos = [100, 999, 0]
    assert_close(run_paged(gpu, pb, q_pos=q_pos), W.reference_decode(pb, q_pos=q_pos), "q_pos")


# ---------------------------------------------------------------- tracked (attention_tracked)

def run_tracked(gpu, pb, q_pos=None, window=0, global_stride=0, init=None, stride_pad=5):
    q = to_dev(pb.q)
    kp, vp = to_dev(pb.k_pool), to_dev(pb.v_pool)
    tab, ctx = to_dev(pb.tables), to_dev(pb.ctx_lens)
    qp = None if q_pos is None else to_dev(np.asarray(q_pos, np.int32))
    out = torch.full_like(q, float("nan"))
    max_ctx = int(pb.ctx_lens.max())
    imp0 = np.zeros((pb.batch, max_ctx + stride_pad)) if init is None else init
    imp = torch.from_numpy(imp0.copy()).cuda()
    gpu.paged_decode_tracked(q, kp, vp, tab, ctx, out, imp, pb.n_heads, pb.n_kv_heads,
                             pb.head_dim, pb.block_tokens, kv_dtype=pb.kv_dtype, window=window,
                             global_stride=global_stride, q_pos=qp)
    torch.cuda.synchronize()
    return out.cpu().numpy(), imp.cpu().numpy()


def test_tracked_importance_matches_oracle(gpu):
    """ops::attention_tracked: outputs and importance[t] = sum_h p_h[t] (f64),
    accumulated onto the caller's array, untouched past valid_end."""
    pb = W.paged_batch([300, 4096, 1, 2000], seed=7)
    q_pos = [250, 4095, 0, 1500]
    rng = np.random.default_rng(3)
    init = rng.random((pb.batch, 4096 + 3))
    out, imp = run_tracked(gpu, pb, q_pos=q_pos, init=init, stride_pad=3)
    assert_close(out, W.reference_decode(pb, q_pos=q_pos), "tracked out")
    for b in range(pb.batch):
        L = int(pb.ctx_lens[b])
        ref_out, ref_imp = oracle.attention(pb.q[b].reshape(-1), pb.layout(b), L, q_pos[b],
                                            pb.n_heads, pb.n_kv_heads, pb.head_dim,
                                            importance=True)
        got = imp[b] - init[b]
        ve = min(q_pos[b], L - 1)
        W.assert_importance(got[:L], ref_imp, f"importance b={b}")
        assert np.all(got[ve + 1:] == 0.0), f"importance past valid_end b={b}"
        assert abs(got.sum() - pb.n_heads) <= 1e-3, f"importance sum b={b}"


def test_tracked_split_and_window(gpu):
    """Tracked form with split-K partials (small partitions), and with a
    window: probabilities of the attended set sum to n_heads per sequence."""
    pb = W.paged_batch([5000, 700], seed=8)
    try:
        gpu.set_partition_tokens(64)
        out, imp = run_tracked(gpu, pb)
    finally:
        gpu.set_partition_tokens(0)
    assert_close(out, W.reference_decode(pb), "tracked split")
    for b in range(pb.batch):
        L = int(pb.ctx_lens[b])
        _, ref_imp = oracle.attention(pb.q[b].reshape(-1), pb.layout(b), L, L - 1, pb.n_heads,
                                      pb.n_kv_heads, pb.head_dim, importance=True)
        W.assert_importance(imp[b][:L], ref_imp, f"split importance b={b}")
    out, imp = run_tracked(gpu, pb, window=512, global_stride=64)
    for b in range(pb.batch):
        L = int(pb.ctx_lens[b])
        ref = W.window_importance(pb, b, L - 1, 512, 64, imp.shape[1])
        W.assert_importance(imp[b], ref, f"window importance b={b}")
        assert np.all(imp[b][ref == 0.0] == 0.0)


@pytest.mark.parametrize("window,global_stride", [(0, 0), (512, 64)])
def test_tracked_scores_then_importance(gpu, window, global_stride):
    """The tracked call's two launches as separate entry points give its
    results bit for bit: on one stream, and with the importance on a second
    stream ordered after the decode by an event while the first stream runs
    another decode into a second scores buffer."""
    pb = W.paged_batch([4096, 700, 1, 2500], seed=21)
    q_pos = [4095, 650, 0, 2499]
    q = to_dev(pb.q)
    kp, vp = to_dev(pb.k_pool), to_dev(pb.v_pool)
    tab, ctx = to_dev(pb.tables), to_dev(pb.ctx_lens)
    qp = to_dev(np.asarray(q_pos, np.int32))
    max_ctx = int(pb.ctx_lens.max())
    init = np.random.default_rng(22).random((pb.batch, max_ctx + 4))
    kw = dict(window=window, global_stride=global_stride, q_pos=qp)

    def fresh():
        return (torch.full_like(q, float("nan")), torch.from_numpy(init.copy()).cuda(),
                torch.full((pb.batch, pb.n_heads, max_ctx + 2), float("nan"), device="cuda"))

    out_t, imp_t, sc_t = fresh()
    gpu.paged_decode_tracked(q, kp, vp, tab, ctx, out_t, imp_t, pb.n_heads, pb.n_kv_heads,
                             pb.head_dim, pb.block_tokens, scores=sc_t, **kw)
    # one stream
    out_1, imp_1, sc_1 = fresh()
    gpu.paged_decode_scores(q, kp, vp, tab, ctx, out_1, sc_1, pb.n_heads, pb.n_kv_heads,
                            pb.head_dim, pb.block_tokens, **kw)
    gpu.paged_decode_importance(ctx, sc_1, imp_1, pb.n_heads, window=window,
                                global_stride=global_stride, q_pos=qp)
    # two streams: the importance of the first decode runs beside a second decode
    main, side = torch.cuda.Stream(), torch.cuda.Stream()
    out_2, imp_2, sc_2 = fresh()
    out_3, _, sc_3 = fresh()
    torch.cuda.synchronize()
    gpu.paged_decode_scores(q, kp, vp, tab, ctx, out_2, sc_2, pb.n_heads, pb.n_kv_heads,
                            pb.head_dim, pb.block_tokens, stream=main, **kw)
    ev = torch.cuda.Event()
    ev.record(main)
    side.wait_event(ev)
    gpu.paged_decode_importance(ctx, sc_2, imp_2, pb.n_heads, window=window,
                                global_stride=global_stride, q_pos=qp, stream=side)
    gpu.paged_decode_scores(q, kp, vp, tab, ctx, out_3, sc_3, pb.n_heads, pb.n_kv_heads,
                            pb.head_dim, pb.block_tokens, stream=main, **kw)
    torch.cuda.synchronize()
    assert gpu.take_status()[0] == 0
    ref = [x.cpu().numpy() for x in (out_t, imp_t, sc_t)]
    for name, got in (("one stream", (out_1, imp_1, sc_1)), ("two streams", (out_2, imp_2, sc_2))):
        got = [x.cpu().numpy() for x in got]
        assert np.array_equal(got[0], ref[0]), f"{name}: output"
        assert np.array_equal(got[1], ref[1]), f"{name}: importance"
        assert np.array_equal(got[2], ref[2], equal_nan=True), f"{name}: scores"
    assert np.array_equal(out_3.cpu().numpy(), ref[0]), "second decode"
    # and the tracked call itself against the oracle (importance added to init)
    for b in range(pb.batch):
        L = int(pb.ctx_lens[b])
        got = ref[1][b] - init[b]
        if window == 0:
            _, ref_imp = oracle.attention(pb.q[b].reshape(-1), pb.layout(b), L, q_pos[b],
                                          pb.n_heads, pb.n_kv_heads, pb.head_dim, importance=True)
            W.assert_importance(got[:L], ref_imp, f"importance b={b}")
        else:
            ref_imp = W.window_importance(pb, b, q_pos[b], window, global_stride, got.shape[0])
            W.assert_importance(got, ref_imp, f"window importance b={b}")


@pytest.mark.parametrize("lens,window,global_stride", [
    ([4096, 700, 1, 2500], 0, 0),                      # direct partition
    ([4096, 700, 1, 2500], 512, 64),                   # window with strided globals
    ([3000 + 97 * i for i in range(20)], 0, 0),        # stream-K partition
])
def test_tracked_pipelined_chain(gpu, lens, window, global_stride):
    """Three layers through the pipelined tracked decode (layer l's launch
    also sums layer l-1's importance; the last layer's sum is its own call)
    equal three tracked calls bit for bit: outputs, scores and importance."""
    B = len(lens)
    layers = [W.paged_batch(lens, seed=31 + i) for i in range(3)]
    q_pos = [max(0, L - 1 - i % 3) for i, L in enumerate(lens)]
    pb0 = layers[0]
    ctx, qp = to_dev(pb0.ctx_lens), to_dev(np.asarray(q_pos, np.int32))
    max_ctx = max(lens)
    init = np.random.default_rng(33).random((3, B, max_ctx + 3))
    kw = dict(window=window, global_stride=global_stride, q_pos=qp)
    dev = [(to_dev(pb.q), to_dev(pb.k_pool), to_dev(pb.v_pool), to_dev(pb.tables)) for pb in layers]
    ref = []
    for li, (q, kp, vp, tab) in enumerate(dev):
        out = torch.full_like(q, float("nan"))
        imp = torch.from_numpy(init[li].copy()).cuda()
        sc = torch.full((B, pb0.n_heads, max_ctx + 2), float("nan"), device="cuda")
        gpu.paged_decode_tracked(q, kp, vp, tab, ctx, out, imp, pb0.n_heads, pb0.n_kv_heads,
                                 pb0.head_dim, pb0.block_tokens, scores=sc, **kw)
        ref.append([x.cpu().numpy() for x in (out, imp, sc)])
    outs = [torch.full_like(d[0], float("nan")) for d in dev]
    imps = [torch.from_numpy(init[li].copy()).cuda() for li in range(3)]
    scs = [torch.full((B, pb0.n_heads, max_ctx + 2), float("nan"), device="cuda") for _ in range(2)]
    got_sc = []
    for li, (q, kp, vp, tab) in enumerate(dev):
        prev = scs[(li - 1) % 2] if li > 0 else None
        gpu.paged_decode_tracked_pipelined(q, kp, vp, tab, ctx, outs[li], scs[li % 2], prev,
                                           imps[li - 1] if li > 0 else None, pb0.n_heads,
                                           pb0.n_kv_heads, pb0.head_dim, pb0.block_tokens, **kw)
        if li > 0:
            got_sc.append(scs[(li - 1) % 2].cpu().numpy())  # after its sum ran (same stream)
    got_sc.append(scs[2 % 2].cpu().numpy())
    gpu.paged_decode_importance(ctx, scs[2 % 2], imps[2], pb0.n_heads, window=window,
                                global_stride=global_stride, q_pos=qp)
    torch.cuda.synchronize()
    assert gpu.take_status()[0] == 0
    for li in range(3):
        assert np.array_equal(outs[li].cpu().numpy(), ref[li][0]), f"layer {li}: output"
        assert np.array_equal(imps[li].cpu().numpy(), ref[li][1]), f"layer {li}: importance"
        assert np.array_equal(got_sc[li], ref[li][2], equal_nan=True), f"layer {li}: scores"
    # the chain's own checks: probabilities of each sequence's attended set sum to n_heads
    for li in range(3):
        got = imps[li].cpu().numpy() - init[li]
        assert np.allclose(got.sum(axis=1), pb0.n_heads, atol=1e-3), f"layer {li}: sums"
    # the previous scores may not be this call's scores buffer
    with pytest.raises(Exception):
        q, kp, vp, tab = dev[0]
        gpu.paged_decode_tracked_pipelined(q, kp, vp, tab, ctx, outs[0], scs[0], scs[0], imps[0],
                                           pb0.n_heads, pb0.n_kv_heads, pb0.head_dim,
                                           pb0.block_tokens, **kw)


def _check_tracked(pb, out, imp, init=None):
    assert_close(out, W.reference_decode(pb), "tracked out")
    for b in range(pb.batch):
        L = int(pb.ctx_lens[b])
        _, ref_imp = oracle.attention(pb.q[b].reshape(-1), pb.layout(b), L, L - 1, pb.n_heads,
                                      pb.n_kv_heads, pb.head_dim, importance=True)
        got = imp[b] - (0.0 if init is None else init[b])
        W.assert_importance(got[:L], ref_imp, f"importance b={b}")
        assert np.all(got[L:] == 0.0), f"importance past the context b={b}"


def test_tracked_calls_in_a_row_share_a_workspace(gpu):
    """Three tracked calls in a row on one workspace (batch 1, then 3, then 1
    at other lengths, so the split-K counters the previous call left at zero
    are reused under another layout) each match the oracle, onto nonzero
    importance arrays, with a clean status word."""
    ws = gpu.alloc_workspace(gpu.decode_workspace_size(3, 32, 4, 64, 6000))
    for lens, seed in (([4096], 11), ([5000, 64, 1777], 12), ([6000], 13)):
        pb = W.paged_batch(lens, seed=seed)
        q = to_dev(pb.q)
        kp, vp = to_dev(pb.k_pool), to_dev(pb.v_pool)
        tab, ctx = to_dev(pb.tables), to_dev(pb.ctx_lens)
        out = torch.full_like(q, float("nan"))
        init = np.random.default_rng(seed).random((pb.batch, 6000 + 2))
        imp = torch.from_numpy(init.copy()).cuda()
        gpu.paged_decode_tracked(q, kp, vp, tab, ctx, out, imp, pb.n_heads, pb.n_kv_heads,
                                 pb.head_dim, pb.block_tokens, max_ctx=max(lens), workspace=ws)
        assert gpu.take_status()[0] == 0
        torch.cuda.synchronize()
        _check_tracked(pb, out.cpu().numpy(), imp.cpu().numpy(), init)


def test_tracked_large_batch(gpu):
    """A batch with more segments than the direct partition takes (20 x 4
    kv heads: the stream-K partition) through the tracked form."""
    pb = W.paged_batch([97 * (i + 1) for i in range(20)], seed=14)
    out, imp = run_tracked(gpu, pb)
    assert gpu.take_status()[0] == 0
    _check_tracked(pb, out, imp)


@pytest.mark.parametrize("n_heads,n_kv,hd", [(8, 8, 64), (16, 8, 64), (32, 8, 128), (64, 4, 64),
                                             (32, 1, 128), (40, 2, 64)])
def test_paged_head_shapes(gpu, n_heads, n_kv, hd):
    pb = W.paged_batch([37, 700], n_heads=n_heads, n_kv_heads=n_kv, head_dim=hd, seed=5)
    assert_close(run_paged(gpu, pb), W.reference_decode(pb), f"{n_heads}/{n_kv}/{hd}")


def test_paged_c3_full_size(gpu):
    """Continuous batch at full size: 64 sequences, ctx ~ U[512, 32768]."""
    lens = W.c3_lengths(seed=0)
    pb = W.paged_batch(lens, seed=0)
    got = run_paged(gpu, pb)
    ref = W.reference_decode(pb, threads=oracle.max_threads())
    assert_close(got, ref, "64-sequence batch")


# ---------------------------------------------------------------- window / Q4

@pytest.mark.parametrize("stride", [0, 64])
def test_window_boundaries(gpu, stride):
    # valid_end in {window-1, window, window+1} and far past it
    w = 256
    pb = W.paged_batch([w, w + 1, w + 2, 3000, 9000], seed=6)
    got = run_paged(gpu, pb, window=w, global_stride=stride)
    assert_close(got, W.reference_decode(pb, window=w, global_stride=stride), f"window {stride}")


@pytest.mark.parametrize("stride", [0, 64])
def test_q4_window(gpu, stride):
    pb = W.paged_batch([5000, 4097, 300, 12000], seed=7, kv_dtype=oracle.KV_Q4)
    got = run_paged(gpu, pb, window=4096, global_stride=stride)
    assert_close(got, W.reference_decode(pb, window=4096, global_stride=stride), f"q4 {stride}")


def test_q4_full_and_d128(gpu):
    for hd in (64, 128):
        pb = W.paged_batch([1, 33, 2000], head_dim=hd, seed=8, kv_dtype=oracle.KV_Q4)
        assert_close(run_paged(gpu, pb), W.reference_decode(pb), f"q4 full d{hd}")


def test_c4_full_size_window(gpu):
    """4-bit KV: B=8, ctx 131072, window 4096, Q4-20B.  Only the rows
    the position set touches hold quantised N(0,1) data; every other row is
    random bytes, so reading a wrong row shows up as garbage or NaN."""
    B, ctx, w, bt, hkv, hd = 8, 131072, 4096, 16, 4, 64
    rng = np.random.default_rng(9)
    nblk = ctx // bt
    total = B * nblk
    perm = rng.permutation(total).astype(np.int32)
    tables = perm.reshape(B, nblk)
    rb = oracle.q4_row_bytes(hd)
    kp = rng.integers(0, 256, size=(total, hkv, bt, rb), dtype=np.uint8)
    vp = rng.integers(0, 256, size=(total, hkv, bt, rb), dtype=np.uint8)
    q = rng.standard_normal((B, 32, hd), dtype=np.float32)
    for stride in (0, 64):
        pos = oracle.sparse_positions(ctx, ctx - 1, w, stride)
        for b in range(B):
            blk = tables[b, pos // bt]
            kp[blk, :, pos % bt] = oracle.q4_quantize_rows(
                rng.standard_normal((len(pos), hkv, hd), dtype=np.float32))
            vp[blk, :, pos % bt] = oracle.q4_quantize_rows(
                rng.standard_normal((len(pos), hkv, hd), dtype=np.float32))
        pb = W.PagedBatch(q, kp, vp, tables, np.full(B, ctx, np.int32), 32, hkv, hd, bt,
                          oracle.KV_Q4, 9)
        got = run_paged(gpu, pb, window=w, global_stride=stride)
        ref = W.reference_decode(pb, window=w, global_stride=stride, threads=8)
        assert_close(got, ref, f"Q4 window stride {stride}")


# ---------------------------------------------------------------- position lists

def test_positions_fugu_set(gpu):
    pb = W.paged_batch([6000, 2500], seed=10)
    sets = [oracle.fugu_positions(6000, 5999, 256, 64, [5, 77, 5990, 3000, 4]),
            oracle.fugu_positions(2500, 2499, 1024, 0, [17, 18, 2499])]
    maxp = max(len(s) for s in sets)
    pos = np.zeros((2, maxp), np.int32)
    npos = np.array([len(s) for s in sets], np.int32)
    for b, s in enumerate(sets):
        pos[b, :len(s)] = s
    out = torch.full((2, 32, 64), float("nan"), device="cuda")
    import nyion_hip
    nyion_hip.paged_decode_positions(to_dev(pb.q), to_dev(pb.k_pool), to_dev(pb.v_pool),
                                     to_dev(pb.tables), to_dev(pos), to_dev(npos), out, 32, 4, 64,
                                     16)
    torch.cuda.synchronize()
    ref = np.stack([oracle.attention_positions(pb.q[b], pb.layout(b), sets[b], 32, 4, 64).reshape(
        32, 64) for b in range(2)])
    assert_close(out.cpu().numpy(), ref, "positions")


# ---------------------------------------------------------------- errors

def test_error_paths(gpu):
    import nyion_hip
    pb = W.paged_batch([100], seed=11)
    q, kp, vp = to_dev(pb.q), to_dev(pb.k_pool), to_dev(pb.v_pool)
    tab, ctx = to_dev(pb.tables), to_dev(pb.ctx_lens)
    out = torch.empty_like(q)
    with pytest.raises(nyion_hip.NyionError) as e:
        nyion_hip.paged_decode(q, kp, vp, tab, ctx, out, 32, 4, 64, 12)
    assert e.value.code == nyion_hip.ERR_INVALID
    with pytest.raises(nyion_hip.NyionError) as e:
        nyion_hip.paged_decode(q, kp, vp, tab, ctx, out, 32, 4, 96, 16)
    assert e.value.code == nyion_hip.ERR_UNSUPPORTED
    L = nyion_hip.load()
    rc = L.nyion_paged_decode_attention(q.data_ptr(), kp.data_ptr(), vp.data_ptr(), tab.data_ptr(),
                                        tab.shape[1], ctx.data_ptr(), None, 1, 32, 4, 64, 16,
                                        kp.shape[0], 0, 0, 0, 100000, 0.0, out.data_ptr(), None, 0,
                                        None)
    assert rc == nyion_hip.ERR_INVALID  # max_ctx beyond the table
