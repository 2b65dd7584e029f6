"""Per-layer sliding-window rings (PerLayerGpuState, scheduler.rs:36-178) and
the device-built attention_fugu position sets (ops.rs:463-484), against the
oracle (gpu)."""
import numpy as np
import pytest
import torch

import oracle
import workloads as W

pytestmark = pytest.mark.gpu

ATOL = 2e-3
RTOL = 1e-3


def assert_close(got, ref, what):
    err = float(np.max(np.abs(got.astype(np.float64) - ref)))
    rel = err / float(np.max(np.abs(ref)))
    assert np.all(np.isfinite(got)) and err <= ATOL and rel <= RTOL, f"{what}: {err:.3e} {rel:.3e}"


def test_layer_state_ring_window(gpu):
    """Token pos lands in slot pos % window; attention covers the last
    min(seq_len, window) tokens; layers keep separate rings."""
    Hq, Hkv, D, win, N, layers = 32, 4, 64, 256, 600, 2
    rng = np.random.default_rng(11)
    k = rng.standard_normal((layers, N, Hkv, D), dtype=np.float32)
    v = rng.standard_normal((layers, N, Hkv, D), dtype=np.float32)
    q = rng.standard_normal((N, Hq, D), dtype=np.float32)
    st = gpu.LayerState(win, Hq, Hkv, D, layers)
    try:
        for pos in range(N):
            for layer in range(layers):
                st.upload_kv(layer, k[layer, pos], v[layer, pos], pos)
            if pos in (0, 1, 100, 255, 256, 257, 511, 599):
                for layer in range(layers):
                    got = st.attention(layer, q[pos], pos, pos + 1)
                    lay = oracle.token_major_layout(k[layer], v[layer], Hkv, D)
                    first = max(0, pos + 1 - win)
                    ref = oracle.attention_positions(q[pos].reshape(-1), lay,
                                                     np.arange(first, pos + 1), Hq, Hkv, D)
                    assert_close(got.reshape(-1), ref, f"ring pos {pos} layer {layer}")
    finally:
        st.close()


def test_layer_state_errors(gpu):
    with pytest.raises(gpu.NyionError):
        gpu.LayerState(0, 32, 4, 64, 1)
    st = gpu.LayerState(16, 8, 2, 64, 1)
    try:
        with pytest.raises(gpu.NyionError):
            st.upload_kv(1, np.zeros((2, 64)), np.zeros((2, 64)), 0)
        with pytest.raises(gpu.NyionError):
            st.attention(0, np.zeros((8, 64)), 0, 0)
    finally:
        st.close()


def _dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def test_fugu_positions_match_oracle(gpu):
    """Bit-exact position lists: sentinels, window, DSPark extras with the
    first-occurrence rule (duplicates, positions past valid_end, positions
    already in the window or on a sentinel)."""
    ctx = np.array([100, 5000, 20000, 1, 300], np.int32)
    q_pos = np.array([99, 4999, 12345, 0, 200], np.int32)
    window, stride, nd = 256, 64, 12
    rng = np.random.default_rng(2)
    dspark = rng.integers(0, 20000, size=(len(ctx), nd)).astype(np.int32)
    dspark[1, :4] = [128, 4990, 128, 6000]     # sentinel, window, duplicate, future
    dspark[2, 5] = dspark[2, 2]
    maxp = 128 + window + 1 + nd
    pos = torch.full((len(ctx), maxp), -7, dtype=torch.int32, device="cuda")
    npos = torch.zeros(len(ctx), dtype=torch.int32, device="cuda")
    gpu.fugu_positions(_dev(ctx), window, stride, _dev(dspark), pos, npos, q_pos=_dev(q_pos))
    pos, npos = pos.cpu().numpy(), npos.cpu().numpy()
    for b in range(len(ctx)):
        ref = oracle.fugu_positions(int(ctx[b]), int(q_pos[b]), window, stride, dspark[b])
        assert npos[b] == len(ref), f"b={b}"
        assert np.array_equal(pos[b, :npos[b]], ref), f"b={b}"


def test_fugu_decode_end_to_end(gpu):
    """SparseWithDSPark step: device positions -> positions decode, against
    the oracle's attention over the same list."""
    pb = W.paged_batch([3000, 9000], seed=9)
    window, stride, nd = 256, 64, 32
    rng = np.random.default_rng(4)
    dspark = rng.integers(0, 9000, size=(pb.batch, nd)).astype(np.int32)
    maxp = 128 + window + 1 + nd
    ctx = _dev(pb.ctx_lens)
    pos = torch.empty((pb.batch, maxp), dtype=torch.int32, device="cuda")
    npos = torch.empty(pb.batch, dtype=torch.int32, device="cuda")
    gpu.fugu_positions(ctx, window, stride, _dev(dspark), pos, npos)
    q = _dev(pb.q)
    out = torch.full_like(q, float("nan"))
    gpu.paged_decode_positions(q, _dev(pb.k_pool), _dev(pb.v_pool), _dev(pb.tables), pos, npos,
                               out, pb.n_heads, pb.n_kv_heads, pb.head_dim, pb.block_tokens)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for b in range(pb.batch):
        L = int(pb.ctx_lens[b])
        plist = oracle.fugu_positions(L, L - 1, window, stride, dspark[b])
        ref = oracle.attention_positions(pb.q[b], pb.layout(b), plist, pb.n_heads,
                                         pb.n_kv_heads, pb.head_dim)
        assert_close(got[b].reshape(-1), ref, f"fugu decode b={b}")
