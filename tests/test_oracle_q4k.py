"""The Q4_K GEMV oracle (swamp-kernels/src/fused_gemv_q4k.rs) against the
reference's own test weights, an independent numpy restatement and float64
brute force (CPU)."""
import numpy as np
import pytest

import oracle
import workloads as W


def test_scale_packing_round_trips():
    """unpack_scales_q4k inverts the reference test builder's packing for
    every 6-bit value in every slot."""
    rng = np.random.default_rng(0)
    for _ in range(200):
        s = rng.integers(0, 64, 8).astype(np.uint8)
        m = rng.integers(0, 64, 8).astype(np.uint8)
        gs, gm = oracle.q4k_unpack_scales(W.q4k_pack_scales(s, m))
        assert np.array_equal(gs, s) and np.array_equal(gm, m)
    for v in range(64):
        gs, gm = oracle.q4k_unpack_scales(W.q4k_pack_scales([v] * 8, [63 - v] * 8))
        assert np.all(gs == v) and np.all(gm == 63 - v)


@pytest.mark.parametrize("n_rows", [2, 3, 4, 7])
def test_reference_test_weights_closed_form(n_rows):
    """The reference tests' weights (constant nibble 8): every weight of row r
    is f32(d_r*s_r)*8 - f32(dmin_r*m_r), and the scalar path adds the
    products in element order 0..255, so a float32 loop gives the bits."""
    w = W.q4k_reference_test_weights(n_rows)
    x = W.q4k_reference_test_x(256)
    got = oracle.gemv_q4k(w, x, n_rows, 256)
    for r in range(n_rows):
        d = np.float32(np.float16(np.float32(0.5) + np.float32(r) * np.float32(0.1)))
        dm = np.float32(np.float16(np.float32(0.1) + np.float32(r) * np.float32(0.05)))
        sv = np.float32(d * np.float32((r + 1) & 63))
        mv = np.float32(dm * np.float32((r + 2) & 63))
        wf = np.float32(np.float32(sv * np.float32(8)) - mv)
        acc = np.float32(0)
        for i in range(256):
            acc = np.float32(acc + np.float32(wf * x[i]))
        assert got[r] == acc, (r, got[r], acc)
        # and the value itself: (8 sv - mv) * sum(x)
        assert abs(float(got[r]) - float(wf) * float(x.astype(np.float64).sum())) <= 1e-4 * abs(float(wf)) * 256


def test_dequant_matches_numpy_restatement():
    w = W.q4k_random_weights(5, 768, seed=1)
    assert np.array_equal(oracle.q4k_dequant(w, 5, 768), W.q4k_dequant_np(w, 5, 768))


def test_nibble_order():
    """qs pair p: low nibbles are sub-block 2p, high nibbles 2p+1."""
    qs = np.zeros(128, np.uint8)
    qs[32 * 1 + 5] = 0x3A  # pair 1, byte 5: element 64+5 gets 10, element 96+5 gets 3
    b = W.q4k_block(1.0, 0.0, [1] * 8, [0] * 8, qs)
    deq = oracle.q4k_dequant(b, 1, 256)[0]
    nz = np.nonzero(deq)[0]
    assert list(nz) == [69, 101] and deq[69] == 10.0 and deq[101] == 3.0


@pytest.mark.parametrize("n_rows,n_cols", [(1, 256), (9, 512), (33, 2048)])
def test_gemv_vs_float64(n_rows, n_cols):
    w = W.q4k_random_weights(n_rows, n_cols, seed=n_rows)
    x = np.random.default_rng(n_cols).standard_normal(n_cols).astype(np.float32)
    got = oracle.gemv_q4k(w, x, n_rows, n_cols).astype(np.float64)
    ref = W.q4k_dequant_np(w, n_rows, n_cols).astype(np.float64) @ x.astype(np.float64)
    assert np.max(np.abs(got - ref)) <= 1e-5 * max(1.0, np.max(np.abs(ref)))


def test_gemv_rejects_ragged_columns():
    with pytest.raises(ValueError):
        oracle.gemv_q4k(np.zeros(144, np.uint8), np.zeros(300, np.float32), 1, 300)
