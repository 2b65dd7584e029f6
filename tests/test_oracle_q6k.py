"""The Q6_K GEMV oracle (swamp-kernels/src/fused_gemv_q6k.rs) against its own
bit layout, the reference's test blocks, a numpy restatement and float64
brute force (CPU)."""
import numpy as np
import pytest

import oracle
import workloads as W


def test_scale_conversion_all_patterns():
    """Normal values: IEEE binary16.  Exponent 0 and 31: the reference's bit
    formula (zero and subnormals become large negative numbers, inf/NaN finite
    values)."""
    for v in range(1 << 16):
        e = (v >> 10) & 0x1F
        got = np.float32(oracle.q6k_scale_to_f32(v))
        if 0 < e < 31:
            want = np.array([v], np.uint16).view(np.float16).astype(np.float32)[0]
        else:
            sign = (v >> 15) << 31
            mant = (v & 0x3FF) << 13
            bits = (sign | ((1009 << 23) & 0xFFFFFFFF) | mant) if e == 0 else (sign | ((e + 112) << 23) | mant)
            want = np.array([bits & 0xFFFFFFFF], np.uint32).view(np.float32)[0]
        assert got.view(np.uint32) == want.view(np.uint32), hex(v)
    assert oracle.q6k_scale_to_f32(0) < -1e34  # d = +0.0 in the reference


def _zero_block(d=1.0, scale=1):
    b = np.zeros(210, np.uint8)
    b[192:208] = scale
    b[208:210] = np.array([d], np.float16).view(np.uint8)
    return b


def test_bit_layout_probes():
    base = oracle.q6k_dequant(_zero_block(), 1, 256)[0]
    assert np.all(base == -32.0)
    b = _zero_block()
    b[64 + 5] = 0x70      # ql of half 1, l = 5: high nibble 7 (k = 2), low nibble 0
    b[128 + 32 + 5] = 0x20  # qh of half 1, l = 5: bits 4-5 = 2 (k = 2)
    got = oracle.q6k_dequant(b, 1, 256)[0]
    want = base.copy()
    want[128 + 5 + 64] = (7 | (2 << 4)) - 32
    assert np.array_equal(got, want)
    b = _zero_block()
    b[192 + 8 + 4] = np.uint8(253)  # scale -3 for half 1, l < 16, k = 2
    got = oracle.q6k_dequant(b, 1, 256)[0]
    want = base.copy()
    want[128 + 64:128 + 64 + 16] = -3.0 * -32.0
    assert np.array_equal(got, want)


def test_dequant_matches_numpy_restatement():
    w = W.q6k_random_weights(4, 768, seed=1)
    assert np.array_equal(oracle.q6k_dequant(w, 4, 768), W.q6k_dequant_np(w, 4, 768))


def test_reference_test_blocks():
    """fused_gemv_q6k.rs:358-376: the fused sum against dequantise-then-dot."""
    n_rows, n_blocks = 4, 3
    w = W.q6k_reference_test_weights(n_rows, n_blocks)
    n_cols = 256 * n_blocks
    x = np.sin(np.arange(n_cols, dtype=np.float32) * np.float32(0.01)).astype(np.float32)
    got = oracle.gemv_q6k(w, x, n_rows, n_cols).astype(np.float64)
    ref = oracle.q6k_dequant(w, n_rows, n_cols).astype(np.float64) @ x.astype(np.float64)
    assert np.all(np.abs(got - ref) <= 1e-4 * np.maximum(1.0, np.abs(ref)))
    assert np.array_equal(oracle.q6k_dequant(w, n_rows, n_cols), W.q6k_dequant_np(w, n_rows, n_cols))


@pytest.mark.parametrize("n_rows,n_cols", [(1, 256), (9, 512), (33, 2048)])
def test_gemv_vs_float64(n_rows, n_cols):
    w = W.q6k_random_weights(n_rows, n_cols, seed=n_rows)
    x = np.random.default_rng(n_cols).standard_normal(n_cols).astype(np.float32)
    got = oracle.gemv_q6k(w, x, n_rows, n_cols).astype(np.float64)
    ref = W.q6k_dequant_np(w, n_rows, n_cols).astype(np.float64) @ x.astype(np.float64)
    assert np.max(np.abs(got - ref)) <= 1e-5 * max(1.0, np.max(np.abs(ref)))
