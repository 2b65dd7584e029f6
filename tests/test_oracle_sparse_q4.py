"""Pins the oracle's attention_sparse_q4 (swamp-engine/src/ops.rs:597-723) (CPU only).

That function reads Q4-20B rows with its own rules, which differ from the
cache writer's (cache.rs:655-663) and dequant_block's (cache.rs:375-394):
the 16 nibble bytes of a group give elements 0-15 from their low nibbles and
16-31 from their high nibbles (ops.rs:653-656), where the writer interleaves
them (element 2j low, 2j+1 high nibble of byte j).  Checks:
  * hand-built groups decoded element by element against values worked out by
    hand, and shown to differ from the writer's order;
  * a single attended position returns its V row in that order; two positions
    give the closed-form two-way softmax of hand-computed scores;
  * a weight below 1e-8 adds nothing (a zero row beside a non-zero one), a
    weight just above it does;
  * float64 brute force over random rows on a small shape (window + globals).
"""
import numpy as np
import pytest

import oracle

HD = 64
RB = oracle.q4_row_bytes(HD)


def f16_bytes(x: float) -> tuple[int, int]:
    b = np.array([x], np.float16).view(np.uint8)
    return int(b[0]), int(b[1])


def group(d: float, dmin: float, lo, hi) -> np.ndarray:
    """One 20-byte group: f16 d, f16 dmin, byte j = hi[j] << 4 | lo[j]."""
    g = np.zeros(20, np.uint8)
    g[0:2] = f16_bytes(d)
    g[2:4] = f16_bytes(dmin)
    g[4:20] = (np.asarray(hi, np.uint8) << 4) | np.asarray(lo, np.uint8)
    return g


def row(*groups) -> np.ndarray:
    return np.concatenate(groups)


J = np.arange(16)
ROW_A = row(group(1.0, 0.5, J, 15 - J), group(2.0, -3.0, (3 * J) % 16, (J + 5) % 16))


def test_a5_order_by_hand():
    got = oracle.q4_a5_row(ROW_A, HD)
    want = np.concatenate([J + 0.5, (15 - J) + 0.5, 2.0 * ((3 * J) % 16) - 3.0,
                           2.0 * ((J + 5) % 16) - 3.0]).astype(np.float32)
    assert np.array_equal(got, want)
    # the writer's order (dequant_block) reads the same bytes differently
    writer = oracle.q4_dequant_rows(ROW_A[None], HD)[0]
    w0 = np.empty(32, np.float32)
    w0[0::2], w0[1::2] = J + 0.5, (15 - J) + 0.5
    assert np.array_equal(writer[:32], w0)
    assert not np.array_equal(got, writer)


def layout_of(krows, vrows):
    k = np.ascontiguousarray(np.stack(krows)[None])  # [1 kv head][T][row]
    v = np.ascontiguousarray(np.stack(vrows)[None])
    return oracle.contiguous_layout(k, v, k.shape[1], HD, oracle.KV_Q4)


def test_single_position_returns_v_row_in_a5_order():
    zero = row(group(0.0, 0.0, J * 0, J * 0), group(0.0, 0.0, J * 0, J * 0))
    lay = layout_of([zero], [ROW_A])
    q = np.random.default_rng(1).standard_normal((2, HD)).astype(np.float32)
    out = oracle.attention_sparse_q4(q, lay, 1, 0, 2, 1, HD, 4096, 0).reshape(2, HD)
    assert np.array_equal(out, np.stack([oracle.q4_a5_row(ROW_A, HD)] * 2))


def test_two_positions_closed_form_scores():
    """q one-hot at element 1 (times 8, so scale 1/8 gives the element): the
    score of row A is its element 1 in the A5 order (1.5), not the writer's
    (15.5); row Z scores 0; V of row Z is zero, so out = w_A * V_A."""
    zero = row(group(0.0, 0.0, J * 0, J * 0), group(0.0, 0.0, J * 0, J * 0))
    v_a = row(group(0.5, 1.0, J, J), group(0.25, -2.0, 15 - J, J))
    lay = layout_of([ROW_A, zero], [v_a, zero])
    q = np.zeros((1, HD), np.float32)
    q[0, 1] = 8.0
    out = oracle.attention_sparse_q4(q, lay, 2, 1, 1, 1, HD, 4096, 0)
    va = oracle.q4_a5_row(v_a, HD).astype(np.float64)
    w_a5 = 1.0 / (1.0 + np.exp(-1.5))
    w_writer = 1.0 / (1.0 + np.exp(-15.5))
    assert np.allclose(out, w_a5 * va, rtol=2e-6, atol=1e-7)
    assert not np.allclose(out, w_writer * va, rtol=1e-3)


@pytest.mark.parametrize("a,skipped", [(2.0, True), (1.8, False)])
def test_weights_below_1e_8_are_skipped(a, skipped):
    """K row 0 all 1.25, row 1 all 0; q all a: scores 8 a 1.25 = 20 (weight of
    row 1 = e^-20/(1+e^-20) ~ 2.1e-9, skipped) or 18 (1.5e-8, kept).  V row 0
    is zero and V row 1 all 1, so the output is exactly that weight or 0."""
    const = row(group(0.0, 1.25, J * 0, J * 0), group(0.0, 1.25, J * 0, J * 0))
    zero = row(group(0.0, 0.0, J * 0, J * 0), group(0.0, 0.0, J * 0, J * 0))
    ones = row(group(0.0, 1.0, J * 0, J * 0), group(0.0, 1.0, J * 0, J * 0))
    lay = layout_of([const, zero], [zero, ones])
    q = np.full((1, HD), a, np.float32)
    out = oracle.attention_sparse_q4(q, lay, 2, 1, 1, 1, HD, 4096, 0)
    if skipped:
        assert np.all(out == 0.0)
    else:
        s = np.float64(np.float32(a)) * 64 * 1.25 / 8
        w = np.exp(-s) / (1.0 + np.exp(-s))
        assert np.allclose(out, w, rtol=1e-5) and w > 1e-8


@pytest.mark.parametrize("n,q_pos,window,stride,hq,hkv,hd", [
    (300, 299, 64, 16, 4, 2, 64),     # window + 14 globals
    (300, 150, 400, 8, 4, 1, 128),    # window past the start: every position
    (5000, 4999, 100, 20, 2, 1, 64),  # global cap of 128
    (50, 49, 10, 0, 2, 2, 64),        # no globals
])
def test_sparse_q4_matches_float64(n, q_pos, window, stride, hq, hkv, hd):
    rng = np.random.default_rng(n + window)
    rb = oracle.q4_row_bytes(hd)
    kq = oracle.q4_quantize_rows(rng.standard_normal((hkv * n, hd)).astype(np.float32))
    vq = oracle.q4_quantize_rows(rng.standard_normal((hkv * n, hd)).astype(np.float32))
    kq, vq = kq.reshape(hkv, n, rb), vq.reshape(hkv, n, rb)
    q = rng.standard_normal((hq, hd)).astype(np.float32)
    lay = oracle.contiguous_layout(kq, vq, n, hd, oracle.KV_Q4)
    out = oracle.attention_sparse_q4(q, lay, n, q_pos, hq, hkv, hd, window, stride).reshape(hq, hd)
    # the position set of attention_sparse (ops.rs:104-115 = 615-623)
    ve = min(q_pos, n - 1)
    ws = ve - window + 1 if ve > window else 0
    glob = [stride * g for g in range(min(ws // stride, 128))] if stride > 0 else []
    pos = np.array(glob + list(range(ws, ve + 1)))
    assert np.array_equal(pos, oracle.sparse_positions(n, q_pos, window, stride))

    def dec(b):  # independent numpy decode of the A5 order, float64
        g = b.reshape(-1, 20)
        d = g[:, 0:2].copy().view(np.float16).astype(np.float64)
        m = g[:, 2:4].copy().view(np.float16).astype(np.float64)
        nib = np.concatenate([g[:, 4:] & 15, g[:, 4:] >> 4], axis=1).astype(np.float64)
        return (d * nib + m).reshape(-1)

    for h in range(hq):
        kv = h // (hq // hkv)
        k = np.stack([dec(kq[kv, t]) for t in pos])
        v = np.stack([dec(vq[kv, t]) for t in pos])
        s = k @ q[h].astype(np.float64) / np.sqrt(hd)
        w = np.exp(s - s.max())
        w /= w.sum()
        ref = (w[w >= 1e-8, None] * v[w >= 1e-8]).sum(axis=0)
        assert np.max(np.abs(out[h] - ref)) < 2e-5 * max(1.0, np.abs(ref).max()), h
