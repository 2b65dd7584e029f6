"""Pins the CPU oracle before anything is compared against it (CPU only).

Each check is chosen so that a plausible mistake in the restatement (a wrong
index, a dropped term, a swapped nibble, a wrong rounding) fails it:
  * known-answer tests from the reference's own unit tests (golden JSON),
  * float64 brute force and closed forms for attention,
  * an independent numpy implementation of the Q4-20B byte format,
  * IEEE binary16 conversion against numpy on every f16 pattern.
"""
import json
import os

import numpy as np
import pytest

import oracle
import workloads as W

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))
L = oracle.lib()


# ---------------------------------------------------------------- simd.rs

def test_simd_dot_kats():
    for case in GOLD["simd_dot"]:
        if "n" in case:
            n = case["n"]
            a = (np.arange(n) * case["a_scale"]).astype(np.float32)
            b = (np.arange(n) * case["b_scale"]).astype(np.float32)
            expected = float(np.dot(a.astype(np.float64), b.astype(np.float64)))
        else:
            a = np.array(case["a"], np.float32)
            b = np.array(case["b"], np.float32)
            expected = case["expected"]
        got = L.orc_dot_avx512_order(a.ctypes.data, b.ctypes.data, len(a))
        assert abs(got - expected) < case["tol"], (case["ref"], got, expected)


def test_simd_weighted_sum_kat():
    case = GOLD["simd_weighted_sum"][0]
    out = np.array(case["out"], np.float32)
    v = np.array(case["v"], np.float32)
    L.orc_weighted_sum(out.ctypes.data, v.ctypes.data, case["score"], len(v))
    assert np.allclose(out, case["expected"], atol=case["tol"])


def test_dot_matches_float64_on_head_dims():
    rng = np.random.default_rng(1)
    for n in (8, 16, 24, 64, 100, 128):
        a = rng.standard_normal(n, dtype=np.float32)
        b = rng.standard_normal(n, dtype=np.float32)
        got = L.orc_dot_avx512_order(a.ctypes.data, b.ctypes.data, n)
        assert abs(got - float(a.astype(np.float64) @ b.astype(np.float64))) < 1e-5 * n


# ---------------------------------------------------------------- zones

def test_zone_block_sizes_golden():
    for pos, bs in GOLD["zone_block_size"]["cases"]:
        assert L.orc_zone_block_size(pos) == bs


def test_zone_page_ids_golden():
    g = GOLD["zone_page_id"]
    for pos, pid in g["cases"]:
        assert L.orc_zone_page_id(pos, g["max_seq_len"]) == pid, pos


def test_zone_offsets_are_a_bijection():
    """Every (layer, head, pos) of one page maps to a distinct f32 row and Q4 row."""
    n_kv, hd, layers = 3, 64, 2
    for start in (0, 4096, 131072):
        bs = L.orc_zone_block_size(start)
        seen_f, seen_q = set(), set()
        for layer in range(layers):
            for h in range(n_kv):
                for pos in range(start, start + bs):
                    f = L.orc_zone_f32_offset(layer, h, pos, n_kv, hd)
                    q = L.orc_zone_q4_offset(layer, h, pos, n_kv, hd)
                    assert f % hd == 0 and q % 40 == 0
                    seen_f.add(f)
                    seen_q.add(q)
        assert len(seen_f) == len(seen_q) == layers * n_kv * bs
        assert max(seen_f) == (layers * n_kv * bs - 1) * hd


# ---------------------------------------------------------------- f16

def test_f16_to_f32_every_pattern():
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_bits_to_f32(int(x)) for x in h], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_rne_matches_numpy():
    rng = np.random.default_rng(2)
    bits = rng.integers(0, 2**32, size=200000, dtype=np.uint64).astype(np.uint32)
    # concentrate on the f16 range, the subnormals, the rounding boundaries
    special = np.array([0, 0x80000000, 0x477FE000, 0x477FEFFF, 0x477FF000, 0x47800000,
                        0x33000000, 0x33000001, 0x337FFFFF, 0x33800000, 0x38800000, 0x387FC000,
                        0x7F800000, 0xFF800000, 0x3F800000, 0x3F801000, 0x3F803000,
                        0x3F802000, 0x00000001, 0x7F7FFFFF], np.uint32)
    scaled = (rng.standard_normal(100000) * np.exp2(rng.integers(-26, 17, 100000))).astype(
        np.float32).view(np.uint32)
    allb = np.concatenate([bits, special, scaled])
    x = allb.view(np.float32)
    ref = x.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f32_to_f16_bits(float(v)) for v in x], np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], ref[~nan])
    assert np.all(np.isnan(got[nan].view(np.float16)))


# ---------------------------------------------------------------- Q4-20B codec

def numpy_q4_quantize(x: np.ndarray) -> np.ndarray:
    """Independent vectorised statement of the Q4-20B writer for rows of 32*k
    elements: f32 arithmetic throughout, numpy's float16 cast, numpy's
    round-half-away built from floor."""
    x = np.asarray(x, np.float32)
    rows, d = x.shape
    g = x.reshape(rows, d // 32, 32)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        mx = np.nanmax(np.abs(g), axis=2, initial=np.float32(0.0)).astype(np.float32)
        mn = np.nanmin(g, axis=2, initial=np.float32(np.finfo(np.float32).max)).astype(np.float32)
        d_ = np.where(mx > np.float32(1e-10), mx / np.float32(7.0), np.float32(0.0)).astype(np.float32)
        t = ((g - mn[..., None]) / d_[..., None]).astype(np.float32)
        r = np.where(t >= 0, np.floor(t + np.float32(0.5)), -np.floor(-t + np.float32(0.5)))
        # half away from zero without the double-rounding of t+0.5
        r = np.where(np.abs(t - np.trunc(t)) == np.float32(0.5), np.trunc(t) + np.sign(t),
                     np.round(t))
        r = np.where(np.isnan(r), 0, r)
        r = np.clip(r, 0, 15)
        q = np.where(d_[..., None] > np.float32(1e-10), r, 0).astype(np.uint8)
    out = np.zeros((rows, d // 32, 20), np.uint8)
    out[..., 0:2] = d_.astype(np.float16).view(np.uint8).reshape(rows, d // 32, 2)
    out[..., 2:4] = mn.astype(np.float16).view(np.uint8).reshape(rows, d // 32, 2)
    out[..., 4:] = q[..., 0::2] | (q[..., 1::2] << 4)
    return out.reshape(rows, d // 32 * 20)


def numpy_q4_dequant(b: np.ndarray, d: int) -> np.ndarray:
    g = b.reshape(b.shape[0], d // 32, 20)
    dd = g[..., 0:2].copy().view(np.float16).astype(np.float32)
    dm = g[..., 2:4].copy().view(np.float16).astype(np.float32)
    nib = np.empty(g.shape[:2] + (32,), np.float32)
    nib[..., 0::2] = g[..., 4:] & 0x0F
    nib[..., 1::2] = g[..., 4:] >> 4
    return ((dd * nib).astype(np.float32) + dm).astype(np.float32).reshape(b.shape[0], d)


def _q4_rows(seed=3):
    rng = np.random.default_rng(seed)
    parts = [rng.standard_normal((20000, 64), dtype=np.float32),
             (rng.standard_normal((2000, 64)) * 1e-6).astype(np.float32),   # subnormal f16 d
             (rng.standard_normal((2000, 64)) * 3e4).astype(np.float32),    # near f16 max
             (rng.standard_normal((500, 64)) * 1e5).astype(np.float32),     # f16 overflow
             np.zeros((10, 64), np.float32),
             np.full((10, 64), 5.0, np.float32), np.full((10, 64), -3.25, np.float32),
             (rng.standard_normal((100, 64)) * 1e-12).astype(np.float32)]   # below 1e-10
    x = np.concatenate(parts)
    x[5, 3] = 0.0
    x[6, :] = -0.0
    return x


def test_q4_bytes_match_independent_numpy_statement():
    x = _q4_rows()
    got = oracle.q4_quantize_rows(x)
    ref = numpy_q4_quantize(x)
    assert np.array_equal(got, ref)


def test_q4_dequant_matches_independent_numpy_statement():
    x = _q4_rows()
    b = oracle.q4_quantize_rows(x)
    got = oracle.q4_dequant_rows(b, 64)
    ref = numpy_q4_dequant(b, 64)
    fin = np.isfinite(ref)
    assert np.array_equal(np.isfinite(got), fin)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))


def test_q4_nibble_order_and_header_layout():
    """Element i goes to byte 4 + i/2, low nibble when i is even (cache.rs:653-660)."""
    x = np.zeros((1, 32), np.float32)
    x[0, 1] = 7.0  # d = 1, dmin = 0: element 1 -> high nibble of byte 4
    x[0, 4] = 3.0  # element 4 -> low nibble of byte 6
    b = oracle.q4_quantize_rows(x)[0]
    assert b[0:2].view(np.float16)[0] == 1.0 and b[2:4].view(np.float16)[0] == 0.0
    assert b[4] == 0x70 and b[6] == 0x03 and b[5] == 0 and b[7:].sum() == 0


def test_q4_invariants_on_random_rows():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((5000, 128), dtype=np.float32)
    b = oracle.q4_quantize_rows(x)
    g = b.reshape(-1, 4, 20)
    nib = np.concatenate([g[..., 4:] & 15, g[..., 4:] >> 4], axis=-1)
    assert nib.max() <= 14  # (x - min)/(max|x|/7) <= 14
    xh = oracle.q4_dequant_rows(b, 128).reshape(-1, 4, 32)
    xg = x.reshape(-1, 4, 32)
    d32 = np.abs(xg).max(axis=2) / np.float32(7)
    d16 = g[..., 0:2].copy().view(np.float16).astype(np.float32)[..., 0]
    m16 = g[..., 2:4].copy().view(np.float16).astype(np.float32)[..., 0]
    bound = 0.5 * d32 + 15 * np.abs(d16 - d32) + np.abs(m16 - xg.min(axis=2)) + 1e-5
    assert np.all(np.abs(xg - xh) <= bound[..., None])


def test_q4_reference_roundtrip_tests():
    # cache.rs:892-926: constant rows round-trip exactly
    for pos in range(32):
        for val in (float(pos), float(2 * pos)):
            x = np.full((1, 64), val, np.float32)
            assert np.array_equal(oracle.q4_dequant_rows(oracle.q4_quantize_rows(x), 64), x)
    # cache.rs:853-890: first element pos*100+h (rest 0) within 1.0
    for pos in range(3):
        for h in range(4):
            for scale in (100, 1000):
                x = np.zeros((1, 64), np.float32)
                x[0, 0] = pos * scale + h
                xh = oracle.q4_dequant_rows(oracle.q4_quantize_rows(x), 64)
                assert abs(xh[0, 0] - x[0, 0]) < 1.0
    # cache.rs:1031-1068: D=128 constant rows at large magnitude within 10
    for pos in GOLD["q4_zone_read_write"]["positions"]:
        for val in (float(pos), float(3 * pos)):
            x = np.full((1, 128), val, np.float32)
            xh = oracle.q4_dequant_rows(oracle.q4_quantize_rows(x), 128)
            assert np.all(np.abs(xh - val) < 10.0)


# ---------------------------------------------------------------- position sets

@pytest.mark.parametrize("args,expected", [
    ((10, 9, 4, 2), [0, 2, 4, 6, 7, 8, 9]),
    ((5, 4, 4, 2), [0, 1, 2, 3, 4]),              # valid_end == window: strict '>'
    ((4, 3, 4, 2), [0, 1, 2, 3]),                 # valid_end == window - 1
    ((6, 5, 4, 2), [0, 2, 3, 4, 5]),              # valid_end == window + 1
    ((100, 50, 10, 0), list(range(41, 51))),      # q_pos < seq_len-1, no globals
    ((100, 500, 10, 64), [0] + list(range(90, 100))),  # q_pos past the end clamps; 90/64 = 1 global
])
def test_sparse_positions_golden(args, expected):
    assert oracle.sparse_positions(*args).tolist() == expected


def test_sparse_positions_global_cap():
    pos = oracle.sparse_positions(20000, 19999, 256, 64)
    assert pos[:128].tolist() == [64 * g for g in range(128)]
    assert pos[128:].tolist() == list(range(19744, 20000))


def test_fugu_positions_golden():
    pos = oracle.fugu_positions(100, 50, 10, 16, [3, 60, 41, 3, 200])
    assert pos.tolist() == [0, 16] + list(range(41, 51)) + [3]


# ---------------------------------------------------------------- attention

def _gather(pool, table, bt, h, n):
    t = np.arange(n)
    return pool[table[t // bt], h, t % bt]


def test_attention_c1_matches_float64():
    q, k, v = W.c1_contiguous(seed=0)
    lay = oracle.contiguous_layout(k, v, 128, 64)
    out = oracle.attention(q.reshape(-1), lay, 128, 127, 32, 4, 64).reshape(32, 64)
    for h in range(32):
        ref = W.brute_force_attention(q[h], k[h // 8], v[h // 8], 127)
        assert np.max(np.abs(out[h] - ref)) < 2e-6


def test_attention_paged_matches_float64_gather():
    pb = W.paged_batch([1, 15, 16, 17, 100, 333], seed=5)
    out = W.reference_decode(pb)
    for b in range(pb.batch):
        n = int(pb.ctx_lens[b])
        for h in range(pb.n_heads):
            kv = h // 8
            ref = W.brute_force_attention(pb.q[b, h], _gather(pb.k_pool, pb.tables[b], 16, kv, n),
                                          _gather(pb.v_pool, pb.tables[b], 16, kv, n), n - 1)
            assert np.max(np.abs(out[b, h] - ref)) < 5e-6, (b, h)


def test_attention_q_pos_masks_future():
    pb = W.paged_batch([200], seed=6)
    lay = pb.layout(0)
    out = oracle.attention(pb.q[0], lay, 200, 120, 32, 4, 64).reshape(32, 64)
    for h in (0, 9, 31):
        ref = W.brute_force_attention(pb.q[0, h], _gather(pb.k_pool, pb.tables[0], 16, h // 8, 200),
                                      _gather(pb.v_pool, pb.tables[0], 16, h // 8, 200), 120)
        assert np.max(np.abs(out[h] - ref)) < 5e-6


def test_attention_closed_forms():
    rng = np.random.default_rng(7)
    D = 64
    q = rng.standard_normal((8, D), dtype=np.float32)
    v = rng.standard_normal((1, 50, D), dtype=np.float32)
    # seq_len 1 -> V[0]
    k = rng.standard_normal((1, 50, D), dtype=np.float32)
    out = oracle.attention(q, oracle.contiguous_layout(k, v, 50, D), 1, 0, 8, 1, D).reshape(8, D)
    assert np.array_equal(out, np.repeat(v[0, :1], 8, axis=0))
    # identical keys -> uniform weights -> mean of V
    k2 = np.repeat(k[:, :1], 50, axis=1).copy()
    out = oracle.attention(q, oracle.contiguous_layout(k2, v, 50, D), 50, 49, 8, 1, D).reshape(8, D)
    assert np.max(np.abs(out - v[0].mean(axis=0))) < 2e-6
    # one key far ahead (score gap >= 40) -> that row of V
    k3 = rng.standard_normal((1, 50, D), dtype=np.float32) * 0.01
    k3[0, 17] = q[0] * (400.0 / float(q[0] @ q[0]))  # score = 400/8 = 50
    out = oracle.attention(q[:1].copy(), oracle.contiguous_layout(k3, v, 50, D), 50, 49, 1, 1,
                           D)
    assert np.max(np.abs(out - v[0, 17])) < 1e-6


def test_attention_importance_sums_to_heads():
    pb = W.paged_batch([300], seed=8)
    _, imp = oracle.attention(pb.q[0], pb.layout(0), 300, 250, 32, 4, 64, importance=True)
    assert np.all(imp >= 0) and np.all(imp[251:] == 0)
    assert abs(imp.sum() - 32.0) < 1e-4


def test_attention_gqa_head_permutation():
    pb = W.paged_batch([90], seed=9)
    lay = pb.layout(0)
    out = oracle.attention(pb.q[0], lay, 90, 89, 32, 4, 64).reshape(32, 64)
    perm = np.arange(32)
    perm[8:16] = perm[8:16][::-1]
    out2 = oracle.attention(pb.q[0][perm].copy(), lay, 90, 89, 32, 4, 64).reshape(32, 64)
    assert np.array_equal(out2, out[perm])


def test_attention_q4_equals_attention_on_dequantised_pool():
    pb = W.paged_batch([77, 260], seed=10, kv_dtype=oracle.KV_Q4)
    kf = oracle.q4_dequant_rows(pb.k_pool, 64)
    vf = oracle.q4_dequant_rows(pb.v_pool, 64)
    for b in range(2):
        n = int(pb.ctx_lens[b])
        o4 = oracle.attention(pb.q[b], pb.layout(b), n, n - 1, 32, 4, 64)
        of = oracle.attention(pb.q[b], oracle.paged_layout(kf, vf, pb.tables[b], 16, 4, 64), n,
                              n - 1, 32, 4, 64)
        assert np.array_equal(o4, of)


def test_attention_f16_equals_attention_on_widened_pool():
    """binary16 rows are widened exactly before use: the oracle on an f16 pool
    equals the oracle on the f32 pool holding the same values, bit for bit."""
    pb = W.paged_batch([300, 17], seed=4, kv_dtype=oracle.KV_F16)
    kf = pb.k_pool.view(np.float16).astype(np.float32)
    vf = pb.v_pool.view(np.float16).astype(np.float32)
    for b in range(2):
        lay_f = oracle.paged_layout(kf, vf, pb.tables[b], 16, 4, 64)
        L = int(pb.ctx_lens[b])
        a = oracle.attention(pb.q[b], pb.layout(b), L, L - 1, 32, 4, 64)
        r = oracle.attention(pb.q[b], lay_f, L, L - 1, 32, 4, 64)
        assert np.array_equal(a, r)
    # and the f16 pool holds numpy's round-to-nearest-even of the f32 draw
    rng = np.random.default_rng(4)
    x = rng.standard_normal(1000, dtype=np.float32)
    assert np.array_equal(np.array([oracle.f32_to_f16_bits(float(v)) for v in x], np.uint16),
                          x.astype(np.float16).view(np.uint16))


def test_attention_positions_matches_float64():
    pb = W.paged_batch([5000], seed=11)
    pos = oracle.sparse_positions(5000, 4999, 256, 64)
    out = oracle.attention_positions(pb.q[0], pb.layout(0), pos, 32, 4, 64).reshape(32, 64)
    for h in (0, 13, 31):
        kk = _gather(pb.k_pool, pb.tables[0], 16, h // 8, 5000)[pos]
        vv = _gather(pb.v_pool, pb.tables[0], 16, h // 8, 5000)[pos]
        ref = W.brute_force_attention(pb.q[0, h], kk, vv, len(pos) - 1)
        assert np.max(np.abs(out[h] - ref)) < 5e-6


def test_attention_rows_is_causal_prefill():
    q, k, v = W.prefill_inputs(96, n_heads=8, n_kv_heads=2, head_dim=64, seed=12)
    lay = oracle.token_major_layout(k, v, 2, 64)
    rows = [0, 1, 31, 32, 95]
    out = oracle.attention_rows(q.reshape(96, -1), lay, rows, 8, 2, 64).reshape(96, 8, 64)
    for r in rows:
        for h in range(8):
            ref = W.brute_force_attention(q[r, h], k[:, h // 4], v[:, h // 4], r)
            assert np.max(np.abs(out[r, h] - ref)) < 5e-6


# ---------------------------------------------------------------- swamp-kernels

def test_exp_q16_16_reference_accuracy():
    g = GOLD["exp_q16_16"]
    worst = 0.0
    for x in range(g["x_from"], g["x_to"] + 1, g["step"]):
        got = oracle.exp_q16_16(x) / 65536.0
        exp = np.exp(x / 65536.0)
        worst = max(worst, abs(got - exp) / exp)
    assert worst < g["max_rel_err"]
    assert oracle.exp_q16_16(0) == 65536 and oracle.exp_q16_16(5) == 65536
    assert oracle.exp_q16_16(-655361) == 0 and oracle.exp_q16_16(-655360) == 3


def test_softmax_padic_reference_test():
    g = GOLD["softmax_padic"]
    p = oracle.softmax_padic(g["logits"], g["temperature"])
    assert abs(p.sum() - 1.0) < g["sum_tol"]
    assert int(np.argmax(p)) == g["argmax"]


def test_softmax_padic_integer_pipeline_by_hand():
    # two equal logits (scalar tail lanes): e = 65536 each, inv = 2^32/2^17
    assert oracle.softmax_padic([0.0, 0.0]).tolist() == [0.5, 0.5]
    # sixteen equal logits (vector lanes): (65536*4096 mod 2^32) >> 16 = 4096
    assert np.all(oracle.softmax_padic(np.zeros(16)) == 1.0 / 16)
    # one dominant logit: e*inv = 2^32 wraps to 0 in the vector lanes ...
    x = np.zeros(16, np.float32)
    x[0] = 100.0
    assert oracle.softmax_padic(x)[0] == 0.0
    # ... but not in the scalar tail
    assert oracle.softmax_padic([100.0, 0.0]).tolist() == [1.0, 0.0]
    # temperature is clamped to 1e-6; NaN logits become fixed-point 0
    assert oracle.softmax_padic([1e-7, 0.0], 0.0)[0] > 0.5
    assert oracle.softmax_padic([np.nan, 0.0]).tolist() == [0.5, 0.5]


def test_stokes_evicts_first_minimum():
    c = L.orc_stokes_init(4)
    key = np.zeros(4, np.float32)
    for i in range(4097):
        key[:] = i
        score = 1.0 if i != 1234 else -5.0
        assert L.orc_stokes_append(c, i, key.ctypes.data, key.ctypes.data, score) == 0
    assert L.orc_stokes_count(c) == 4096
    keys = np.zeros((4096, 4), np.float32)
    scores = np.zeros(4096, np.float32)
    L.orc_stokes_read(c, keys.ctypes.data, None, scores.ctypes.data)
    assert 1234.0 not in keys[:, 0] and keys[1233, 0] == 1233.0 and keys[1234, 0] == 1235.0
    # ties: the first minimum goes
    key[:] = 9999
    L.orc_stokes_append(c, 0, key.ctypes.data, key.ctypes.data, 1.0)
    L.orc_stokes_read(c, keys.ctypes.data, None, None)
    assert keys[0, 0] == 1.0 and keys[-1, 0] == 9999.0
    # NaN scores make the reference panic; here: error code
    L.orc_stokes_append(c, 0, key.ctypes.data, key.ctypes.data, float("nan"))
    assert L.orc_stokes_append(c, 0, key.ctypes.data, key.ctypes.data, 2.0) == -1
    L.orc_stokes_free(c)


# ---------------------------------------------------------------- RoPE

def test_rope_lut_against_float64():
    """init_rope_lut (ops.rs:20-37): cos/sin of m * 10000^(-2k/D) with the
    angle formed in f32; checked against float64 trigonometry of the exact
    angle, within the f32 rounding of freq (powf, divide) and of m * freq."""
    D, M = 128, 4096
    lut = oracle.rope_lut(D, M).astype(np.float64)
    k = np.arange(D // 2)
    exact = np.arange(M)[:, None] * np.power(10000.0, -2.0 * k / D)[None, :]
    tol = 2e-7 + np.abs(exact) * 3.6e-7
    assert np.all(np.abs(lut[..., 0] - np.cos(exact)) < tol)
    assert np.all(np.abs(lut[..., 1] - np.sin(exact)) < tol)
    assert np.all(lut[0, :, 0] == 1.0) and np.all(lut[0, :, 1] == 0.0)
    # k = 0: freq is exactly 1, the angle is m itself
    assert np.max(np.abs(lut[:, 0, 0] - np.cos(np.arange(M)))) < 2e-7


def test_apply_rope_rotation():
    """apply_rope_ufc: pos 0 is the identity; pairs keep their norm; the
    result matches a float64 rotation by the table's (cos, sin); positions
    past max_ctx use the last row (ops.rs:53)."""
    rng = np.random.default_rng(0)
    D, M = 64, 300
    lut = oracle.rope_lut(D, M)
    q = rng.standard_normal((8, D), dtype=np.float32)
    k = rng.standard_normal((2, D), dtype=np.float32)
    q0, k0 = oracle.apply_rope(q, k, 0, M, lut)
    assert np.array_equal(q0, q) and np.array_equal(k0, k)
    q1, k1 = oracle.apply_rope(q, k, 123, M, lut)
    c, s = lut[123, :, 0].astype(np.float64), lut[123, :, 1].astype(np.float64)
    x, y = q[:, 0::2].astype(np.float64), q[:, 1::2].astype(np.float64)
    assert np.max(np.abs(q1[:, 0::2] - (x * c - y * s))) < 1e-6
    assert np.max(np.abs(q1[:, 1::2] - (x * s + y * c))) < 1e-6
    n0 = x ** 2 + y ** 2
    n1 = q1[:, 0::2].astype(np.float64) ** 2 + q1[:, 1::2].astype(np.float64) ** 2
    assert np.max(np.abs(n1 - n0) / n0) < 1e-5
    qa, _ = oracle.apply_rope(q, k, 10 * M, M, lut)
    qb, _ = oracle.apply_rope(q, k, M - 1, M, lut)
    assert np.array_equal(qa, qb)


# ---------------------------------------------------------------- Mojo FFI

def _mojo_dequant(rows, head_dim):
    """f32 values of Mojo-format rows through the Q4-20B dequantiser (an
    independent path: the words carry the f16 d, dmin and nibble bytes)."""
    n = rows.shape[0]
    blocks = (head_dim + 31) // 32
    w = rows.reshape(n, blocks, 20)
    b = np.zeros((n, blocks, 20), np.uint8)
    b[:, :, 0:2] = w[:, :, 0].astype(np.float16).view(np.uint8).reshape(n, blocks, 2)
    b[:, :, 2:4] = w[:, :, 1].astype(np.float16).view(np.uint8).reshape(n, blocks, 2)
    b[:, :, 4:20] = w[:, :, 2:18].astype(np.uint8)
    return oracle.q4_dequant_rows(b.reshape(n, blocks * 20), head_dim)


def test_mojo_one_tile_is_softmax_attention():
    """<= 64 positions: one tile, so the result is softmax attention over the
    listed positions (every head against the one K/V)."""
    rng = np.random.default_rng(7)
    for hd, n_pos in ((64, 40), (128, 64), (96, 17)):
        x_k = rng.standard_normal((300, hd)).astype(np.float32)
        x_v = rng.standard_normal((300, hd)).astype(np.float32)
        kq, vq = oracle.mojo_q4_rows(x_k), oracle.mojo_q4_rows(x_v)
        q = rng.standard_normal((3, hd)).astype(np.float32)
        pos = rng.choice(300, n_pos, replace=False).astype(np.int32)
        got = oracle.mojo_sparse_attention_q4(q, kq, vq, pos, 3, hd)
        k = _mojo_dequant(kq, hd)[None]
        v = _mojo_dequant(vq, hd)[None]
        lay = oracle.contiguous_layout(np.ascontiguousarray(k), np.ascontiguousarray(v), 300, hd)
        ref = oracle.attention_positions(q, lay, pos, 3, 1, hd).reshape(3, hd)
        assert np.allclose(got, ref, rtol=1e-5, atol=1e-6), (hd, np.abs(got - ref).max())


def test_mojo_tiles_normalise_by_the_running_denominator():
    """Equal scores over 150 positions (tiles of 64, 64, 22): tile k's weights
    are 1 / (positions seen so far), so out = sum(v1)/64 + sum(v2)/128 +
    sum(v3)/150, not the mean."""
    rng = np.random.default_rng(8)
    hd = 64
    kq = np.repeat(oracle.mojo_q4_rows(rng.standard_normal((1, hd)).astype(np.float32)), 150, axis=0)
    vq = oracle.mojo_q4_rows(rng.standard_normal((150, hd)).astype(np.float32))
    q = rng.standard_normal((2, hd)).astype(np.float32)
    pos = np.arange(150, dtype=np.int32)
    got = oracle.mojo_sparse_attention_q4(q, kq, vq, pos, 2, hd)
    v = _mojo_dequant(vq, hd).astype(np.float64)
    want = v[:64].sum(0) / 64 + v[64:128].sum(0) / 128 + v[128:].sum(0) / 150
    assert np.allclose(got, np.broadcast_to(want, got.shape), rtol=1e-5, atol=1e-6)
    assert not np.allclose(got[0], v.mean(0), rtol=1e-3)


def test_mojo_skips_weights_below_1e_8():
    """Position 1's weight exp(-21.2) ~ 6e-10 is skipped: its V row (9e5 per
    element) would otherwise add ~5.5e-4 to an output of 1.0."""
    hd = 32
    k = np.zeros((2, 20), np.float32)
    k[0, 0], k[0, 2:18] = 0.25, 255.0     # k0 = 3.75 per element: s0 = 3.75*32/sqrt(32)
    v = np.zeros((2, 20), np.float32)
    v[0, 0], v[0, 2:18] = 1.0 / 15.0, 255.0  # v0 = 15 * (1/15) per element
    v[1, 0], v[1, 2:18] = 60000.0, 255.0     # v1 = 900000 per element
    q = np.ones((1, hd), np.float32)
    got = oracle.mojo_sparse_attention_q4(q, k, v, np.array([0, 1], np.int32), 1, hd)
    v0 = np.float32(np.float32(1.0 / 15.0) * np.float32(15.0))
    assert np.all(got == v0), got[0, :4]
