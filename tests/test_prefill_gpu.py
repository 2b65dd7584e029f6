"""Causal prefill on MFMA against the oracle (gpu).

The oracle runs ops::attention per query row (as the reference's prefill
loop does) on the bf16-rounded q, k, v, in fp32.  Tolerance: max-abs-err <=
2e-3 and rel-err (max|diff| / max|ref|) <= 1e-3.
"""
import numpy as np
import pytest
import torch

import oracle
import workloads as W

pytestmark = pytest.mark.gpu

ATOL = 2e-3
RTOL = 1e-3


def run_prefill(gpu, q, k, v, causal=True, **kw):
    n, hq, d = q.shape
    hkv = k.shape[1]
    dq = torch.from_numpy(W.bf16_bits(q).view(np.int16)).cuda().view(torch.bfloat16)
    dk = torch.from_numpy(W.bf16_bits(k).view(np.int16)).cuda().view(torch.bfloat16)
    dv = torch.from_numpy(W.bf16_bits(v).view(np.int16)).cuda().view(torch.bfloat16)
    out = torch.full((n, hq, d), float("nan"), device="cuda")
    gpu.prefill_bf16(dq, dk, dv, out, hq, hkv, d, causal=causal, **kw)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def oracle_rows(q, k, v, rows, causal=True):
    n, hq, d = q.shape
    hkv = k.shape[1]
    qb, kb, vb = W.bf16_round(q), W.bf16_round(k), W.bf16_round(v)
    lay = oracle.token_major_layout(kb, vb, hkv, d)
    if causal:
        return oracle.attention_rows(qb.reshape(n, -1), lay, rows, hq, hkv, d,
                                     threads=oracle.max_threads()).reshape(n, hq, d)
    out = np.zeros_like(q)
    for r in rows:
        out[r] = oracle.attention(qb[r].reshape(-1), lay, n, n - 1, hq, hkv, d,
                                  threads=oracle.max_threads()).reshape(hq, d)
    return out


def check(got, ref, rows, what):
    g = got[rows].astype(np.float64)
    r = ref[rows].astype(np.float64)
    assert np.all(np.isfinite(g)), what
    err = np.max(np.abs(g - r))
    rel = err / np.max(np.abs(r))
    assert err <= ATOL and rel <= RTOL, f"{what}: max-abs {err:.3e} rel {rel:.3e}"


@pytest.mark.parametrize("n,hq,hkv,d", [(300, 8, 2, 128), (129, 4, 4, 64), (64, 8, 8, 128),
                                        (200, 16, 2, 128), (97, 2, 1, 64)])
def test_prefill_small_all_rows(gpu, n, hq, hkv, d):
    q, k, v = W.prefill_inputs(n, hq, hkv, d, seed=n)
    got = run_prefill(gpu, q, k, v)
    rows = np.arange(n)
    check(got, oracle_rows(q, k, v, rows), rows, f"prefill {n},{hq}/{hkv},{d}")


@pytest.mark.parametrize("shape", ["rising", "falling", "wide"])
def test_prefill_running_max_moves(gpu, shape):
    """Scores that rise along the keys (every tile passes the running max by
    far more than the weight-sum limit, so each half recomputes its
    weights against a new max), fall (the first tile holds the max, later
    weights underflow), or spread wide (random, scaled by 6): all rows
    against the oracle."""
    n, hq, hkv, d = 700, 4, 1, 64
    rng = np.random.default_rng(17)
    u = rng.standard_normal(d).astype(np.float32)
    u /= np.linalg.norm(u)
    t = np.arange(n, dtype=np.float32)
    if shape == "wide":
        q, k, v = W.prefill_inputs(n, hq, hkv, d, seed=18)
        q *= 6.0
        k *= 6.0
    else:
        # score of key t for every query (scale 1/8 at head_dim 64):
        # +-t / (2 ln 2) = +-0.72 t, i.e. 1.04 t in exp2 units, 33 per 32-key half
        sign = 1.0 if shape == "rising" else -1.0
        q = np.tile(u * 8.0, (n, hq, 1)).astype(np.float32)
        k = (sign * 0.5 / np.log(2.0) * t[:, None, None] * u[None, None, :]).astype(np.float32)
        k = np.repeat(k, hkv, axis=1)
        v = rng.standard_normal((n, hkv, d)).astype(np.float32)
    got = run_prefill(gpu, q, k, v)
    rows = np.arange(n)
    check(got, oracle_rows(q, k, v, rows), rows, f"running max {shape}")


def test_prefill_non_causal(gpu):
    q, k, v = W.prefill_inputs(257, 8, 2, 128, seed=1)
    got = run_prefill(gpu, q, k, v, causal=False)
    rows = np.array([0, 1, 100, 255, 256])
    check(got, oracle_rows(q, k, v, rows, causal=False), rows, "non-causal")


def test_prefill_c5_full_size_sampled_rows(gpu):
    """Causal prefill of 8192 tokens, 32/8 heads, D=128; every output is computed,
    416 rows (first, last and random) are checked against the oracle."""
    n = 8192
    q, k, v = W.prefill_inputs(n, 32, 8, 128, seed=0)
    got = run_prefill(gpu, q, k, v)
    rng = np.random.default_rng(5)
    rows = np.unique(np.concatenate([np.arange(64), np.arange(n - 64, n),
                                     rng.integers(0, n, 288)])).astype(np.int32)
    check(got, oracle_rows(q, k, v, rows), rows, "prefill 8192")
    assert np.all(np.isfinite(got))
    # the same rows against the oracle on the un-rounded fp32 inputs: this
    # measures the bf16 input cast, not the kernel, so it is reported with a
    # bound of its own (bf16 keeps 8 bits: scores move by ~1e-2 at D=128)
    lay = oracle.token_major_layout(k, v, 8, 128)
    ref32 = oracle.attention_rows(q.reshape(n, -1), lay, rows, 32, 8, 128,
                                  threads=oracle.max_threads()).reshape(n, 32, 128)
    err32 = float(np.max(np.abs(got[rows].astype(np.float64) - ref32[rows])))
    print(f"prefill 8192 vs un-rounded fp32 inputs: max-abs-err {err32:.3e}")
    assert err32 <= 5e-2, err32


def test_prefill_c5_full_size_with_paged_write(gpu):
    """The configuration's whole work: the 8192-token chunk (32/8 heads, D=128)
    attended and written into an f32 pool of 16-token blocks through a shuffled
    table (the save_at loop of executor.rs:106-111, cache.rs:749-811).  Every
    pool row of every token and kv head equals the bf16-rounded input (the
    chunk's K/V as the kernel reads them), blocks outside the table stay
    untouched, the output equals the call without pools bit for bit, and
    sampled rows match the oracle."""
    n, hq, hkv, d, bt = 8192, 32, 8, 128, 16
    q, k, v = W.prefill_inputs(n, hq, hkv, d, seed=0)
    nb = n // bt + 5
    table = np.random.default_rng(9).permutation(nb)[: n // bt].astype(np.int32)
    kp = torch.full((nb, hkv, bt, d), 7.0, device="cuda")
    vp = torch.full((nb, hkv, bt, d), 7.0, device="cuda")
    got = run_prefill(gpu, q, k, v, k_pool=kp, v_pool=vp,
                      block_table=torch.from_numpy(table).cuda(), block_tokens=bt,
                      kv_dtype=oracle.KV_F32, start_pos=0)
    assert gpu.take_status()[0] == 0
    bare = run_prefill(gpu, q, k, v)
    assert np.array_equal(got, bare), "output with the pool write differs from the bare call"
    kpn, vpn = kp.cpu().numpy(), vp.cpu().numpy()
    t = np.arange(n)
    assert np.array_equal(kpn[table[t // bt], :, t % bt], W.bf16_round(k)), "K pool rows"
    assert np.array_equal(vpn[table[t // bt], :, t % bt], W.bf16_round(v)), "V pool rows"
    spare = np.setdiff1d(np.arange(nb), table)
    assert len(spare) == 5 and np.all(kpn[spare] == 7.0) and np.all(vpn[spare] == 7.0)
    rng = np.random.default_rng(10)
    rows = np.unique(np.concatenate([np.arange(16), np.arange(n - 16, n),
                                     rng.integers(0, n, 96)])).astype(np.int32)
    check(got, oracle_rows(q, k, v, rows), rows, "prefill 8192 with paged write")


@pytest.mark.parametrize("kv_dtype,d,hq", [(oracle.KV_F32, 128, 8), (oracle.KV_F16, 128, 8),
                                           (oracle.KV_Q4, 128, 8), (oracle.KV_F32, 64, 8),
                                           (oracle.KV_F16, 64, 2), (oracle.KV_F32, 128, 16)])
def test_prefill_writes_paged_kv(gpu, kv_dtype, d, hq):
    """The chunk's K/V rows land in the pool at start_pos + row through the
    block table: f32 and binary16 (round to nearest even) by the prefill
    kernel itself (head_dim 128 and 64 kernels, one and two head subsets per
    kv head), Q4-20B by the quantising write."""
    n, hkv, bt, start = 200, 2, 16, 16
    q, k, v = W.prefill_inputs(n, hq, hkv, d, seed=2)
    nb = (start + n + bt - 1) // bt + 3
    table = np.random.default_rng(3).permutation(nb).astype(np.int32)
    rb = {oracle.KV_F32: d, oracle.KV_F16: d}.get(kv_dtype, oracle.q4_row_bytes(d))
    dt = {oracle.KV_F32: torch.float32, oracle.KV_F16: torch.int16}.get(kv_dtype, torch.uint8)
    kp = torch.zeros((nb, hkv, bt, rb), dtype=dt, device="cuda")
    vp = torch.zeros_like(kp)
    got = run_prefill(gpu, q, k, v, k_pool=kp, v_pool=vp,
                      block_table=torch.from_numpy(table).cuda(), block_tokens=bt,
                      kv_dtype=kv_dtype, start_pos=start)
    rows = np.arange(n)
    check(got, oracle_rows(q, k, v, rows), rows, "prefill+kv")
    t = np.arange(start, start + n)
    kh = kp.cpu().numpy()[table[t // bt], :, t % bt]
    vh = vp.cpu().numpy()[table[t // bt], :, t % bt]
    kb, vb = W.bf16_round(k), W.bf16_round(v)
    if kv_dtype == oracle.KV_F32:
        assert np.array_equal(kh, kb) and np.array_equal(vh, vb)
    elif kv_dtype == oracle.KV_F16:
        assert np.array_equal(kh.view(np.uint16), kb.astype(np.float16).view(np.uint16))
        assert np.array_equal(vh.view(np.uint16), vb.astype(np.float16).view(np.uint16))
    else:
        assert np.array_equal(kh, oracle.q4_quantize_rows(kb))
        assert np.array_equal(vh, oracle.q4_quantize_rows(vb))


# ---------------------------------------------------------------------------
# chunked prefill after a cached prefix (pos_offset > 0)
# ---------------------------------------------------------------------------

def to_dev_bf16(x):
    return torch.from_numpy(W.bf16_bits(x).view(np.int16)).cuda().view(torch.bfloat16)


def run_prefill_ctx(gpu, q, k, v, kh, vh, causal=True, **kw):
    n, hq, d = q.shape
    hkv = k.shape[1]
    out = torch.full((n, hq, d), float("nan"), device="cuda")
    dkh = None if kh is None else to_dev_bf16(kh)
    dvh = None if vh is None else to_dev_bf16(vh)
    gpu.prefill_bf16_ctx(to_dev_bf16(q), to_dev_bf16(k), to_dev_bf16(v), dkh, dvh, out, hq, hkv,
                         d, causal=causal, **kw)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def oracle_ctx_rows(q, k, v, kh, vh, rows, causal=True):
    """Row i of the chunk is query position n_hist + i over the history followed
    by the chunk: ops::attention with seq_len = n_hist + i + 1 (causal) or
    n_hist + n (non-causal), on bf16-rounded inputs."""
    n, hq, d = q.shape
    hkv = k.shape[1]
    nh = kh.shape[0]
    kall = W.bf16_round(np.concatenate([kh, k]))
    vall = W.bf16_round(np.concatenate([vh, v]))
    lay = oracle.token_major_layout(kall, vall, hkv, d)
    qb = W.bf16_round(q)
    out = np.zeros_like(q)
    if causal:
        qall = np.zeros((nh + n, hq * d), dtype=np.float32)
        qall[nh:] = qb.reshape(n, -1)
        res = oracle.attention_rows(qall, lay, np.asarray(rows) + nh, hq, hkv, d,
                                    threads=oracle.max_threads())
        out[rows] = res[np.asarray(rows) + nh].reshape(-1, hq, d)
        return out
    for r in rows:
        out[r] = oracle.attention(qb[r].reshape(-1), lay, nh + n, nh + n - 1, hq, hkv, d,
                                  threads=oracle.max_threads()).reshape(hq, d)
    return out


@pytest.mark.parametrize("n_hist,n,hq,hkv,d", [(1, 64, 8, 2, 128), (63, 130, 8, 2, 128),
                                               (64, 1, 4, 4, 64), (100, 97, 2, 1, 64),
                                               (257, 300, 16, 2, 128), (640, 33, 8, 8, 128)])
def test_prefill_ctx_all_rows(gpu, n_hist, n, hq, hkv, d):
    """History lengths on, just off and far from the 64-key tile edge, chunks of
    one row to several row blocks."""
    q, k, v = W.prefill_inputs(n, hq, hkv, d, seed=n + n_hist)
    _, kh, vh = W.prefill_inputs(n_hist, hq, hkv, d, seed=7 * n_hist + 1)
    got = run_prefill_ctx(gpu, q, k, v, kh, vh)
    rows = np.arange(n)
    check(got, oracle_ctx_rows(q, k, v, kh, vh, rows), rows,
          f"ctx {n_hist}+{n},{hq}/{hkv},{d}")


@pytest.mark.parametrize("n_hist,n,hq,hkv,d,causal", [
    (200, 150, 16, 2, 128, True),   # GQA 8:1: two four-head subsets per kv head
    (130, 70, 8, 1, 64, True),      # GQA 8:1 at D=64
    (65, 129, 4, 2, 64, True),      # GQA 2:1, history one past a tile edge
    (190, 40, 8, 2, 128, False),    # non-causal with a ragged history
    (33, 96, 6, 6, 64, True),       # MHA, six heads
])
def test_prefill_ctx_more_shapes(gpu, n_hist, n, hq, hkv, d, causal):
    q, k, v = W.prefill_inputs(n, hq, hkv, d, seed=3 * n + n_hist)
    _, kh, vh = W.prefill_inputs(n_hist, hq, hkv, d, seed=5 * n_hist + 2)
    got = run_prefill_ctx(gpu, q, k, v, kh, vh, causal=causal)
    rows = np.arange(n) if causal else np.array([0, 1, n // 2, n - 1])
    check(got, oracle_ctx_rows(q, k, v, kh, vh, rows, causal=causal), rows,
          f"ctx {n_hist}+{n},{hq}/{hkv},{d},causal={causal}")


def test_prefill_ctx_non_causal(gpu):
    q, k, v = W.prefill_inputs(100, 8, 2, 128, seed=11)
    _, kh, vh = W.prefill_inputs(77, 8, 2, 128, seed=12)
    got = run_prefill_ctx(gpu, q, k, v, kh, vh, causal=False)
    rows = np.array([0, 1, 50, 98, 99])
    check(got, oracle_ctx_rows(q, k, v, kh, vh, rows, causal=False), rows, "ctx non-causal")


def test_prefill_ctx_without_history_is_plain_prefill(gpu):
    """n_hist = 0 runs the same kernel path as nyion_prefill_attention_bf16:
    bit-identical outputs."""
    q, k, v = W.prefill_inputs(300, 8, 2, 128, seed=13)
    a = run_prefill(gpu, q, k, v)
    b = run_prefill_ctx(gpu, q, k, v, None, None)
    assert np.array_equal(a, b)


def test_prefill_ctx_rejects_missing_history(gpu):
    q, k, v = (to_dev_bf16(x) for x in W.prefill_inputs(8, 4, 4, 64, seed=1))
    out = torch.empty((8, 4, 64), device="cuda")
    rc = gpu.load().nyion_prefill_attention_bf16_ctx(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), None, None, 5, 8, 4, 4, 64, 1, 0.0,
        out.data_ptr(), None, None, None, 16, 0, 0, 0, None)
    assert rc != 0 and "history" in gpu.last_error()


@pytest.mark.parametrize("kv_dtype", [oracle.KV_F32, oracle.KV_Q4])
def test_chunked_prefill_through_paged_cache(gpu, kv_dtype):
    """prefill_slice over a 520-token prompt in chunks of 200, 200, 120: each
    chunk writes its K/V into the paged cache, the next chunk's history is
    gathered back from the cache (bf16) and attended.  With an f32 cache every
    row matches the one-shot oracle over the whole prompt; with Q4-20B the
    history is the quantised cache, as ops::attention reads it."""
    hq, hkv, d, bt = 8, 2, 128, 16
    chunks = [200, 200, 120]
    total = sum(chunks)
    q, k, v = W.prefill_inputs(total, hq, hkv, d, seed=21)
    nb = (total + bt - 1) // bt + 2
    table_np = np.random.default_rng(22).permutation(nb).astype(np.int32)
    table = torch.from_numpy(table_np).cuda()
    rb = d if kv_dtype == oracle.KV_F32 else oracle.q4_row_bytes(d)
    dt = torch.float32 if kv_dtype == oracle.KV_F32 else torch.uint8
    kp = torch.zeros((nb, hkv, bt, rb), dtype=dt, device="cuda")
    vp = torch.zeros_like(kp)
    got = np.zeros_like(q)
    pos = 0
    for c in chunks:
        sl = slice(pos, pos + c)
        kh = vh = None
        if pos:
            kh = torch.empty((pos, hkv, d), dtype=torch.bfloat16, device="cuda")
            vh = torch.empty_like(kh)
            gpu.kv_gather_bf16(kp, table, bt, hkv, d, kv_dtype, pos, kh)
            gpu.kv_gather_bf16(vp, table, bt, hkv, d, kv_dtype, pos, vh)
        out = torch.full((c, hq, d), float("nan"), device="cuda")
        gpu.prefill_bf16_ctx(to_dev_bf16(q[sl]), to_dev_bf16(k[sl]), to_dev_bf16(v[sl]), kh, vh,
                             out, hq, hkv, d, k_pool=kp, v_pool=vp, block_table=table,
                             block_tokens=bt, kv_dtype=kv_dtype)
        torch.cuda.synchronize()
        got[sl] = out.cpu().numpy()
        pos += c
    rows = np.arange(total)
    if kv_dtype == oracle.KV_F32:
        check(got, oracle_rows(q, k, v, rows), rows, "chunked f32")
        return
    # Q4: history keys/values are the dequantised cache rows
    kq = oracle.q4_dequant_rows(oracle.q4_quantize_rows(W.bf16_round(k)), d)
    vq = oracle.q4_dequant_rows(oracle.q4_quantize_rows(W.bf16_round(v)), d)
    pos = 0
    for c in chunks:
        sl = slice(pos, pos + c)
        r = np.arange(c)
        ref = oracle_ctx_rows(q[sl], k[sl], v[sl], kq[:pos], vq[:pos], r)
        check(got[sl], ref, r, f"chunked q4 at {pos}")
        pos += c


def test_chunked_prefill_f32_history_error(gpu):
    """A chunk after a history the f32 cache holds at full f32 precision (rows
    written by earlier decode steps, not by a bf16 prefill): the kernel attends
    the history gathered to bf16.  Against the oracle on that bf16 history it
    is held to the attention tolerance; against the reference's own semantics
    (ops::attention over the f32 cache, executor.rs:131-137, with the chunk's
    own bf16 q/k/v) the error is reported, bounded like the bf16 input cast of
    the full-size prefill."""
    hq, hkv, d, bt, n_hist, n = 8, 2, 128, 16, 1000, 300
    q, k, v = W.prefill_inputs(n, hq, hkv, d, seed=51)
    _, kh, vh = W.prefill_inputs(n_hist, hq, hkv, d, seed=52)
    nb = n_hist // bt + 2
    table_np = np.random.default_rng(53).permutation(nb).astype(np.int32)
    t = np.arange(n_hist)
    kpool = np.zeros((nb, hkv, bt, d), np.float32)
    vpool = np.zeros_like(kpool)
    kpool[table_np[t // bt], :, t % bt] = kh
    vpool[table_np[t // bt], :, t % bt] = vh
    table = torch.from_numpy(table_np).cuda()
    dkh = torch.empty((n_hist, hkv, d), dtype=torch.bfloat16, device="cuda")
    dvh = torch.empty_like(dkh)
    gpu.kv_gather_bf16(torch.from_numpy(kpool).cuda(), table, bt, hkv, d, oracle.KV_F32, n_hist, dkh)
    gpu.kv_gather_bf16(torch.from_numpy(vpool).cuda(), table, bt, hkv, d, oracle.KV_F32, n_hist, dvh)
    out = torch.full((n, hq, d), float("nan"), device="cuda")
    gpu.prefill_bf16_ctx(to_dev_bf16(q), to_dev_bf16(k), to_dev_bf16(v), dkh, dvh, out, hq, hkv, d)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    rows = np.arange(n)
    check(got, oracle_ctx_rows(q, k, v, kh, vh, rows), rows, "f32 history, bf16 semantics")
    # the reference's semantics: f32 history, the chunk's bf16 values
    kall = np.concatenate([kh, W.bf16_round(k)])
    vall = np.concatenate([vh, W.bf16_round(v)])
    lay = oracle.token_major_layout(kall, vall, hkv, d)
    qall = np.zeros((n_hist + n, hq * d), np.float32)
    qall[n_hist:] = W.bf16_round(q).reshape(n, -1)
    ref32 = oracle.attention_rows(qall, lay, rows + n_hist, hq, hkv, d,
                                  threads=oracle.max_threads())[n_hist:].reshape(n, hq, d)
    err32 = float(np.max(np.abs(got.astype(np.float64) - ref32)))
    rel32 = err32 / float(np.max(np.abs(ref32)))
    print(f"chunked prefill vs f32 history: max-abs-err {err32:.3e} rel {rel32:.3e}")
    assert err32 <= 5e-2, err32


@pytest.mark.parametrize("kv_dtype", [oracle.KV_F32, oracle.KV_Q4])
def test_kv_gather_bf16_bit_exact(gpu, kv_dtype):
    """bf16 gather = round-to-nearest-even of the f32 gather (dequantised for
    Q4-20B), token-major."""
    hkv, d, bt, n = 4, 64, 16, 150
    _, k, _ = W.prefill_inputs(n, 4, hkv, d, seed=31)
    nb = (n + bt - 1) // bt + 1
    table_np = np.random.default_rng(32).permutation(nb).astype(np.int32)
    table = torch.from_numpy(table_np).cuda()
    t = np.arange(n)
    if kv_dtype == oracle.KV_F32:
        pool = np.zeros((nb, hkv, bt, d), np.float32)
        pool[table_np[t // bt], :, t % bt] = k
        rows = k
    else:
        pool = np.zeros((nb, hkv, bt, oracle.q4_row_bytes(d)), np.uint8)
        pool[table_np[t // bt], :, t % bt] = oracle.q4_quantize_rows(k)
        rows = oracle.q4_dequant_rows(oracle.q4_quantize_rows(k), d)
    dpool = torch.from_numpy(pool).cuda()
    out = torch.empty((n, hkv, d), dtype=torch.bfloat16, device="cuda")
    gpu.kv_gather_bf16(dpool, table, bt, hkv, d, kv_dtype, n, out)
    torch.cuda.synchronize()
    got = out.cpu().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, W.bf16_bits(rows))
