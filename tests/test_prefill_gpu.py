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


def test_prefill_non_causal(gpu):
    q, k, v = W.prefill_inputs(257, 8, 2, 128, seed=1)
    got = run_prefill(gpu, q, k, v, causal=False)
    rows = np.array([0, 1, 100, 255, 256])
    check(got, oracle_rows(q, k, v, rows, causal=False), rows, "non-causal")


def test_prefill_c5_full_size_sampled_rows(gpu):
    """N=8192, 32/8 heads, D=128; every output is computed,
    416 rows (first, last and random) are checked against the oracle."""
    n = 8192
    q, k, v = W.prefill_inputs(n, 32, 8, 128, seed=0)
    got = run_prefill(gpu, q, k, v)
    rng = np.random.default_rng(5)
    rows = np.unique(np.concatenate([np.arange(64), np.arange(n - 64, n),
                                     rng.integers(0, n, 288)])).astype(np.int32)
    check(got, oracle_rows(q, k, v, rows), rows, "C5")
    assert np.all(np.isfinite(got))


@pytest.mark.parametrize("kv_dtype", [oracle.KV_F32, oracle.KV_Q4])
def test_prefill_writes_paged_kv(gpu, kv_dtype):
    n, hkv, d, bt, start = 200, 2, 128, 16, 16
    q, k, v = W.prefill_inputs(n, 8, hkv, d, seed=2)
    nb = (start + n + bt - 1) // bt + 3
    table = np.random.default_rng(3).permutation(nb).astype(np.int32)
    rb = d if kv_dtype == oracle.KV_F32 else oracle.q4_row_bytes(d)
    dt = torch.float32 if kv_dtype == oracle.KV_F32 else torch.uint8
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
    else:
        assert np.array_equal(kh, oracle.q4_quantize_rows(kb))
        assert np.array_equal(vh, oracle.q4_quantize_rows(vb))
