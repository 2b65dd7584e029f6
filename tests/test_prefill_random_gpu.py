"""Seeded random sweep of causal prefill against the oracle (gpu).

Each case draws kv heads (1..8), a GQA group of 1..16 q heads per kv head
(odd groups included: 3, 5 and 7 run one q head per workgroup),
head_dim 64 or 128, a chunk of 1..400 rows and, in two cases of three, a
cached history of 1..400 tokens before it (the chunked prefill of
swamp-engine/src/executor.rs:85-137: row i attends to keys [0, n_hist + i]),
causal in most cases.  The oracle is the per-row ops::attention loop on the
bf16-rounded inputs; tolerance max-abs-err <= 2e-3 and max|diff| / max|ref|
<= 1e-3 (the helpers are those of test_prefill_gpu)."""
import numpy as np
import pytest

import test_prefill_gpu as P
import workloads as W

pytestmark = pytest.mark.gpu

N_CASES = 24


def draw(seed):
    rng = np.random.default_rng(2000 + seed)
    hkv = int(rng.choice([1, 2, 4, 8]))
    group = int(rng.choice([1, 2, 3, 4, 5, 6, 7, 8, 12, 16]))
    while hkv * group > 32:
        group //= 2
    d = int(rng.choice([64, 128]))
    n = int(rng.integers(1, 401))
    n_hist = int(rng.integers(1, 401)) if seed % 3 else 0
    causal = bool(rng.random() < 0.85)
    return dict(hkv=hkv, hq=hkv * group, d=d, n=n, n_hist=n_hist, causal=causal)


@pytest.mark.parametrize("seed", range(N_CASES))
def test_random_prefill(gpu, seed):
    c = draw(seed)
    print(f"case {seed}: {c}", flush=True)
    n, hq, hkv, d = c["n"], c["hq"], c["hkv"], c["d"]
    q, k, v = W.prefill_inputs(n, hq, hkv, d, seed=seed)
    rows = np.arange(n) if c["causal"] else np.unique([0, n // 3, n // 2, n - 1])
    if c["n_hist"] == 0:
        got = P.run_prefill(gpu, q, k, v, causal=c["causal"])
        ref = P.oracle_rows(q, k, v, rows, causal=c["causal"])
    else:
        _, kh, vh = W.prefill_inputs(c["n_hist"], hq, hkv, d, seed=100 + seed)
        got = P.run_prefill_ctx(gpu, q, k, v, kh, vh, causal=c["causal"])
        ref = P.oracle_ctx_rows(q, k, v, kh, vh, rows, causal=c["causal"])
    P.check(got, ref, rows, str(c))


@pytest.mark.parametrize("seed", range(12))
def test_random_prefill_writes_pool(gpu, seed):
    """The prefill's own paged write over random shapes: the attention output
    is bit-identical to the same call without pools, every row of the chunk
    lands at start_pos + row through a shuffled block table (f32 exactly,
    binary16 rounded to nearest even), and the pool's other rows stay zero."""
    import oracle
    import torch

    rng = np.random.default_rng(3000 + seed)
    hkv = int(rng.choice([1, 2, 4, 8]))
    group = int(rng.choice([1, 2, 3, 4, 8, 16]))
    while hkv * group > 32:
        group //= 2
    hq = hkv * group
    d = int(rng.choice([64, 128]))
    n = int(rng.integers(1, 401))
    start = int(rng.integers(0, 300))
    bt = int(rng.choice([16, 32, 64]))
    kv_dtype = oracle.KV_F32 if seed % 2 == 0 else oracle.KV_F16
    causal = bool(rng.random() < 0.85)
    print(f"case {seed}: hq={hq} hkv={hkv} d={d} n={n} start={start} bt={bt} "
          f"dtype={kv_dtype} causal={causal}", flush=True)
    q, k, v = W.prefill_inputs(n, hq, hkv, d, seed=40 + seed)
    nb = (start + n + bt - 1) // bt + 2
    table = rng.permutation(nb).astype(np.int32)
    dt = torch.float32 if kv_dtype == oracle.KV_F32 else torch.int16
    kp = torch.zeros((nb, hkv, bt, d), dtype=dt, device="cuda")
    vp = torch.zeros_like(kp)
    plain = P.run_prefill(gpu, q, k, v, causal=causal)
    got = P.run_prefill(gpu, q, k, v, causal=causal, k_pool=kp, v_pool=vp,
                        block_table=torch.from_numpy(table).cuda(), block_tokens=bt,
                        kv_dtype=kv_dtype, start_pos=start)
    assert np.array_equal(got, plain), "output differs with the pool write"
    t = np.arange(start, start + n)
    kpn, vpn = kp.cpu().numpy(), vp.cpu().numpy()
    kb, vb = W.bf16_round(k), W.bf16_round(v)
    if kv_dtype == oracle.KV_F32:
        want_k, want_v = kb, vb
    else:
        want_k = kb.astype(np.float16).view(np.int16)
        want_v = vb.astype(np.float16).view(np.int16)
    assert np.array_equal(kpn[table[t // bt], :, t % bt], want_k), "K rows"
    assert np.array_equal(vpn[table[t // bt], :, t % bt], want_v), "V rows"
    written = np.zeros((nb, bt), bool)
    written[table[t // bt], t % bt] = True
    # pools are [block][kv head][token][dim]: look at [block][token] across heads
    kt_, vt_ = kpn.transpose(0, 2, 1, 3), vpn.transpose(0, 2, 1, 3)
    assert not np.any(kt_[~written]) and not np.any(vt_[~written]), "rows outside the chunk"
