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
