"""Seeded random sweep of the k-quant GEMVs against the oracle (gpu).

Each case draws the format (Q4_K, swamp-kernels/src/fused_gemv_q4k.rs:
395-448, or Q6_K, fused_gemv_q6k.rs:248-293), 1..5000 rows, 1..64 blocks of
256 columns (every rows-per-unit and wavefronts-per-row variant the launch
picks from) and 1..5 inputs through the batched entry point; every input's
output is checked against the oracle at max-abs-err <= 2e-3 and max|diff| /
max|ref| <= 1e-3, and the padding past n_rows stays untouched."""
import numpy as np
import pytest
import torch

import oracle
import workloads as W

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-3
N_CASES = 24


def draw(seed):
    rng = np.random.default_rng(3000 + seed)
    fmt = "q4k" if seed % 2 == 0 else "q6k"
    n_rows = int(rng.choice([int(rng.integers(1, 65)), int(rng.integers(65, 5001))]))
    n_cols = 256 * int(rng.choice([int(rng.integers(1, 9)), int(rng.integers(9, 65))]))
    batch = int(rng.integers(1, 6))
    return dict(fmt=fmt, n_rows=n_rows, n_cols=n_cols, batch=batch)


@pytest.mark.parametrize("seed", range(N_CASES))
def test_random_gemv(gpu, seed):
    c = draw(seed)
    print(f"case {seed}: {c}", flush=True)
    n_rows, n_cols, batch = c["n_rows"], c["n_cols"], c["batch"]
    if c["fmt"] == "q4k":
        w = W.q4k_random_weights(n_rows, n_cols, seed=seed)
        run, ref_fn = gpu.gemv_q4k_batched, oracle.gemv_q4k
    else:
        w = W.q6k_random_weights(n_rows, n_cols, seed=seed)
        run, ref_fn = gpu.gemv_q6k_batched, oracle.gemv_q6k
    xs = np.random.default_rng(seed).standard_normal((batch, n_cols + 8)).astype(np.float32)
    out = torch.full((batch, n_rows + 5), float("nan"), device="cuda")
    run(torch.from_numpy(w).cuda(), torch.from_numpy(xs).cuda(), out, n_rows, n_cols)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.isnan(got[:, n_rows:]).all(), f"{c}: stride padding written"
    for b in range(batch):
        ref = ref_fn(w, np.ascontiguousarray(xs[b, :n_cols]), n_rows, n_cols).astype(np.float64)
        g = got[b, :n_rows].astype(np.float64)
        assert np.all(np.isfinite(g)), c
        err = np.max(np.abs(g - ref))
        rel = err / max(np.max(np.abs(ref)), 1e-30)
        assert err <= ATOL and rel <= RTOL, f"{c} input {b}: max-abs {err:.3e} rel {rel:.3e}"
