"""Q4_K weight GEMV on the GPU against the oracle (gpu).

The oracle is the scalar path of swamp-kernels/src/fused_gemv_q4k.rs
(395-448) restated in C.  The kernel sums in another order, so outputs
agree to tolerance: max-abs-err <= 2e-3 and rel-err (max|diff| / max|ref|)
<= 1e-3.  Multi-matrix and batched calls must equal the single call bit for
bit (same per-row arithmetic).
"""
import numpy as np
import pytest
import torch

import oracle
import workloads as W

pytestmark = pytest.mark.gpu

ATOL = 2e-3
RTOL = 1e-3


def check(got, ref, what):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert np.all(np.isfinite(got)), what
    err = np.max(np.abs(got - ref))
    rel = err / max(np.max(np.abs(ref)), 1e-30)
    assert err <= ATOL and rel <= RTOL, f"{what}: max-abs {err:.3e} rel {rel:.3e}"


def dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    return t.cuda() if dtype is None else t.to(dtype).cuda()


# TinyLlama-1.1B projections (q/o 2048x2048, k/v 256x2048, gate/up 5632x2048,
# down 2048x5632), the smallest matrix and ragged row counts for both
# rows-per-wavefront paths
SHAPES = [(1, 256), (7, 512), (2048, 2048), (256, 2048), (5632, 2048), (2048, 5632),
          (4097, 256), (4099, 768)]


@pytest.mark.parametrize("n_rows,n_cols", SHAPES)
def test_gemv_q4k_vs_oracle(gpu, n_rows, n_cols):
    w = W.q4k_random_weights(n_rows, n_cols, seed=n_rows + n_cols)
    x = np.random.default_rng(n_cols).standard_normal(n_cols).astype(np.float32)
    out = torch.full((n_rows,), float("nan"), device="cuda")
    gpu.gemv_q4k(dev(w), dev(x), out, n_rows, n_cols)
    torch.cuda.synchronize()
    check(out.cpu().numpy(), oracle.gemv_q4k(w, x, n_rows, n_cols), f"gemv {n_rows}x{n_cols}")


@pytest.mark.parametrize("n_rows,n_cols", [(37, 16640), (9, 32768), (130, 20480)])
def test_gemv_q4k_long_rows(gpu, n_rows, n_cols):
    """Rows longer than eight wavefronts' single pass (16384 columns): each
    wavefront makes several passes and reloads its x values per pass."""
    w = W.q4k_random_weights(n_rows, n_cols, seed=n_cols)
    x = np.random.default_rng(n_rows).standard_normal(n_cols).astype(np.float32)
    out = torch.full((n_rows,), float("nan"), device="cuda")
    gpu.gemv_q4k(dev(w), dev(x), out, n_rows, n_cols)
    torch.cuda.synchronize()
    check(out.cpu().numpy(), oracle.gemv_q4k(w, x, n_rows, n_cols), f"gemv {n_rows}x{n_cols}")


def test_gemv_q4k_long_rows_batched_equals_single(gpu):
    n_rows, n_cols, batch = 33, 16896, 3
    w = dev(W.q4k_random_weights(n_rows, n_cols, seed=11))
    xs = torch.from_numpy(np.random.default_rng(12).standard_normal((batch, n_cols))
                          .astype(np.float32)).cuda()
    out = torch.empty((batch, n_rows), device="cuda")
    gpu.gemv_q4k_batched(w, xs, out, n_rows, n_cols)
    for b in range(batch):
        single = torch.empty(n_rows, device="cuda")
        gpu.gemv_q4k(w, xs[b].contiguous(), single, n_rows, n_cols)
        torch.cuda.synchronize()
        assert torch.equal(out[b], single), b


def test_gemv_q4k_reference_test_weights(gpu):
    """The reference tests' weights and input (fused_gemv_q4k.rs:830-845)."""
    for n_rows in (2, 3, 4, 7):
        w = W.q4k_reference_test_weights(n_rows)
        x = W.q4k_reference_test_x(256)
        out = torch.empty(n_rows, device="cuda")
        gpu.gemv_q4k(dev(w), dev(x), out, n_rows, 256)
        torch.cuda.synchronize()
        check(out.cpu().numpy(), oracle.gemv_q4k(w, x, n_rows, 256), f"reference weights {n_rows}")


def test_gemv_q4k_multi_equals_single(gpu):
    """q/k/v of one layer in one launch (2048 + 256 + 256 rows)."""
    n_cols = 2048
    rows = [2048, 256, 256]
    ws = [W.q4k_random_weights(r, n_cols, seed=i) for i, r in enumerate(rows)]
    x = dev(np.random.default_rng(3).standard_normal(n_cols).astype(np.float32))
    dws = [dev(w) for w in ws]
    outs = [torch.full((r,), float("nan"), device="cuda") for r in rows]
    gpu.gemv_q4k_multi(dws, x, outs, n_cols)
    for dw, o, r, w in zip(dws, outs, rows, ws):
        single = torch.empty(r, device="cuda")
        gpu.gemv_q4k(dw, x, single, r, n_cols)
        torch.cuda.synchronize()
        assert torch.equal(o, single)
        check(o.cpu().numpy(), oracle.gemv_q4k(w, x.cpu().numpy(), r, n_cols), "multi")


@pytest.mark.parametrize("batch", [1, 2, 3, 4, 5, 7, 9])
def test_gemv_q4k_batched_equals_single(gpu, batch):
    n_rows, n_cols = 640, 1024
    w = dev(W.q4k_random_weights(n_rows, n_cols, seed=batch))
    xs = torch.from_numpy(np.random.default_rng(batch).standard_normal((batch, n_cols + 4))
                          .astype(np.float32)).cuda()
    out = torch.full((batch, n_rows + 3), float("nan"), device="cuda")
    gpu.gemv_q4k_batched(w, xs, out, n_rows, n_cols)
    torch.cuda.synchronize()
    for b in range(batch):
        single = torch.empty(n_rows, device="cuda")
        gpu.gemv_q4k(w, xs[b].contiguous(), single, n_rows, n_cols)
        torch.cuda.synchronize()
        assert torch.equal(out[b, :n_rows], single), b
    assert torch.isnan(out[:, n_rows:]).all()  # stride padding untouched


def test_gemv_q4k_rejects_bad_shapes(gpu):
    w = torch.zeros(144 * 2, dtype=torch.uint8, device="cuda")
    x = torch.zeros(512, device="cuda")
    out = torch.zeros(2, device="cuda")
    L = gpu.load()
    assert L.nyion_gemv_q4k(w.data_ptr(), x.data_ptr(), out.data_ptr(), 1, 300, None) != 0
    assert "multiple of 256" in gpu.last_error()
    assert L.nyion_gemv_q4k(w.data_ptr() + 4, x.data_ptr(), out.data_ptr(), 1, 256, None) != 0
    import ctypes as C
    five = (C.c_void_p * 5)(*([w.data_ptr()] * 5))
    outs = (C.c_void_p * 5)(*([out.data_ptr()] * 5))
    rows = (C.c_int32 * 5)(*([1] * 5))
    assert L.nyion_gemv_q4k_multi(five, x.data_ptr(), outs, rows, 5, 256, None) != 0
