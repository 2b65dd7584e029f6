"""Q6_K weight GEMV and mixed Q4_K / Q6_K GEMV lists on the GPU against the
oracle (gpu).

The oracle is the scalar path of swamp-kernels/src/fused_gemv_q6k.rs
(248-293) restated in C, with the reference's own f16 conversion of d.  The
kernel sums in another order, so outputs agree to tolerance: max-abs-err
<= 2e-3 and rel-err (max|diff| / max|ref|) <= 1e-3.  Batched calls and
spec lists must equal the single call bit for bit (same per-row arithmetic).
"""
import ctypes as C

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


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def dev_at(a, offset):
    """a copied to device memory `offset` bytes past a 256-byte aligned base."""
    flat = np.ascontiguousarray(a).reshape(-1)
    buf = torch.zeros(flat.size + offset, dtype=torch.uint8, device="cuda")
    buf[offset:] = torch.from_numpy(flat).cuda()
    return buf[offset:]


# TinyLlama-1.1B Q6_K tensors (output 32000x2048, v 256x2048, down 2048x5632),
# one-block rows (every other block starts 2 bytes past a dword), odd block
# counts, ragged row counts for both rows-per-wavefront paths
SHAPES = [(1, 256), (3, 256), (7, 768), (256, 2048), (2048, 5632), (32000, 2048),
          (4097, 256), (4099, 768), (33, 2816)]


@pytest.mark.parametrize("n_rows,n_cols", SHAPES)
def test_gemv_q6k_vs_oracle(gpu, n_rows, n_cols):
    w = W.q6k_random_weights(n_rows, n_cols, seed=n_rows + n_cols)
    x = np.random.default_rng(n_cols).standard_normal(n_cols).astype(np.float32)
    out = torch.full((n_rows,), float("nan"), device="cuda")
    gpu.gemv_q6k(dev(w), dev(x), out, n_rows, n_cols)
    torch.cuda.synchronize()
    check(out.cpu().numpy(), oracle.gemv_q6k(w, x, n_rows, n_cols), f"gemv {n_rows}x{n_cols}")


@pytest.mark.parametrize("offset", [2, 6, 14])
@pytest.mark.parametrize("n_rows,n_cols", [(5, 256), (9, 1280), (300, 2048)])
def test_gemv_q6k_weights_off_dword(gpu, n_rows, n_cols, offset):
    """W 2 bytes past a dword boundary: the blocks that were dword aligned are
    not and the others are."""
    w = W.q6k_random_weights(n_rows, n_cols, seed=offset)
    x = np.random.default_rng(offset).standard_normal(n_cols).astype(np.float32)
    out = torch.full((n_rows,), float("nan"), device="cuda")
    gpu.gemv_q6k(dev_at(w, offset), dev(x), out, n_rows, n_cols)
    torch.cuda.synchronize()
    check(out.cpu().numpy(), oracle.gemv_q6k(w, x, n_rows, n_cols), f"offset {offset}")


@pytest.mark.parametrize("n_rows,n_cols", [(37, 16640), (9, 32768)])
def test_gemv_q6k_long_rows(gpu, n_rows, n_cols):
    """Rows longer than eight wavefronts' single pass (16384 columns)."""
    w = W.q6k_random_weights(n_rows, n_cols, seed=n_cols)
    x = np.random.default_rng(n_rows).standard_normal(n_cols).astype(np.float32)
    out = torch.full((n_rows,), float("nan"), device="cuda")
    gpu.gemv_q6k(dev(w), dev(x), out, n_rows, n_cols)
    torch.cuda.synchronize()
    check(out.cpu().numpy(), oracle.gemv_q6k(w, x, n_rows, n_cols), f"gemv {n_rows}x{n_cols}")


def test_gemv_q6k_reference_test_weights(gpu):
    """The reference tests' blocks and input (fused_gemv_q6k.rs:329-376).
    Their outputs reach 3.7e4, where one f32 step is 4e-3, so this case takes
    the reference test's own bound (diff < 1 or diff / max(|ref|, 1) < 1e-4,
    fused_gemv_q6k.rs:372-374), tightened to diff / max(|ref|, 1) < 1e-5."""
    for n_rows, n_blocks in ((1, 1), (4, 3), (7, 2)):
        n_cols = 256 * n_blocks
        w = W.q6k_reference_test_weights(n_rows, n_blocks)
        x = np.sin(np.arange(n_cols, dtype=np.float32) * np.float32(0.01)).astype(np.float32)
        out = torch.empty(n_rows, device="cuda")
        gpu.gemv_q6k(dev(w), dev(x), out, n_rows, n_cols)
        torch.cuda.synchronize()
        got = out.cpu().numpy().astype(np.float64)
        ref = oracle.gemv_q6k(w, x, n_rows, n_cols).astype(np.float64)
        rel = np.abs(got - ref) / np.maximum(np.abs(ref), 1.0)
        assert np.all(rel < 1e-5), (n_rows, n_blocks, got, ref)


def test_gemv_q6k_reference_scale_conversion(gpu):
    """d with exponent 31 (0x7c00, 0xfc01) converts as the reference does
    (65536 and -65600), not to inf/NaN."""
    n_rows, n_cols = 2, 512
    w = W.q6k_random_weights(n_rows, n_cols, seed=5).reshape(-1, 210)
    w[:, 192:208] = 1
    w[0, 208:210] = np.array([0x7C00], np.uint16).view(np.uint8)
    w[3, 208:210] = np.array([0xFC01], np.uint16).view(np.uint8)
    w = w.reshape(n_rows, -1)
    x = (np.random.default_rng(6).standard_normal(n_cols) * 1e-6).astype(np.float32)
    out = torch.empty(n_rows, device="cuda")
    gpu.gemv_q6k(dev(w), dev(x), out, n_rows, n_cols)
    torch.cuda.synchronize()
    ref = oracle.gemv_q6k(w, x, n_rows, n_cols)
    assert oracle.q6k_scale_to_f32(0x7C00) == 65536.0
    check(out.cpu().numpy(), ref, "exponent-31 d")


@pytest.mark.parametrize("batch", [1, 2, 3, 5, 8])
def test_gemv_q6k_batched_equals_single(gpu, batch):
    n_rows, n_cols = 640, 1792
    w = dev(W.q6k_random_weights(n_rows, n_cols, seed=batch))
    xs = torch.from_numpy(np.random.default_rng(batch).standard_normal((batch, n_cols + 4))
                          .astype(np.float32)).cuda()
    out = torch.full((batch, n_rows + 3), float("nan"), device="cuda")
    gpu.gemv_q6k_batched(w, xs, out, n_rows, n_cols)
    torch.cuda.synchronize()
    for b in range(batch):
        single = torch.empty(n_rows, device="cuda")
        gpu.gemv_q6k(w, xs[b].contiguous(), single, n_rows, n_cols)
        torch.cuda.synchronize()
        assert torch.equal(out[b, :n_rows], single), b
    assert torch.isnan(out[:, n_rows:]).all()  # stride padding untouched
    check(out[0, :n_rows].cpu().numpy(),
          oracle.gemv_q6k(w.cpu().numpy(), xs[0, :n_cols].cpu().numpy(), n_rows, n_cols), "batched")


def test_gemv_specs_mixed_layer(gpu):
    """A Q4_K_M layer: q/k/o/gate/up Q4_K, v/down Q6_K (forward_gemvs,
    linear.rs:379-432), two inputs, an empty spec; every output equals its
    single call bit for bit."""
    d, kv, ff = 2048, 256, 5632
    rng = np.random.default_rng(21)
    x1 = dev(rng.standard_normal(d).astype(np.float32))
    x2 = dev(rng.standard_normal(ff).astype(np.float32))
    mats = [  # (format, rows, cols, x)
        (144, d, d, x1), (144, kv, d, x1), (210, kv, d, x1), (144, ff, d, x1), (144, ff, d, x1),
        (210, d, ff, x2), (144, d, ff, x2), (144, d, d, x1), (210, 0, d, x1)]
    specs, expect = [], []
    for i, (bb, r, c, x) in enumerate(mats):
        gen = W.q4k_random_weights if bb == 144 else W.q6k_random_weights
        w = dev(gen(max(r, 1), c, seed=100 + i))
        out = torch.full((max(r, 1),), float("nan"), device="cuda")
        specs.append((w, x, out, r, c, bb))
        single = torch.empty(max(r, 1), device="cuda")
        if r:
            (gpu.gemv_q4k if bb == 144 else gpu.gemv_q6k)(w, x, single, r, c)
        expect.append(single)
    gpu.gemv_specs(specs)
    torch.cuda.synchronize()
    for i, ((w, x, out, r, c, bb), single) in enumerate(zip(specs, expect)):
        if r == 0:
            assert torch.isnan(out).all(), "empty spec written"
            continue
        assert torch.equal(out, single), i
        ref = (oracle.gemv_q4k if bb == 144 else oracle.gemv_q6k)(w.cpu().numpy(), x.cpu().numpy(), r, c)
        check(out.cpu().numpy(), ref, f"spec {i}")


def test_gemv_q6k_rejects_bad_arguments(gpu):
    w = torch.zeros(210 * 4, dtype=torch.uint8, device="cuda")
    x = torch.zeros(512, device="cuda")
    out = torch.full((2,), 7.0, device="cuda")
    L = gpu.load()
    assert L.nyion_gemv_q6k(w.data_ptr(), x.data_ptr(), out.data_ptr(), 1, 300, None) != 0
    assert "multiple of 256" in gpu.last_error()
    assert L.nyion_gemv_q6k(w.data_ptr() + 1, x.data_ptr(), out.data_ptr(), 1, 256, None) != 0
    # a bad spec anywhere in the list launches nothing
    specs = (gpu.GemvSpec * 2)(gpu.GemvSpec(w.data_ptr(), x.data_ptr(), out.data_ptr(), 2, 512, 210, 0),
                               gpu.GemvSpec(w.data_ptr(), x.data_ptr(), out.data_ptr(), 1, 256, 200, 0))
    assert L.nyion_gemv_specs(specs, 2, None) != 0
    assert "block_bytes" in gpu.last_error()
    # so does a misaligned spec after a valid group
    specs = (gpu.GemvSpec * 2)(gpu.GemvSpec(w.data_ptr(), x.data_ptr(), out.data_ptr(), 2, 512, 210, 0),
                               gpu.GemvSpec(w.data_ptr(), x.data_ptr() + 4, out.data_ptr(), 1, 256, 144, 0))
    assert L.nyion_gemv_specs(specs, 2, None) != 0
    assert "aligned" in gpu.last_error()
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), torch.full((2,), 7.0))
    assert L.nyion_gemv_specs(None, 0, None) == 0
    assert L.nyion_gemv_specs(None, 1, None) != 0
