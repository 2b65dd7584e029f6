"""swamp-kernels C-ABI on the GPU: mojo_softmax_padic and mojo_stokes_* (gpu).

The Q16.16 softmax is integer arithmetic around one expf per element; its
exp_q16_16 takes one of 655360 negative inputs, and the library holds those
values in a per-device table filled with the host C library's expf (what the
reference's f32::exp and the oracle call).  Outputs therefore equal the
oracle's bit for bit on every input.
"""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def gpu_softmax(gpu, x, t):
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros_like(x)
    gpu.load().mojo_softmax_padic(x.ctypes.data, out.ctypes.data, len(x), float(t))
    return out


def test_softmax_padic_exact_cases(gpu):
    for x, t in [([0.0, 0.0], 1.0), (np.zeros(16), 1.0), (np.r_[100.0, np.zeros(15)], 1.0),
                 ([100.0, 0.0], 1.0), ([1e-7, 0.0], 0.0), ([np.nan, 0.0], 1.0),
                 ([1, 2, 3, .5, -1, 4, 2.5, 1.5], 1.0)]:
        assert np.array_equal(gpu_softmax(gpu, x, t), oracle.softmax_padic(x, t)), x


def test_softmax_padic_vocab(gpu):
    rng = np.random.default_rng(0)
    for n, t in [(32000, 1.0), (50000, 0.7), (17, 2.0), (4096, 1.0)]:
        x = (rng.standard_normal(n) * 3).astype(np.float32)
        got = gpu_softmax(gpu, x, t)
        assert np.array_equal(got, oracle.softmax_padic(x, t)), n


def test_exp_q16_16_every_input(gpu):
    """Every input of exp_q16_16 through the softmax: logits 0 and x/65536 (T=1)
    make e_1 = exp_q16_16(x) for x in [-655360, 0]; probabilities are compared
    bit for bit with the oracle, which calls the same expf."""
    for lo in range(-655360, 1, 65536):
        xs = np.arange(lo, min(lo + 65536, 1), dtype=np.int64)
        for x in xs[::4097]:
            logits = np.array([0.0, x / 65536.0], np.float32)
            assert np.array_equal(gpu_softmax(gpu, logits, 1.0), oracle.softmax_padic(logits, 1.0)), x
    # and a whole vocabulary whose differences sweep the table densely
    x = (-np.arange(700000) / 65536.0).astype(np.float32)
    assert np.array_equal(gpu_softmax(gpu, x, 1.0), oracle.softmax_padic(x, 1.0))


def test_softmax_padic_staging_sizes_and_threads(gpu):
    """Arrays up to 2^20 go through the library's staging array (back-to-back
    calls of different sizes reuse it; two host threads take turns), longer
    ones through memory allocated for the call."""
    import threading
    rng = np.random.default_rng(1)
    cases = [((rng.standard_normal(n) * 3).astype(np.float32), t)
             for n, t in [(1 << 20, 1.0), (300, 0.5), ((1 << 20) + 5000, 1.3), (70000, 1.0)]]
    for x, t in cases:
        assert np.array_equal(gpu_softmax(gpu, x, t), oracle.softmax_padic(x, t)), len(x)
    results = {}

    def worker(k):
        x, t = cases[k % 2 * 3]  # the 2^20 case and the 70000 case, from two threads
        results[k] = [gpu_softmax(gpu, x, t) for _ in range(3)]

    ths = [threading.Thread(target=worker, args=(k,)) for k in range(2)]
    for th in ths:
        th.start()
    for th in ths:
        th.join()
    for k in range(2):
        x, t = cases[k % 2 * 3]
        ref = gpu_softmax(gpu, x, t)
        assert all(np.array_equal(r, ref) for r in results[k])


def test_softmax_padic_device_entry(gpu):
    x = torch.randn(1000, device="cuda") * 2
    p = torch.empty_like(x)
    gpu.softmax_padic_dev(x, p, 1.0)
    torch.cuda.synchronize()
    ref = oracle.softmax_padic(x.cpu().numpy(), 1.0)
    assert np.array_equal(p.cpu().numpy(), ref)


def test_stokes_matches_oracle(gpu):
    L = gpu.load()
    O = oracle.lib()
    hd = 8
    c = L.mojo_stokes_init(hd)
    o = O.orc_stokes_init(hd)
    assert c
    rng = np.random.default_rng(1)
    scores = rng.standard_normal(4200).astype(np.float32)
    scores[4150] = scores[:4150].min()  # a tie with an earlier minimum
    for i in range(4200):
        kv = np.full(hd, i, np.float32)
        L.mojo_stokes_append(c, i, kv.ctypes.data, kv.ctypes.data, float(scores[i]))
        O.orc_stokes_append(o, i, kv.ctypes.data, kv.ctypes.data, float(scores[i]))
    n = L.nyion_stokes_count(c)
    assert n == O.orc_stokes_count(o) == 4096
    kg, vg, sg = (np.zeros((n, hd), np.float32), np.zeros((n, hd), np.float32),
                  np.zeros(n, np.float32))
    ko, vo, so = np.zeros_like(kg), np.zeros_like(vg), np.zeros_like(sg)
    assert L.nyion_stokes_read(c, kg.ctypes.data, vg.ctypes.data, sg.ctypes.data) == n
    O.orc_stokes_read(o, ko.ctypes.data, vo.ctypes.data, so.ctypes.data)
    assert np.array_equal(kg, ko) and np.array_equal(vg, vo) and np.array_equal(sg, so)
    L.mojo_stokes_free(c)
    O.orc_stokes_free(o)
    # null handles return silently, as the reference's extern "C" functions do
    L.mojo_stokes_append(None, 0, None, None, 0.0)
    L.mojo_stokes_free(None)
    L.mojo_softmax_padic(None, None, 0, 1.0)
    _ = C
