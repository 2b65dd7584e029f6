"""The Mojo FFI symbol sparse_attention_q4 (swamp-gpu/src/mojo.rs:5,38;
swamp-gpu/kernels/attention.mojo:38-152) against the oracle's restatement
(gpu).  Tolerance: rel <= 1e-5 of max|ref|, abs <= 1e-6 — the two sides
compute the same operations in the same order, and differ only by the
device's and the host's expf."""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def check(got, ref):
    err = np.max(np.abs(got.astype(np.float64) - ref))
    assert err <= max(1e-6, 1e-5 * np.max(np.abs(ref))), err


@pytest.mark.parametrize("hd,n_heads,n_sparse", [(64, 4, 40), (64, 2, 64), (64, 3, 65), (128, 2, 300),
                                                 (96, 1, 200), (40, 2, 130)])
def test_sparse_attention_q4_matches_oracle(gpu, hd, n_heads, n_sparse):
    rng = np.random.default_rng(hd * 1000 + n_sparse)
    n_rows = 500
    kq = oracle.mojo_q4_rows(rng.standard_normal((n_rows, hd)).astype(np.float32))
    vq = oracle.mojo_q4_rows(rng.standard_normal((n_rows, hd)).astype(np.float32))
    q = (rng.standard_normal((n_heads, hd)) * 2).astype(np.float32)
    pos = rng.integers(0, n_rows, n_sparse).astype(np.int32)  # repeats allowed, as in the list
    got = gpu.sparse_attention_q4(q, kq, vq, pos, n_heads, hd, window=4096, global_stride=64)
    check(got, oracle.mojo_sparse_attention_q4(q, kq, vq, pos, n_heads, hd))


def test_sparse_attention_q4_skip_and_empty(gpu):
    hd = 32
    k = np.zeros((2, 20), np.float32)
    k[0, 0], k[0, 2:18] = 0.25, 255.0
    v = np.zeros((2, 20), np.float32)
    v[0, 0], v[0, 2:18] = 1.0 / 15.0, 255.0
    v[1, 0], v[1, 2:18] = 60000.0, 255.0
    q = np.ones((1, hd), np.float32)
    got = gpu.sparse_attention_q4(q, k, v, np.array([0, 1], np.int32), 1, hd)
    assert np.array_equal(got, oracle.mojo_sparse_attention_q4(q, k, v, np.array([0, 1], np.int32), 1, hd))
    empty = gpu.sparse_attention_q4(q, k, v, np.zeros(0, np.int32), 1, hd)
    assert np.all(empty == 0.0)


def test_sparse_attention_q4_rejects_negative_position(gpu):
    hd = 32
    k = np.zeros((2, 20), np.float32)
    q = np.ones((1, hd), np.float32)
    with pytest.raises(gpu.NyionError):
        gpu.sparse_attention_q4(q, k, k, np.array([0, -1], np.int32), 1, hd)


def test_sparse_attention_q4_staging_sizes_and_threads(gpu):
    """Calls whose arrays fit the library's 16 MiB staging array reuse it
    (back to back, and from two host threads taking turns); a call whose K/V
    rows up to the largest position do not fit (60000 rows of head_dim 64:
    19.2 MB) runs on memory allocated for the call."""
    import threading
    hd = 64

    def case(n_rows, n_sparse, n_heads, seed):
        rng = np.random.default_rng(seed)
        kq = oracle.mojo_q4_rows(rng.standard_normal((n_rows, hd)).astype(np.float32))
        vq = oracle.mojo_q4_rows(rng.standard_normal((n_rows, hd)).astype(np.float32))
        q = rng.standard_normal((n_heads, hd)).astype(np.float32)
        pos = rng.integers(0, n_rows, n_sparse).astype(np.int32)
        pos[-1] = n_rows - 1  # the copy reaches the last row
        return q, kq, vq, pos, n_heads

    cases = [case(60000, 100, 2, 1), case(20000, 300, 4, 2), case(64, 10, 1, 3)]
    for q, kq, vq, pos, nh in cases:
        got = gpu.sparse_attention_q4(q, kq, vq, pos, nh, hd)
        check(got, oracle.mojo_sparse_attention_q4(q, kq, vq, pos, nh, hd))
    results = {}

    def worker(k):
        q, kq, vq, pos, nh = cases[1 + k]
        results[k] = [gpu.sparse_attention_q4(q, kq, vq, pos, nh, hd) for _ in range(3)]

    ths = [threading.Thread(target=worker, args=(k,)) for k in range(2)]
    for th in ths:
        th.start()
    for th in ths:
        th.join()
    for k in range(2):
        q, kq, vq, pos, nh = cases[1 + k]
        ref = gpu.sparse_attention_q4(q, kq, vq, pos, nh, hd)
        assert all(np.array_equal(r, ref) for r in results[k])
