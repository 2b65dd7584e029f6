"""Paged KV writes, Q4-20B codec and block-table gathers on the GPU (gpu).

Integer and byte work is checked bit-exactly against the oracle."""
import numpy as np
import pytest
import torch

import oracle
import workloads as W

pytestmark = pytest.mark.gpu


def to_dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def edge_rows(rng):
    parts = [rng.standard_normal((500000, 64), dtype=np.float32),     # 1e6 groups
             (rng.standard_normal((4000, 64)) * 1e-6).astype(np.float32),  # subnormal f16 d
             (rng.standard_normal((4000, 64)) * 3e4).astype(np.float32),
             (rng.standard_normal((1000, 64)) * 1e5).astype(np.float32),   # f16 overflow
             (rng.standard_normal((500, 64)) * 1e-12).astype(np.float32),  # d below 1e-10
             np.zeros((16, 64), np.float32), np.full((16, 64), -0.0, np.float32),
             np.full((16, 64), 7.5, np.float32)]
    x = np.concatenate(parts)
    x[-40, 5] = np.nan         # f32::max/min skip NaN
    x[-41, :] = np.nan
    x[-42, 9] = np.inf
    return x


def test_q4_quantize_bit_exact(gpu):
    x = edge_rows(np.random.default_rng(0))
    ref = oracle.q4_quantize_rows(x)
    out = torch.zeros(ref.shape, dtype=torch.uint8, device="cuda")
    gpu.q4_quantize(to_dev(x), x.shape[0], 64, out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    bad = np.nonzero(np.any(got != ref, axis=1))[0]
    assert bad.size == 0, f"{bad.size} rows differ, first {bad[:5]}: {got[bad[0]]} vs {ref[bad[0]]}"


@pytest.mark.parametrize("hd,shift", [(128, 0), (96, 0), (64, 1), (80, 0)])
def test_q4_quantize_paths(gpu, hd, shift):
    """The eight-lane quantiser (head_dim a multiple of 32, 16-byte aligned
    rows) and the per-group one (a partial group, or rows one float off the
    16-byte boundary) write the same bytes as the oracle."""
    rng = np.random.default_rng(hd + shift)
    x = (rng.standard_normal((3001, hd)) * rng.choice([1e-3, 1.0, 50.0], size=(3001, 1))).astype(np.float32)
    x[7, :] = 0.0
    x[8, 3] = np.nan
    ref = oracle.q4_quantize_rows(x)
    buf = torch.zeros(x.size + 4, dtype=torch.float32, device="cuda")
    buf[shift:shift + x.size] = torch.from_numpy(x.reshape(-1)).cuda()
    out = torch.zeros(ref.shape, dtype=torch.uint8, device="cuda")
    gpu.q4_quantize(buf[shift:], x.shape[0], hd, out)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), ref)


def test_q4_dequant_bit_exact(gpu):
    rng = np.random.default_rng(1)
    x = edge_rows(rng)
    b = oracle.q4_quantize_rows(x)
    # also every header bit pattern of d and dmin (incl. subnormal, inf, NaN)
    hdr = np.zeros((65536, 40), np.uint8)
    hdr[:, 0:2] = np.arange(65536, dtype=np.uint16).view(np.uint8).reshape(-1, 2)
    hdr[:, 2:4] = np.roll(np.arange(65536, dtype=np.uint16), 12345).view(np.uint8).reshape(-1, 2)
    hdr[:, 4:20] = rng.integers(0, 256, size=(65536, 16), dtype=np.uint8)
    hdr[:, 20:] = hdr[:, :20]
    b = np.concatenate([b, hdr])
    ref = oracle.q4_dequant_rows(b, 64)
    out = torch.zeros(ref.shape, dtype=torch.float32, device="cuda")
    gpu.q4_dequant(to_dev(b), b.shape[0], 64, out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


@pytest.mark.parametrize("kv_dtype", [oracle.KV_F32, oracle.KV_Q4])
def test_kv_write_and_gather(gpu, kv_dtype):
    """save_at of a prefill chunk into shuffled 16-token blocks, read back
    through the decode kernels' row addressing (nyion_kv_gather)."""
    rng = np.random.default_rng(2)
    n, hkv, hd, bt, start = 1000, 4, 64, 16, 37
    total_blocks = 80
    table = rng.permutation(total_blocks).astype(np.int32)
    k = rng.standard_normal((n, hkv, hd), dtype=np.float32)
    v = rng.standard_normal((n, hkv, hd), dtype=np.float32)
    rb = hd if kv_dtype == oracle.KV_F32 else oracle.q4_row_bytes(hd)
    dt = torch.float32 if kv_dtype == oracle.KV_F32 else torch.uint8
    kp = torch.zeros((total_blocks, hkv, bt, rb), dtype=dt, device="cuda")
    vp = torch.zeros_like(kp)
    dtab = to_dev(table)
    gpu.kv_write(kp, vp, dtab, bt, hkv, hd, kv_dtype, start, to_dev(k), to_dev(v))
    torch.cuda.synchronize()
    # host-side expectation: the same rows at (table[t/bt], t%bt)
    t = np.arange(start, start + n)
    kh, vh = kp.cpu().numpy(), vp.cpu().numpy()
    if kv_dtype == oracle.KV_F32:
        assert np.array_equal(kh[table[t // bt], :, t % bt], k)
        assert np.array_equal(vh[table[t // bt], :, t % bt], v)
    else:
        assert np.array_equal(kh[table[t // bt], :, t % bt], oracle.q4_quantize_rows(k))
        assert np.array_equal(vh[table[t // bt], :, t % bt], oracle.q4_quantize_rows(v))
    # untouched slots before start stay zero
    assert not kh[table[0], :, :start % bt].any() if start < bt else True
    # gather through the kernels' RowMap
    ntok = start + n
    out = torch.zeros((hkv, ntok, hd), dtype=torch.float32, device="cuda")
    gpu.kv_gather(kp, dtab, bt, hkv, hd, kv_dtype, ntok, out)
    torch.cuda.synchronize()
    g = out.cpu().numpy()[:, start:]
    expect = k if kv_dtype == oracle.KV_F32 else oracle.q4_dequant_rows(oracle.q4_quantize_rows(k), hd)
    assert np.array_equal(g.transpose(1, 0, 2), expect)


def test_kv_append_batch(gpu):
    rng = np.random.default_rng(3)
    B, hkv, hd, bt = 5, 4, 64, 16
    pos = np.array([0, 15, 16, 100, 511], np.int32)
    tables = rng.permutation(B * 32).astype(np.int32).reshape(B, 32)
    k = rng.standard_normal((B, hkv, hd), dtype=np.float32)
    v = rng.standard_normal((B, hkv, hd), dtype=np.float32)
    for kv_dtype in (oracle.KV_F32, oracle.KV_Q4):
        rb = hd if kv_dtype == oracle.KV_F32 else oracle.q4_row_bytes(hd)
        dt = torch.float32 if kv_dtype == oracle.KV_F32 else torch.uint8
        kp = torch.zeros((B * 32, hkv, bt, rb), dtype=dt, device="cuda")
        vp = torch.zeros_like(kp)
        gpu.kv_append_batch(kp, vp, to_dev(tables), to_dev(pos), bt, hkv, hd, kv_dtype, to_dev(k),
                            to_dev(v))
        torch.cuda.synchronize()
        kh = kp.cpu().numpy()
        for b in range(B):
            row = kh[tables[b, pos[b] // bt], :, pos[b] % bt]
            exp = k[b] if kv_dtype == oracle.KV_F32 else oracle.q4_quantize_rows(k[b])
            assert np.array_equal(row, exp)


def test_paged_gather_matches_table_arithmetic(gpu):
    """Block-table indexing is bit-exact: gather == host fancy-index of the pool."""
    pb = W.paged_batch([777], seed=4)
    out = torch.zeros((4, 777, 64), dtype=torch.float32, device="cuda")
    gpu.kv_gather(to_dev(pb.k_pool), to_dev(pb.tables[0]), 16, 4, 64, oracle.KV_F32, 777, out)
    torch.cuda.synchronize()
    t = np.arange(777)
    exp = pb.k_pool[pb.tables[0][t // 16], :, t % 16].transpose(1, 0, 2)
    assert np.array_equal(out.cpu().numpy(), exp)


@pytest.mark.parametrize("hd", [64, 128])
def test_rope_kv_append_bit_exact(gpu, hd):
    """Decode-step epilogue: RoPE on q and k (apply_rope_ufc) and the save of
    the rotated k and of v, against the oracle's table and rotation,
    bit-exactly (f32 products rounded before the add on both sides); a
    position past max_ctx uses the table's last row."""
    rng = np.random.default_rng(6)
    B, hq, hkv, bt, max_ctx = 5, 16, 4, 16, 600
    pos = np.array([0, 15, 16, 599, 700], np.int32)
    tables = rng.permutation(B * 64).astype(np.int32).reshape(B, 64)
    q = rng.standard_normal((B, hq, hd), dtype=np.float32)
    k = rng.standard_normal((B, hkv, hd), dtype=np.float32)
    v = rng.standard_normal((B, hkv, hd), dtype=np.float32)
    lut_ref = oracle.rope_lut(hd, max_ctx)
    lut = gpu.rope_lut(hd, max_ctx)
    assert np.array_equal(lut.cpu().numpy().view(np.uint32), lut_ref.view(np.uint32))
    for kv_dtype in (oracle.KV_F32, oracle.KV_Q4):
        rb = hd if kv_dtype == oracle.KV_F32 else oracle.q4_row_bytes(hd)
        dt = torch.float32 if kv_dtype == oracle.KV_F32 else torch.uint8
        kp = torch.zeros((B * 64, hkv, bt, rb), dtype=dt, device="cuda")
        vp = torch.zeros_like(kp)
        dq = to_dev(q)
        gpu.rope_kv_append(dq, to_dev(k), to_dev(v), lut, to_dev(pos), kp, vp, to_dev(tables),
                           hq, hkv, hd, bt, kv_dtype)
        torch.cuda.synchronize()
        got_q, kh, vh = dq.cpu().numpy(), kp.cpu().numpy(), vp.cpu().numpy()
        for b in range(B):
            rq, rk = oracle.apply_rope(q[b], k[b], int(pos[b]), max_ctx, lut_ref)
            assert np.array_equal(got_q[b].view(np.uint32), rq.view(np.uint32)), f"q b={b}"
            krow = kh[tables[b, pos[b] // bt], :, pos[b] % bt]
            vrow = vh[tables[b, pos[b] // bt], :, pos[b] % bt]
            if kv_dtype == oracle.KV_F32:
                assert np.array_equal(krow.view(np.uint32), rk.view(np.uint32)), f"k b={b}"
                assert np.array_equal(vrow, v[b])
            else:
                assert np.array_equal(krow, oracle.q4_quantize_rows(rk)), f"k q4 b={b}"
                assert np.array_equal(vrow, oracle.q4_quantize_rows(v[b]))
