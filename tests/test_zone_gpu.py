"""Reference-shaped zone caches on the GPU (gpu).

Pools laid out as PagedKVCache's zone pages (32/128/1024-token pages by
position zone, every layer in one page; swamp-engine/src/cache.rs:20-21,
185-237, 593-611, 700-747) with pages placed in shuffled order.  Expected
rows come from the oracle's zone arithmetic (orc_zone_page_id,
orc_zone_f32_offset, orc_zone_q4_offset), which is pinned to the
reference's golden page ids.  Gathers and writes are byte-exact; decode
uses the tolerance of the other decode tests (max-abs <= 2e-3, rel <= 1e-3).
"""
import numpy as np
import pytest
import torch

import oracle
import workloads as W
from test_decode_gpu import assert_close

pytestmark = pytest.mark.gpu

DTYPES = [oracle.KV_F32, oracle.KV_Q4, oracle.KV_F16]


def to_dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def as_f32(raw, kv_dtype, head_dim):
    """Raw rows [..][row] -> f32 values [..][head_dim] (oracle decode of the format)."""
    if kv_dtype == oracle.KV_Q4:
        shp = raw.shape[:-1]
        return oracle.q4_dequant_rows(raw.reshape(-1, raw.shape[-1]), head_dim).reshape(shp + (head_dim,))
    if kv_dtype == oracle.KV_F16:
        return raw.view(np.float16).astype(np.float32)
    return raw


def page_positions(p):
    first = W.zone_page_first_position(p)
    return first, first + oracle.lib().orc_zone_block_size(first)


def gather(gpu, zp, pool, layer, n):
    out = torch.full((zp.n_kv_heads, n, zp.head_dim), float("nan"), device="cuda")
    gpu.zone_kv_gather(to_dev(pool), to_dev(zp.page_base), zp.n_layers, layer, zp.n_kv_heads,
                       zp.head_dim, zp.kv_dtype, n, out)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def check_rows(got, expect, valid):
    """Bit-exact on valid rows, NaN elsewhere."""
    assert np.all(np.isnan(got[~valid])), "rows of absent pages must read as NaN"
    g, e = got[valid], expect[valid]
    nan = np.isnan(e)
    assert np.array_equal(np.isnan(g), nan)
    assert np.array_equal(g[~nan].view(np.uint32), e[~nan].view(np.uint32))


@pytest.mark.parametrize("kv_dtype", DTYPES)
def test_zone_gather_across_4096(gpu, kv_dtype):
    """Tokens [0, 4400) of layer 2 of a 3-layer pool; page 10 absent, page 130
    misaligned by one unit (both read as absent)."""
    n, layer = 4400, 2
    zp = W.zone_pool(n, n_layers=3, n_kv_heads=2, head_dim=64, kv_dtype=kv_dtype, seed=1)
    off = W.zone_row_offsets(zp, layer, n)
    zp.page_base[10] = -1
    zp.page_base[130] += 1
    valid = np.ones(n, bool)
    for p in (10, 130):
        a, b = page_positions(p)
        valid[a:b] = False
    for pool in (zp.k_pool, zp.v_pool):
        got = gather(gpu, zp, pool, layer, n)
        expect = as_f32(W.zone_rows(pool, off, zp.row), kv_dtype, zp.head_dim)
        check_rows(got, expect, np.broadcast_to(valid, (zp.n_kv_heads, n)))


@pytest.mark.parametrize("kv_dtype", [oracle.KV_F32, oracle.KV_Q4])
def test_zone_gather_across_131072(gpu, kv_dtype):
    """Only the pages of [130500, 132300) and pages 0 and 200 exist."""
    n, layer = 132300, 1
    L = oracle.lib()
    present = {0, 200} | {int(L.orc_zone_page_id(t, 1 << 40)) for t in range(130500, n)}
    zp = W.zone_pool(n, n_layers=2, n_kv_heads=1, head_dim=64, kv_dtype=kv_dtype, seed=2,
                     present=present)
    off = W.zone_row_offsets(zp, layer, n)
    valid = off[0] >= 0
    assert valid[131071] and valid[131072] and valid[0] and not valid[100]
    got = gather(gpu, zp, zp.k_pool, layer, n)
    expect = as_f32(W.zone_rows(zp.k_pool, off, zp.row), kv_dtype, zp.head_dim)
    check_rows(got, expect, valid[None, :])


@pytest.mark.parametrize("kv_dtype", DTYPES)
@pytest.mark.parametrize("span", [(3900, 500), (130950, 300)])
def test_zone_write_bit_exact(gpu, kv_dtype, span):
    """save_at of one layer over a zone boundary; one page of the span is
    absent and must stay untouched, as must every byte outside the rows."""
    start, n = span
    layer, hkv, hd = 1, 2, 64
    L = oracle.lib()
    big = 1 << 40
    present = {int(L.orc_zone_page_id(t, big)) for t in range(start - 200, start + n + 200)}
    zp = W.zone_pool(start + n + 200, n_layers=2, n_kv_heads=hkv, head_dim=hd, kv_dtype=kv_dtype,
                     seed=4, present=present)
    hole = int(L.orc_zone_page_id(start + n // 2, big))
    zp.page_base[hole] = -1
    rng = np.random.default_rng(5)
    k = (rng.standard_normal((n, hkv, hd)) * 3).astype(np.float32)
    v = (rng.standard_normal((n, hkv, hd)) * 3).astype(np.float32)
    kd, vd = to_dev(zp.k_pool), to_dev(zp.v_pool)
    gpu.zone_kv_write(kd, vd, to_dev(zp.page_base), zp.n_layers, layer, hkv, hd, kv_dtype, start,
                      to_dev(k), to_dev(v))
    torch.cuda.synchronize()
    off = W.zone_row_offsets(zp, layer, start + n)[:, start:]
    for pool, src, got in ((zp.k_pool, k, kd), (zp.v_pool, v, vd)):
        expect = pool.copy()
        rows = np.transpose(src, (1, 0, 2))  # [Hkv][n][D]
        if kv_dtype == oracle.KV_Q4:
            rows = oracle.q4_quantize_rows(rows.reshape(-1, hd)).reshape(hkv, n, -1)
        elif kv_dtype == oracle.KV_F16:
            rows = rows.astype(np.float16).view(np.uint16)
        ok = off >= 0
        assert not ok.all()  # the hole is inside the span
        expect[off[ok][:, None] + np.arange(zp.row)] = rows[ok]
        assert np.array_equal(got.cpu().numpy(), expect)


def zone_batch(ctx_lens, n_layers, hkv, hd, kv_dtype, seed, present=None):
    """One shared pool holding each sequence's own pages: [B][n_pages] bases."""
    pools = [W.zone_pool(int(c), n_layers=n_layers, n_kv_heads=hkv, head_dim=hd,
                         kv_dtype=kv_dtype, seed=seed + i,
                         present=None if present is None else present[i])
             for i, c in enumerate(ctx_lens)]
    n_pages = max(len(z.page_base) for z in pools)
    bases = np.full((len(pools), n_pages), -1, np.int64)
    ks, vs, at = [], [], 0
    for i, z in enumerate(pools):
        nb = len(z.page_base)
        bases[i, :nb] = np.where(z.page_base >= 0, z.page_base + at, -1)
        ks.append(z.k_pool)
        vs.append(z.v_pool)
        at += z.k_pool.size
    return pools, np.concatenate(ks), np.concatenate(vs), bases


def run_zone_decode(gpu, q, k, v, bases, n_layers, layer, ctx, hkv, kv_dtype, **kw):
    qd = to_dev(q)
    out = torch.full_like(qd, float("nan"))
    gpu.zone_decode(qd, to_dev(k), to_dev(v), to_dev(bases), n_layers, layer,
                    to_dev(np.asarray(ctx, np.int32)), out, q.shape[1], hkv, q.shape[2],
                    kv_dtype=kv_dtype, **kw)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def expected_decode(q, zp, layer, n, q_pos, positions=None):
    off = W.zone_row_offsets(zp, layer, n)
    kc = W.zone_rows(zp.k_pool, off, zp.row)
    vc = W.zone_rows(zp.v_pool, off, zp.row)
    lay = oracle.contiguous_layout(kc, vc, n, zp.head_dim, zp.kv_dtype)
    hq = q.shape[0]
    if positions is None:
        return oracle.attention(q, lay, n, q_pos, hq, zp.n_kv_heads, zp.head_dim).reshape(hq, -1)
    return oracle.attention_positions(q, lay, positions, hq, zp.n_kv_heads,
                                      zp.head_dim).reshape(hq, -1)


@pytest.mark.parametrize("kv_dtype,hd", [(oracle.KV_F32, 64), (oracle.KV_Q4, 64),
                                         (oracle.KV_F16, 64), (oracle.KV_F32, 128),
                                         (oracle.KV_Q4, 128), (oracle.KV_F16, 128)])
def test_zone_decode_full(gpu, kv_dtype, hd):
    ctx = [4100, 4500, 700]
    hq, hkv, n_layers, layer = 16, 2, 3, 1
    pools, k, v, bases = zone_batch(ctx, n_layers, hkv, hd, kv_dtype, seed=10)
    rng = np.random.default_rng(11)
    q = rng.standard_normal((len(ctx), hq, hd)).astype(np.float32)
    q_pos = np.array([4099, 4200, 699], np.int32)
    got = run_zone_decode(gpu, q, k, v, bases, n_layers, layer, ctx, hkv, kv_dtype,
                          q_pos=to_dev(q_pos))
    for b, zp in enumerate(pools):
        assert_close(got[b], expected_decode(q[b], zp, layer, ctx[b], int(q_pos[b])),
                     f"zone decode seq {b}")


@pytest.mark.parametrize("kv_dtype", [oracle.KV_F32, oracle.KV_Q4])
def test_zone_decode_window_across_131072(gpu, kv_dtype):
    """attention_sparse over a 132200-token zone cache: globals every 1024
    tokens in zones 0 and 1, the window across 131072; only the attended pages
    exist."""
    n, window, stride = 132200, 2048, 1024
    hq, hkv, n_layers, layer = 16, 2, 2, 1
    pos = oracle.sparse_positions(n, n - 1, window, stride)
    L = oracle.lib()
    present = {int(L.orc_zone_page_id(int(t), 1 << 40)) for t in pos}
    pools, k, v, bases = zone_batch([n], n_layers, hkv, 64, kv_dtype, seed=20, present=[present])
    q = np.random.default_rng(21).standard_normal((1, hq, 64)).astype(np.float32)
    got = run_zone_decode(gpu, q, k, v, bases, n_layers, layer, [n], hkv, kv_dtype,
                          window=window, global_stride=stride)
    assert_close(got[0], expected_decode(q[0], pools[0], layer, n, n - 1, positions=pos),
                 "zone window decode")


def test_zone_decode_full_across_131072(gpu):
    n = 131500
    hq, hkv, n_layers, layer = 8, 1, 2, 1
    pools, k, v, bases = zone_batch([n], n_layers, hkv, 64, oracle.KV_F32, seed=30)
    q = np.random.default_rng(31).standard_normal((1, hq, 64)).astype(np.float32)
    got = run_zone_decode(gpu, q, k, v, bases, n_layers, layer, [n], hkv, oracle.KV_F32)
    assert_close(got[0], expected_decode(q[0], pools[0], layer, n, n - 1), "zone decode 131500")


def test_zone_decode_skips_absent_pages(gpu):
    """A page marked absent contributes nothing: the softmax runs over the
    present positions only."""
    n, hq, hkv, n_layers = 600, 8, 2, 2
    pools, k, v, bases = zone_batch([n], n_layers, hkv, 64, oracle.KV_F32, seed=40)
    bases[0, 5] = -1
    q = np.random.default_rng(41).standard_normal((1, hq, 64)).astype(np.float32)
    got = run_zone_decode(gpu, q, k, v, bases, n_layers, 0, [n], hkv, oracle.KV_F32)
    keep = np.array([t for t in range(n) if not 160 <= t < 192], np.int32)
    assert_close(got[0], expected_decode(q[0], pools[0], 0, n, n - 1, positions=keep),
                 "absent page")


def test_zone_decode_all_pages_absent_is_zero(gpu):
    """Every page absent: every tile is masked (its loads read the pool's
    first rows) and the output is zero, as for a sequence with nothing to
    attend."""
    pools, k, v, bases = zone_batch([700], 1, 2, 64, oracle.KV_F32, seed=60)
    bases[:] = -1
    q = np.random.default_rng(61).standard_normal((1, 8, 64)).astype(np.float32)
    got = run_zone_decode(gpu, q, k, v, bases, 1, 0, [700], 2, oracle.KV_F32)
    assert np.all(got == 0.0)


def test_zone_decode_rejects_short_table(gpu):
    pools, k, v, bases = zone_batch([4200], 1, 1, 64, oracle.KV_F32, seed=50)
    q = np.zeros((1, 8, 64), np.float32)
    with pytest.raises(gpu.NyionError):
        run_zone_decode(gpu, q, k, v, bases[:, :100], 1, 0, [4200], 1, oracle.KV_F32,
                        max_ctx=4200)


def test_zone_write_rejects_rows_past_the_table(gpu):
    """A write whose last row lies on a page past the page table is refused
    before anything is written (rows are never dropped silently)."""
    zp = W.zone_pool(4400, n_layers=1, n_kv_heads=1, head_dim=64, kv_dtype=oracle.KV_F32, seed=51)
    k = to_dev(np.ones((200, 1, 64), np.float32))
    kd, vd = to_dev(zp.k_pool), to_dev(zp.v_pool)
    # rows 4100..4299: the last is on page 128 + (4299 - 4096) // 128 = 129
    with pytest.raises(gpu.NyionError):
        gpu.zone_kv_write(kd, vd, to_dev(zp.page_base[:129]), 1, 0, 1, 64, oracle.KV_F32, 4100,
                          k, k)
    assert "page 129" in gpu.last_error()
    gpu.zone_kv_write(kd, vd, to_dev(zp.page_base[:130]), 1, 0, 1, 64, oracle.KV_F32, 4100, k, k)
    torch.cuda.synchronize()
    assert not np.array_equal(kd.cpu().numpy(), zp.k_pool)
