"""Device-resident paged KV pool with a pinned-host cold tier (gpu).

Data written through the pool's block table survives eviction to the cold
tier and reload bit for bit (f32 and Q4-20B rows), the cold slot holds the
page's bytes in [layer][K|V][block] order, the table marks pages not in HBM
with -1, and decode attention over reloaded pages matches the oracle on the
original data (max-abs <= 2e-3, rel <= 1e-3)."""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle
import workloads as W

pytestmark = pytest.mark.gpu

L, HKV, D, BT = 3, 2, 64, 16


def fill_pool(gpu, pool, n_pages, kv_dtype, seed=0):
    """Writes n_pages pages of every layer through the pool, a page at a time
    (ensure, then the chunk's K/V via nyion_kv_write); returns the f32 data."""
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((L, n_pages * BT, HKV, D)).astype(np.float32)
    v = rng.standard_normal((L, n_pages * BT, HKV, D)).astype(np.float32)
    dk, dv = torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda()
    for p in range(n_pages):
        pool.ensure(p)
        for layer in range(L):
            kp, vp = pool.layer(layer)
            rc = gpu.load().nyion_kv_write(
                kp, vp, pool.table(), BT, pool.hot_blocks, HKV, D, kv_dtype, p * BT, BT,
                dk[layer, p * BT:(p + 1) * BT].data_ptr(), dv[layer, p * BT:(p + 1) * BT].data_ptr(),
                None)
            gpu.check(rc, "kv_write")
    torch.cuda.synchronize()
    return k, v


def gather(gpu, pool, layer, n_tokens, which):
    kp, vp = pool.layer(layer)
    out = torch.full((HKV, n_tokens, D), 7.0, device="cuda")
    gpu.check(gpu.load().nyion_kv_gather(kp if which == "k" else vp, pool.table(), BT, pool.hot_blocks,
                                         HKV, D, pool.kv_dtype, n_tokens, out.data_ptr(), None),
              "kv_gather")
    torch.cuda.synchronize()
    return out.cpu().numpy().transpose(1, 0, 2)  # [tokens][HKV][D]


def expected_rows(x, kv_dtype):
    if kv_dtype == oracle.KV_F32:
        return x
    if kv_dtype == oracle.KV_F16:  # written round-to-nearest-even, widened exactly
        return x.astype(np.float16).astype(np.float32)
    return oracle.q4_dequant_rows(oracle.q4_quantize_rows(x), D)


@pytest.mark.parametrize("kv_dtype", [oracle.KV_F32, oracle.KV_Q4, oracle.KV_F16])
def test_spill_and_reload_round_trip(gpu, kv_dtype):
    n_pages, hot = 13, 4
    pool = gpu.KvPool(L, HKV, D, BT, kv_dtype, hot, 16, 32)
    k, v = fill_pool(gpu, pool, n_pages, kv_dtype, seed=kv_dtype)
    st = pool.stats()
    assert st == {"hot": hot, "cold": n_pages - hot, "evictions": n_pages - hot, "reloads": 0}
    for first in (0, 3, 9):
        pool.ensure(first, first + hot - 1)
        n = (first + hot) * BT
        for layer in range(L):
            for which, src in (("k", k), ("v", v)):
                got = gather(gpu, pool, layer, n, which)
                want = expected_rows(src[layer, :n], kv_dtype)
                hot_tok = slice(first * BT, n)
                assert np.array_equal(got[hot_tok], want[hot_tok]), (first, layer, which)
                # pages outside HBM have table entry -1: the gather marks them NaN
                assert np.all(np.isnan(got[:first * BT]))
    assert pool.stats()["reloads"] > 0
    pool.close()


def test_cold_slot_holds_the_page_bytes(gpu):
    pool = gpu.KvPool(L, HKV, D, BT, oracle.KV_F32, 2, 4, 8)
    k, v = fill_pool(gpu, pool, 3, oracle.KV_F32, seed=5)  # page 0 -> slot 0
    assert pool.state(0)[:2] == (gpu.PAGE_COLD, 0)
    n = L * 2 * HKV * BT * D
    host = np.ctypeslib.as_array(C.cast(pool.cold_slot_ptr(0), C.POINTER(C.c_float)), shape=(n,))
    host = host.reshape(L, 2, HKV, BT, D)
    for layer in range(L):
        assert np.array_equal(host[layer, 0], k[layer, :BT].transpose(1, 0, 2))
        assert np.array_equal(host[layer, 1], v[layer, :BT].transpose(1, 0, 2))
    pool.close()


def test_new_pages_are_zeroed(gpu):
    """A created page is zeroed (cache.rs:279 alloc_zeroed), also in a block
    that held another page."""
    pool = gpu.KvPool(L, HKV, D, BT, oracle.KV_F32, 2, 4, 8)
    fill_pool(gpu, pool, 2, oracle.KV_F32, seed=6)
    pool.ensure(2)  # evicts a page, reuses its block
    torch.cuda.synchronize()
    got = gather(gpu, pool, 1, 3 * BT, "k")
    assert np.all(got[2 * BT:] == 0.0)
    pool.close()


def test_decode_attention_over_reloaded_pages(gpu):
    """8 pages through a 4-block hot tier, pages 0..3 brought back, then one
    decode step over the first 64 positions through the pool's table."""
    pool = gpu.KvPool(L, HKV, D, BT, oracle.KV_F32, 4, 8, 8)
    k, v = fill_pool(gpu, pool, 8, oracle.KV_F32, seed=7)
    pool.ensure(0, 3)
    ctx, hq, layer = 4 * BT, 8, 2
    q = np.random.default_rng(8).standard_normal((1, hq, D)).astype(np.float32)
    kp, vp = pool.layer(layer)
    out = torch.full((1, hq, D), float("nan"), device="cuda")
    ws_bytes = gpu.load().nyion_paged_decode_workspace_size(1, hq, HKV, D, ctx, 0, 0)
    ws = torch.zeros(max(ws_bytes, 256), dtype=torch.uint8, device="cuda")
    ctx_lens = torch.tensor([ctx], dtype=torch.int32, device="cuda")
    rc = gpu.load().nyion_paged_decode_attention(
        torch.from_numpy(q).cuda().data_ptr(), kp, vp, pool.table(), pool.max_pages,
        ctx_lens.data_ptr(), None, 1, hq, HKV, D, BT, pool.hot_blocks, oracle.KV_F32, 0, 0, ctx, 0.0,
        out.data_ptr(), ws.data_ptr(), ws.numel(), None)
    gpu.check(rc, "paged_decode")
    torch.cuda.synchronize()
    lay = oracle.token_major_layout(k[layer, :ctx], v[layer, :ctx], HKV, D)
    ref = oracle.attention(q.reshape(-1), lay, ctx, ctx - 1, hq, HKV, D).reshape(1, hq, D)
    err = np.max(np.abs(out.cpu().numpy() - ref))
    assert err <= 2e-3 and err / np.max(np.abs(ref)) <= 1e-3
    pool.close()


def test_importance_hand_off(gpu):
    """executor.rs:751-755: positions above 0.001 add to their page."""
    pool = gpu.KvPool(L, HKV, D, BT, oracle.KV_F32, 4, 4, 8)
    pool.ensure(0, 2)
    imp = np.zeros(3 * BT)
    imp[3] = 0.5
    imp[5] = 0.0005  # below the threshold
    imp[BT + 1] = 0.25
    imp[2 * BT:] = 0.01
    pool.record_importance(imp)
    assert pool.state(0)[2] == 0.5
    assert pool.state(1)[2] == 0.25
    assert abs(pool.state(2)[2] - 0.16) < 1e-12
    pool.close()
