"""attention_sparse_q4 on the GPU against the oracle (gpu).

ops::attention_sparse_q4 (swamp-engine/src/ops.rs:597-723) over zone pools
of Q4-20B rows (PagedKVCache's 32/128/1024-token pages holding every layer,
cache.rs:20-21, 185-237, 726-747), pages placed in shuffled order.  The
expected output is the oracle's orc_attention_sparse_q4 on the same rows
gathered through the oracle's golden-pinned zone arithmetic.  Tolerance as
for every attention output: max-abs-err <= 2e-3 and max|diff| / max|ref| <=
1e-3.
"""
import numpy as np
import pytest
import torch

import oracle
import workloads as W
from test_decode_gpu import assert_close
from test_zone_gpu import zone_batch

pytestmark = pytest.mark.gpu


def to_dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def run(gpu, q, k, v, bases, n_layers, layer, ctx, hkv, window, stride, q_pos=None, **kw):
    qd = to_dev(q)
    out = torch.full_like(qd, float("nan"))
    gpu.attention_sparse_q4(qd, to_dev(k), to_dev(v), to_dev(bases), n_layers, layer,
                            to_dev(np.asarray(ctx, np.int32)), out, q.shape[1], hkv, q.shape[2],
                            window, stride,
                            q_pos=None if q_pos is None else to_dev(np.asarray(q_pos, np.int32)),
                            **kw)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def expected(q, zp, layer, n, q_pos, window, stride):
    off = W.zone_row_offsets(zp, layer, n)
    kc = W.zone_rows(zp.k_pool, off, zp.row)
    vc = W.zone_rows(zp.v_pool, off, zp.row)
    lay = oracle.contiguous_layout(kc, vc, n, zp.head_dim, oracle.KV_Q4)
    hq = q.shape[0]
    return oracle.attention_sparse_q4(q, lay, n, q_pos, hq, zp.n_kv_heads, zp.head_dim, window,
                                      stride, threads=oracle.max_threads()).reshape(hq, -1)


@pytest.mark.parametrize("hd,hq,hkv,window,stride", [
    (64, 32, 4, 1024, 64),    # TinyLlama heads, window + globals across 4096
    (64, 16, 2, 300, 0),      # no globals
    (128, 32, 1, 600, 37),    # 32 q heads on one kv head, D=128
    (128, 8, 8, 5000, 16),    # window longer than every context: all positions
    (64, 40, 2, 700, 50),     # 20 q heads per kv head (two heads per thread, the second partial)
    (128, 12, 2, 2000, 0),    # 6 q heads per kv head at D=128
    (64, 12, 4, 3000, 9),     # 3 q heads per kv head (position ranges split five ways)
])
def test_sparse_q4_across_4096(gpu, hd, hq, hkv, window, stride):
    ctx = [4100, 4500, 700, 1]
    q_pos = [4099, 4300, 650, 0]
    n_layers, layer = 3, 2
    pools, k, v, bases = zone_batch(ctx, n_layers, hkv, hd, oracle.KV_Q4, seed=hd + window)
    q = np.random.default_rng(window).standard_normal((len(ctx), hq, hd)).astype(np.float32)
    got = run(gpu, q, k, v, bases, n_layers, layer, ctx, hkv, window, stride, q_pos=q_pos)
    for b, zp in enumerate(pools):
        assert_close(got[b], expected(q[b], zp, layer, ctx[b], q_pos[b], window, stride),
                     f"sparse q4 seq {b}")


def test_sparse_q4_window_across_131072(gpu):
    """The configuration's window shape on one sequence: ctx 132200, window
    4096 across the 131072 zone boundary, globals every 1000 (the cap of
    128); only the attended pages exist."""
    n, window, stride = 132200, 4096, 1000
    hq, hkv, n_layers, layer = 32, 4, 2, 1
    pos = oracle.sparse_positions(n, n - 1, window, stride)
    assert len(pos) == window + 128
    L = oracle.lib()
    present = {int(L.orc_zone_page_id(int(t), 1 << 40)) for t in pos}
    pools, k, v, bases = zone_batch([n], n_layers, hkv, 64, oracle.KV_Q4, seed=70,
                                    present=[present])
    q = np.random.default_rng(71).standard_normal((1, hq, 64)).astype(np.float32)
    got = run(gpu, q, k, v, bases, n_layers, layer, [n], hkv, window, stride)
    assert_close(got[0], expected(q[0], pools[0], layer, n, n - 1, window, stride),
                 "sparse q4 across 131072")


def test_sparse_q4_globals_only_and_single_position(gpu):
    """window 0: valid_end > 0 attends the globals alone; q_pos 0 attends
    position 0 alone, whose V row (read in the A5 order) is the output."""
    ctx = [3000, 3000]
    q_pos = [2999, 0]
    pools, k, v, bases = zone_batch(ctx, 1, 2, 64, oracle.KV_Q4, seed=72)
    q = np.random.default_rng(73).standard_normal((2, 8, 64)).astype(np.float32)
    got = run(gpu, q, k, v, bases, 1, 0, ctx, 2, 0, 100, q_pos=q_pos)
    for b, zp in enumerate(pools):
        assert_close(got[b], expected(q[b], zp, 0, ctx[b], q_pos[b], 0, 100), f"seq {b}")
    zp = pools[1]
    off = W.zone_row_offsets(zp, 0, 1)
    for h in range(8):
        vrow = oracle.q4_a5_row(zp.v_pool[off[h // 4, 0]:off[h // 4, 0] + zp.row], 64)
        assert np.array_equal(got[1, h], vrow)


def test_sparse_q4_differs_from_writer_order(gpu):
    """The same pools through the window decode of the writer's order
    (nyion_zone_decode_attention, A3 semantics over dequant_block rows) give
    another result: the nibble order is what is being matched."""
    ctx = [2000]
    pools, k, v, bases = zone_batch(ctx, 1, 2, 64, oracle.KV_Q4, seed=74)
    q = np.random.default_rng(75).standard_normal((1, 16, 64)).astype(np.float32)
    a5 = run(gpu, q, k, v, bases, 1, 0, ctx, 2, 512, 64)
    qd = to_dev(q)
    a3 = torch.full_like(qd, float("nan"))
    gpu.zone_decode(qd, to_dev(k), to_dev(v), to_dev(bases), 1, 0, to_dev(np.asarray(ctx, np.int32)),
                    a3, 16, 2, 64, kv_dtype=oracle.KV_Q4, window=512, global_stride=64)
    torch.cuda.synchronize()
    assert np.max(np.abs(a5 - a3.cpu().numpy())) > 1e-2


def test_sparse_q4_rejects_short_workspace(gpu):
    pools, k, v, bases = zone_batch([700], 1, 1, 64, oracle.KV_Q4, seed=76)
    q = np.zeros((1, 8, 64), np.float32)
    with pytest.raises(gpu.NyionError):
        run(gpu, q, k, v, bases, 1, 0, [700], 1, 512, 0,
            workspace=torch.empty(256, dtype=torch.uint8, device="cuda"))


@pytest.mark.parametrize("seed", range(16))
def test_sparse_q4_random(gpu, seed):
    """Seeded random configurations: head_dim 64 or 128, 1-8 kv heads and
    1-16 q heads per kv head, batches of 1-4 sequences of 1-9000 tokens
    (zone pages of 32 and 128 tokens), windows of 1-5000, global strides of
    0-300, with and without q positions."""
    rng = np.random.default_rng(3000 + seed)
    hd = int(rng.choice([64, 128]))
    hkv = int(rng.choice([1, 2, 4, 8]))
    hq = hkv * int(rng.choice([1, 2, 3, 4, 8, 16]))
    ctx = [int(x) for x in rng.integers(1, 9001, size=int(rng.integers(1, 5)))]
    window = int(rng.integers(1, 5001))
    stride = int(rng.choice([0, 7, 64, 300]))
    q_pos = [int(rng.integers(0, c)) for c in ctx] if rng.random() < 0.4 else None
    n_layers, layer = 2, int(rng.integers(0, 2))
    print(f"case {seed}: hd {hd} heads {hq}/{hkv} ctx {ctx} window {window} stride {stride} "
          f"q_pos {q_pos}", flush=True)
    pools, k, v, bases = zone_batch(ctx, n_layers, hkv, hd, oracle.KV_Q4, seed=4000 + seed)
    q = rng.standard_normal((len(ctx), hq, hd)).astype(np.float32)
    got = run(gpu, q, k, v, bases, n_layers, layer, ctx, hkv, window, stride, q_pos=q_pos)
    for b, zp in enumerate(pools):
        qp = ctx[b] - 1 if q_pos is None else q_pos[b]
        assert_close(got[b], expected(q[b], zp, layer, ctx[b], qp, window, stride),
                     f"case {seed} seq {b}")
