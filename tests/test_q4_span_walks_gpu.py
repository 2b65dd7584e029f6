"""Q4-20B decode on contiguous walks against the oracle (gpu).

Paged decode over 16-token blocks (ops::attention / ops::attention_sparse,
swamp-engine/src/ops.rs:170-278, 85-168) on Q4-20B rows at head_dim 64: the
walk loads each tile's 16 K rows and 16 V rows as two spans and, untracked,
consumes tiles in pairs from a ring of four, so a wavefront's walk length
(odd or even, shorter than the ring, ending in a partial tile) decides which
slots hold which tile.  The partition size (tiles per workgroup, four
wavefronts each, a power of two of tokens) with context lengths and q
positions that cut segments unevenly sweeps those lengths: at 64 tokens per
workgroup every wavefront has at most one tile; at 256 a 1337-token
sequence's 84 tiles go to six workgroups of 14, i.e. wavefronts of 3 and 4
tiles; at 4096 one workgroup takes a whole segment.  Tolerance as for
every attention output: max-abs-err <= 2e-3 and max|diff| / max|ref| <=
1e-3; the tracked form's importance as in test_decode_gpu.  The Attention
node's contiguous 4-bit layout is held to the same bar.
"""
import numpy as np
import pytest
import torch

import oracle
import workloads as W
from test_decode_gpu import assert_close, run_tracked

pytestmark = pytest.mark.gpu

CTX = [1, 15, 17, 250, 1000, 1337]
Q_POS = [0, 7, 16, 100, 999, 640]


def to_dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def decode(gpu, pb, window=0, stride=0, q_pos=None):
    out = torch.full((pb.batch, pb.n_heads, pb.head_dim), float("nan"), device="cuda")
    gpu.paged_decode(to_dev(pb.q), to_dev(pb.k_pool), to_dev(pb.v_pool), to_dev(pb.tables),
                     to_dev(pb.ctx_lens), out, pb.n_heads, pb.n_kv_heads, pb.head_dim,
                     pb.block_tokens, kv_dtype=pb.kv_dtype, window=window, global_stride=stride,
                     max_ctx=int(pb.ctx_lens.max()),
                     q_pos=None if q_pos is None else to_dev(np.asarray(q_pos, np.int32)))
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("tokens", [64, 128, 256, 512, 1024, 4096])
def test_q4_span_walk_lengths(gpu, tokens):
    pb = W.paged_batch(CTX, n_heads=32, n_kv_heads=4, head_dim=64, block_tokens=16, seed=tokens,
                       kv_dtype=oracle.KV_Q4)
    try:
        gpu.set_partition_tokens(tokens)
        full = decode(gpu, pb)
        qpos = decode(gpu, pb, q_pos=Q_POS)
        win = decode(gpu, pb, window=40, stride=0)
        glob = decode(gpu, pb, window=200, stride=16)
    finally:
        gpu.set_partition_tokens(0)
    assert_close(full, W.reference_decode(pb), f"{tokens} tokens: full")
    assert_close(qpos, W.reference_decode(pb, q_pos=Q_POS), f"{tokens} tokens: q_pos")
    assert_close(win, W.reference_decode(pb, window=40), f"{tokens} tokens: window 40")
    assert_close(glob, W.reference_decode(pb, window=200, global_stride=16),
                 f"{tokens} tokens: window 200, globals every 16")


@pytest.mark.parametrize("tokens", [64, 256])
def test_q4_span_walk_tracked(gpu, tokens):
    """The tracked form walks single span tiles: outputs and importance
    against the oracle at the same walk lengths."""
    pb = W.paged_batch(CTX, n_heads=32, n_kv_heads=4, head_dim=64, block_tokens=16, seed=5 + tokens,
                       kv_dtype=oracle.KV_Q4)
    try:
        gpu.set_partition_tokens(tokens)
        out, imp = run_tracked(gpu, pb, q_pos=Q_POS)
    finally:
        gpu.set_partition_tokens(0)
    assert_close(out, W.reference_decode(pb, q_pos=Q_POS), f"{tokens} tokens: tracked out")
    for b in range(pb.batch):
        L = int(pb.ctx_lens[b])
        _, ref_imp = oracle.attention(pb.q[b].reshape(-1), pb.layout(b), L, Q_POS[b], pb.n_heads,
                                      pb.n_kv_heads, pb.head_dim, importance=True)
        W.assert_importance(imp[b][:L], ref_imp, f"{tokens} tokens: importance b={b}")


@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("seq_len", [1, 17, 128, 1000])
def test_q4_attention_node(gpu, head_dim, seq_len):
    """The Attention node on Q4-20B rows laid out [Hkv][kv_stride][row]
    (compute_graph.rs:14-25 with the 4-bit cache): no block table, so a span
    walk's tile offsets come from the row positions alone (head_dim 64;
    head_dim 128 walks per-row tiles), with and without the scores buffer
    (whole segments, or split-K pieces merged through it)."""
    rng = np.random.default_rng(seq_len + head_dim)
    hq, hkv, stride = 32, 4, seq_len + 24
    q = rng.standard_normal((hq, head_dim), dtype=np.float32)
    k = oracle.q4_quantize_rows(rng.standard_normal((hkv, stride, head_dim), dtype=np.float32))
    v = oracle.q4_quantize_rows(rng.standard_normal((hkv, stride, head_dim), dtype=np.float32))
    ref = oracle.attention(q.reshape(-1), oracle.contiguous_layout(k, v, stride, head_dim, oracle.KV_Q4),
                           seq_len, seq_len - 1, hq, hkv, head_dim).reshape(hq, head_dim)
    dq, dk, dv = to_dev(q), to_dev(k), to_dev(v)
    out = torch.full_like(dq, float("nan"))
    gpu.attention_node(dq, dk, dv, out, hq, hkv, seq_len, head_dim, stride, kv_dtype=oracle.KV_Q4)
    scores = torch.empty(hq * seq_len, device="cuda")
    split = torch.full_like(dq, float("nan"))
    gpu.attention_node(dq, dk, dv, split, hq, hkv, seq_len, head_dim, stride, kv_dtype=oracle.KV_Q4,
                       scores=scores)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), ref, f"q4 node, {seq_len} positions")
    assert_close(split.cpu().numpy(), ref, f"q4 node with scores buffer, {seq_len} positions")
