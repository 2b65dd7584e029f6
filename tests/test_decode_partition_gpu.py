"""Window-mode decode with strided globals over the direct partition (gpu).

ops::attention_sparse (swamp-engine/src/ops.rs:85-168) over a few
sequences: each (sequence, kv head) segment is cut into pieces of a fixed
number of tiles, four wavefronts to a piece, the window's contiguous tiles
first and the globals' gathered tiles after them.  The windows, lengths and
partition sizes below put the boundary between the two inside a piece at
every offset a wavefront split can take, so the piece's wave ranges are
re-cut there; the default partition (0) sizes pieces by the bytes of the KV
format.  Every KV format and head size, blocks of one, four and sixteen
tiles, against the oracle, tolerance as for every attention output: max-abs-err
<= 2e-3 and max|diff| / max|ref| <= 1e-3.
"""
import numpy as np
import pytest
import torch

import oracle
import workloads as W
from test_decode_gpu import assert_close

pytestmark = pytest.mark.gpu

CTX = [3000, 2531, 1777, 2222]
PARTITIONS = [64, 128, 256, 512, 1024, 0]


def to_dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def decode(gpu, pb, window, stride, q_pos=None):
    out = torch.full((pb.batch, pb.n_heads, pb.head_dim), float("nan"), device="cuda")
    gpu.paged_decode(to_dev(pb.q), to_dev(pb.k_pool), to_dev(pb.v_pool), to_dev(pb.tables),
                     to_dev(pb.ctx_lens), out, pb.n_heads, pb.n_kv_heads, pb.head_dim,
                     pb.block_tokens, kv_dtype=pb.kv_dtype, window=window, global_stride=stride,
                     max_ctx=int(pb.ctx_lens.max()),
                     q_pos=None if q_pos is None else to_dev(np.asarray(q_pos, np.int32)))
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("kv_dtype", [oracle.KV_F32, oracle.KV_F16, oracle.KV_Q4], ids=["f32", "f16", "q4"])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("block_tokens", [16, 64, 256])
def test_window_globals_direct_partitions(gpu, kv_dtype, head_dim, block_tokens):
    pb = W.paged_batch(CTX, n_heads=16, n_kv_heads=4, head_dim=head_dim, block_tokens=block_tokens,
                       seed=head_dim + kv_dtype + block_tokens, kv_dtype=kv_dtype)
    for window, stride in ((300, 16), (1000, 16), (1500, 7)):
        ref = W.reference_decode(pb, window=window, global_stride=stride)
        for p in PARTITIONS:
            try:
                gpu.set_partition_tokens(p)
                got = decode(gpu, pb, window, stride)
            finally:
                gpu.set_partition_tokens(0)
            assert_close(got, ref, f"window {window} stride {stride} partition {p}")


@pytest.mark.parametrize("block_tokens", [16, 64])
def test_window_walk_start_at_host_bound(gpu, block_tokens):
    """4-bit window walks request their block-table entries before the
    length arrives, assuming a sequence at the host's max_ctx with q at its
    end; sequences at max_ctx with q elsewhere, and shorter ones, take their
    own window start."""
    ctx = [3000, 3000, 3000, 1777]
    q_pos = [2999, 2000, 1234, 1776]
    pb = W.paged_batch(ctx, n_heads=16, n_kv_heads=4, head_dim=64, block_tokens=block_tokens,
                       seed=31 + block_tokens, kv_dtype=oracle.KV_Q4)
    for window, stride in ((300, 16), (1000, 0), (1500, 7)):
        ref = W.reference_decode(pb, window=window, global_stride=stride, q_pos=q_pos)
        for p in (256, 1024, 0):
            try:
                gpu.set_partition_tokens(p)
                got = decode(gpu, pb, window, stride, q_pos)
            finally:
                gpu.set_partition_tokens(0)
            assert_close(got, ref, f"window {window} stride {stride} partition {p}")
