"""nyion_paged_decode_attention_noalloc, the decode entry point that
allocates nothing, against nyion_paged_decode_attention with a caller
workspace, through the C ABI (gpu).  Two calls in a row, the second with a
smaller input whose counters fall where the first call left partials: each
output equals the workspace entry point's bit for bit (same plan, same
kernels) and the oracle within max-abs-err <= 2e-3, rel-err <= 1e-3."""
import numpy as np
import pytest
import torch

import nyion_hip as nh
import oracle
import workloads as W
from test_decode_gpu import assert_close, to_dev

pytestmark = pytest.mark.gpu


def noalloc(pb, q, kp, vp, tab, ctx, out, window=0, global_stride=0):
    return nh.load().nyion_paged_decode_attention_noalloc(
        q.data_ptr(), kp.data_ptr(), vp.data_ptr(), tab.data_ptr(), tab.shape[1], ctx.data_ptr(),
        None, q.shape[0], pb.n_heads, pb.n_kv_heads, pb.head_dim, pb.block_tokens, kp.shape[0],
        pb.kv_dtype, window, global_stride, int(pb.ctx_lens.max()), 0.0, out.data_ptr(),
        torch.cuda.current_stream().cuda_stream)


CASES = [  # (lens, head_dim, kv_dtype, window, global_stride, seed): the second is smaller
    ([9000, 20000, 4096, 17, 12345, 30000], 128, oracle.KV_F32, 0, 0, 1),
    ([3000, 700], 64, oracle.KV_F32, 0, 0, 2),
]


def test_noalloc_equals_workspace_entry_point_twice(gpu):
    for lens, d, kvt, window, gs, seed in CASES:
        pb = W.paged_batch(lens, head_dim=d, kv_dtype=kvt, seed=seed)
        q, kp, vp = to_dev(pb.q), to_dev(pb.k_pool), to_dev(pb.v_pool)
        tab, ctx = to_dev(pb.tables), to_dev(pb.ctx_lens)
        need = nh.decode_workspace_size(len(lens), 32, 4, d, int(pb.ctx_lens.max()), window, gs)
        assert 0 < need <= nh.load().nyion_paged_decode_workspace_size(
            len(lens), 32, 4, d, int(pb.ctx_lens.max()), window, gs)
        want = torch.full_like(q, float("nan"))
        gpu.paged_decode(q, kp, vp, tab, ctx, want, 32, 4, d, 16, kv_dtype=kvt, window=window,
                         global_stride=gs)
        got = torch.full_like(q, float("nan"))
        rc = noalloc(pb, q, kp, vp, tab, ctx, got, window, gs)
        assert rc == nh.OK, nh.last_error()
        torch.cuda.synchronize()
        assert torch.equal(got, want), (lens, d)
        ref = W.reference_decode(pb, window=window, global_stride=gs, threads=8)
        assert_close(got.cpu().numpy(), ref, f"no-allocation decode {lens}")


def test_noalloc_rejects_a_workspace_beyond_its_scratch(gpu):
    """2048 sequences of up to 32768 tokens at head_dim 128 need more split-K
    workspace than the 32 MiB scratch: refused before any launch."""
    B, d, maxc = 2048, 128, 32768
    need = nh.decode_workspace_size(B, 32, 4, d, maxc)
    assert need > (32 << 20)
    q = torch.zeros((B, 32, d), device="cuda")
    out = torch.zeros_like(q)
    tab = torch.zeros((B, maxc // 16), dtype=torch.int32, device="cuda")
    ctx = torch.full((B,), maxc, dtype=torch.int32, device="cuda")
    kp = torch.zeros((1, 4, 16, d), device="cuda")
    rc = nh.load().nyion_paged_decode_attention_noalloc(
        q.data_ptr(), kp.data_ptr(), kp.data_ptr(), tab.data_ptr(), tab.shape[1], ctx.data_ptr(),
        None, B, 32, 4, d, 16, 1, nh.KV_F32, 0, 0, maxc, 0.0, out.data_ptr(), None)
    assert rc == nh.ERR_WORKSPACE and "scratch holds" in nh.last_error()
    torch.cuda.synchronize()
    assert torch.count_nonzero(out) == 0  # nothing ran
