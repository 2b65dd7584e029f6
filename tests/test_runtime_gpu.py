"""Runtime contracts on the GPU (gpu): the HMA arena with a device, the
range-status report of the reduced-precision operands, the node's use of a
scores buffer of exactly n_heads*seq_len floats, and concurrent decode
calls from two host threads on two streams.

Tolerance for attention outputs: max-abs-err <= 2e-3 and rel-err <= 1e-3
(rel-err = max|gpu - ref| / max|ref|), against the oracle.
"""
import os
import threading
import time

import numpy as np
import pytest
import torch

import nyion_hip as nh
import oracle
import workloads as W
from test_decode_gpu import assert_close, to_dev

pytestmark = pytest.mark.gpu

HP, DL, UM = nh.MEM_HOST_PINNED, nh.MEM_DEVICE_LOCAL, nh.MEM_UNIFIED_MAPPED


# ---------------------------------------------------------------- HMA arena

def test_hma_with_a_device(gpu):
    """DeviceLocal from the hipMalloc region (first fit, 256-byte aligned,
    coalescing), HostPinned from the pinned region, UnifiedMapped per
    allocation; round trips, out-of-memory, stats, reset
    (swamp-tensors/src/hma.rs:215-260)."""
    h = nh.Hma(1 << 20, 1 << 16)
    try:
        assert h.has_device
        a = h.alloc(1000, DL)
        b = h.alloc(2000, DL)
        c = h.alloc(256, DL)
        assert a.device_handle == a.ptr and a.ptr % 256 == 0 and a.location == DL
        assert (b.ptr - a.ptr, c.ptr - b.ptr) == (1024, 2048)
        data = os.urandom(2000)
        assert h.upload(b, data) == nh.OK and h.download(b, 2000) == (nh.OK, data)
        assert h.upload(b, os.urandom(2001)) == nh.ERR_INVALID
        assert h.free(a) == nh.OK and h.free(b) == nh.OK
        d = h.alloc(3072, DL)  # a and b merged
        assert d.ptr == a.ptr
        assert h.stats(DL) == (3072 + 256, 1 << 20)
        rc, _ = h.try_alloc(1 << 20, DL)
        assert rc == nh.ERR_OOM and "device arena exhausted" in nh.last_error()
        p = h.alloc(5000, HP)
        assert p.location == HP and p.device_handle == 0
        pd = os.urandom(5000)
        assert h.upload(p, pd) == nh.OK and h.download(p, 5000) == (nh.OK, pd)
        u = h.alloc(4096, UM)
        assert u.location == UM and u.device_handle == u.ptr
        ud = os.urandom(4096)
        assert h.upload(u, ud) == nh.OK and h.download(u, 4096) == (nh.OK, ud)
        assert h.stats(UM)[0] == 4096
        assert h.free(u) == nh.OK and h.stats(UM)[0] == 0
        assert h.reset() == nh.OK
        assert h.stats(DL)[0] == 0 and h.stats(HP)[0] == 0
        assert h.alloc(1 << 20, DL).ptr == a.ptr  # the whole region again
    finally:
        h.close()


# ---------------------------------------------------------------- range report

def test_prefill_reports_v_outside_binary16(gpu):
    rng = np.random.default_rng(5)
    n, hq, hkv, d = 96, 4, 1, 64
    q = torch.from_numpy(rng.standard_normal((n, hq, d), dtype=np.float32)).cuda().bfloat16()
    k = torch.from_numpy(rng.standard_normal((n, hkv, d), dtype=np.float32)).cuda().bfloat16()
    v = torch.from_numpy(rng.standard_normal((n, hkv, d), dtype=np.float32)).cuda().bfloat16()
    out = torch.empty((n, hq, d), device="cuda")
    nh.take_status()  # start clean
    gpu.prefill_bf16(q, k, v, out, hq, hkv, d)
    assert nh.take_status() == (nh.OK, "")  # in range: nothing reported
    v[40, 0, 7] = 1e5
    gpu.prefill_bf16(q, k, v, out, hq, hkv, d)
    rc, msg = nh.take_status()
    assert rc == nh.ERR_RANGE and "prefill" in msg and "65520" in msg
    assert nh.take_status() == (nh.OK, "")  # taken: cleared
    v[40, 0, 7] = 65280.0  # the largest bf16 below the binary16 overflow
    gpu.prefill_bf16(q, k, v, out, hq, hkv, d)
    assert nh.take_status() == (nh.OK, "")


@pytest.mark.parametrize("kvt", [oracle.KV_F16, oracle.KV_Q4])
def test_binary16_decode_reports_q_outside_binary16(gpu, kvt):
    """Decode over binary16 and Q4-20B pools splits q into binary16 parts."""
    pb = W.paged_batch([300, 77], kv_dtype=kvt, seed=9)
    q = to_dev(pb.q)
    kp, vp = to_dev(pb.k_pool), to_dev(pb.v_pool)
    tab, ctx = to_dev(pb.tables), to_dev(pb.ctx_lens)
    out = torch.empty_like(q)
    nh.take_status()
    gpu.paged_decode(q, kp, vp, tab, ctx, out, 32, 4, 64, 16, kv_dtype=kvt)
    assert nh.take_status() == (nh.OK, "")
    q[1, 5, 3] = -1e5
    gpu.paged_decode(q, kp, vp, tab, ctx, out, 32, 4, 64, 16, kv_dtype=kvt)
    rc, msg = nh.take_status()
    assert rc == nh.ERR_RANGE and "decode" in msg
    # f32 pools carry q as f32: nothing to report
    pf = W.paged_batch([300, 77], seed=9)
    gpu.paged_decode(q, to_dev(pf.k_pool), to_dev(pf.v_pool), tab, ctx, out, 32, 4, 64, 16)
    assert nh.take_status() == (nh.OK, "")


# ---------------------------------------------------------------- node scratch

def test_node_uses_only_n_heads_seq_len_scores(gpu):
    """A scores buffer of exactly n_heads*seq_len floats (what the CUDA path
    allocates, fused_attention.cu:206) with kv_stride = 2*seq_len: the node
    splits over it and never writes past it (a sentinel tail stays)."""
    rng = np.random.default_rng(17)
    hq, hkv, S, stride = 32, 4, 4096, 8192
    assert 0 < nh.node_scratch_bytes(hq, hkv, S, 64) <= 4 * hq * S
    q = rng.standard_normal((hq, 64), dtype=np.float32)
    k = rng.standard_normal((hkv, stride, 64), dtype=np.float32)
    v = rng.standard_normal((hkv, stride, 64), dtype=np.float32)
    ref = oracle.attention(q.reshape(-1), oracle.contiguous_layout(k, v, stride, 64), S, S - 1, hq,
                           hkv, 64, threads=8).reshape(hq, 64)
    buf = torch.full((hq * S + 65536,), 12345.0, device="cuda")
    scores = buf[: hq * S]
    out = torch.full((hq, 64), float("nan"), device="cuda")
    dq, dk, dv = to_dev(q), to_dev(k), to_dev(v)
    for _ in range(3):
        gpu.attention_node(dq, dk, dv, out, hq, hkv, S, 64, stride, scores=scores)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), ref, "node over n_heads*seq_len scores")
    assert torch.all(buf[hq * S:] == 12345.0)


# ---------------------------------------------------------------- concurrency

def test_two_threads_two_streams_two_workspaces(gpu):
    """Re-entrancy per stream: two host threads decode different batches
    concurrently on their own streams and workspaces (pools shared
    read-only) while a third changes the process-wide partition setting;
    every result equals the oracle."""
    lens = [[3000, 1200, 5000, 64], [800, 4100, 2222]]
    pb = W.paged_batch(lens[0] + lens[1], seed=23)
    refs = W.reference_decode(pb, threads=8)
    kp, vp = to_dev(pb.k_pool), to_dev(pb.v_pool)
    parts = [slice(0, 4), slice(4, 7)]
    setups = []
    for sl in parts:
        q, tab, ctx = to_dev(pb.q[sl]), to_dev(pb.tables[sl]), to_dev(pb.ctx_lens[sl])
        maxc = int(pb.ctx_lens[sl].max())
        ws = nh.alloc_workspace(nh.decode_workspace_size(q.shape[0], 32, 4, 64, maxc))
        setups.append((q, tab, ctx, maxc, ws, torch.empty_like(q), torch.cuda.Stream()))
    torch.cuda.synchronize()
    errors, stop = [], threading.Event()

    def worker(i):
        q, tab, ctx, maxc, ws, out, st = setups[i]
        try:
            for it in range(40):
                if it % 10 == 0:
                    with torch.cuda.stream(st):  # ordered before the decode on st
                        out.fill_(float("nan"))
                gpu.paged_decode(q, kp, vp, tab, ctx, out, 32, 4, 64, 16, max_ctx=maxc,
                                 workspace=ws, stream=st)
                if it % 10 == 9:
                    st.synchronize()
                    assert_close(out.cpu().numpy(), refs[parts[i]], f"thread {i} iter {it}")
        except Exception as e:  # noqa: BLE001
            errors.append(e)

    def toggler():
        k = 0
        while not stop.is_set():
            nh.set_partition_tokens((0, 64, 128, 256)[k % 4])
            k += 1
            time.sleep(0.0005)

    ts = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    tg = threading.Thread(target=toggler)
    tg.start()
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=120)
    stop.set()
    tg.join(timeout=10)
    nh.set_partition_tokens(0)
    torch.cuda.synchronize()
    assert not errors, errors
