"""The HMA arena's contract (swamp-tensors/src/hma.rs:215-260) through the C
ABI, on the host region, which needs no device: first-fit allocation with
256-byte granularity, free-list coalescing, alloc after free, reset, stats,
out-of-memory with a message, copy bounds, and -- on a host without a GPU --
the reference's fallback of device requests to host memory (hma.rs:249-256).
"""
import os

import pytest

import nyion_hip as nh

HP, DL, UM = nh.MEM_HOST_PINNED, nh.MEM_DEVICE_LOCAL, nh.MEM_UNIFIED_MAPPED


@pytest.fixture
def hma():
    h = nh.Hma(0, 64 * 1024)
    yield h
    h.close()


def test_first_fit_and_coalescing(hma):
    a = hma.alloc(1000, HP)   # rounded to 1024
    b = hma.alloc(256, HP)
    c = hma.alloc(5000, HP)   # rounded to 5120
    assert (b.ptr - a.ptr, c.ptr - b.ptr) == (1024, 256)
    assert a.ptr % 256 == 0 and hma.stats(HP) == (1024 + 256 + 5120, 64 * 1024)
    assert hma.free(b) == nh.OK
    # a 256-byte hole: a 512-byte request skips it, a 256-byte one takes it
    d = hma.alloc(512, HP)
    assert d.ptr == c.ptr + 5120
    e = hma.alloc(1, HP)
    assert e.ptr == b.ptr
    assert hma.free(e) == nh.OK and hma.free(a) == nh.OK
    # a and the hole after it merged: 1280 bytes fit at a's address
    f = hma.alloc(1280, HP)
    assert f.ptr == a.ptr
    for x in (f, c, d):
        assert hma.free(x) == nh.OK
    # everything merged back into one range: the whole region fits again
    g = hma.alloc(64 * 1024, HP)
    assert g.ptr == a.ptr and hma.stats(HP)[0] == 64 * 1024


def test_out_of_memory_reports_a_message(hma):
    a = hma.alloc(60 * 1024, HP)
    rc, _ = hma.try_alloc(8 * 1024, HP)
    assert rc == nh.ERR_OOM and "exhausted" in nh.last_error()
    assert hma.free(a) == nh.OK
    rc, b = hma.try_alloc(8 * 1024, HP)
    assert rc == nh.OK


def test_double_free_and_foreign_pointers_are_rejected(hma):
    a = hma.alloc(300, HP)
    assert hma.free(a) == nh.OK
    assert hma.free(a) == nh.ERR_INVALID and "not a live allocation" in nh.last_error()
    b = hma.alloc(512, HP)
    inner = nh.Allocation(b.ptr + 256, 256, HP, 0, 0)
    assert hma.free(inner) == nh.ERR_INVALID


def test_reset_frees_everything(hma):
    for _ in range(10):
        hma.alloc(4096, HP)
    assert hma.stats(HP)[0] == 40960
    assert hma.reset() == nh.OK
    assert hma.stats(HP)[0] == 0
    assert hma.alloc(64 * 1024, HP).ptr != 0


def test_upload_download_round_trip_and_bounds(hma):
    a = hma.alloc(1000, HP)
    data = os.urandom(1000)
    assert hma.upload(a, data) == nh.OK
    rc, back = hma.download(a, 1000)
    assert rc == nh.OK and back == data
    assert hma.upload(a, os.urandom(1001)) == nh.ERR_INVALID  # beyond the allocation
    assert hma.free(a) == nh.OK
    assert hma.upload(a, data) == nh.ERR_INVALID  # no longer live


def test_device_requests_without_a_device_fall_back_to_host():
    h = nh.Hma(1 << 20, 64 * 1024)
    try:
        if h.has_device:
            pytest.skip("a device is present: the fallback applies to hosts without one")
        for loc in (DL, UM):
            a = h.alloc(4096, loc)
            # served by the host region, as the reference's host.allocate (hma.rs:254)
            assert a.location == HP and a.device_handle == 0 and a.ptr != 0
            data = os.urandom(4096)
            assert h.upload(a, data) == nh.OK and h.download(a, 4096) == (nh.OK, data)
        assert h.stats(HP)[0] == 8192 and h.stats(DL) == (0, 0)
    finally:
        h.close()


def test_bad_location_and_null_handle():
    h = nh.Hma(0, 4096)
    rc, _ = h.try_alloc(16, 7)
    assert rc == nh.ERR_INVALID
    h.close()
    L = nh.load()
    assert L.nyion_hma_alloc(None, 16, HP, None) == nh.ERR_INVALID
    assert L.nyion_hma_reset(None) == nh.ERR_INVALID
