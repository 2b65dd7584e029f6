"""The C ABI library loads and exports every symbol include/nyion_hip.h
declares; without a GPU every entry point reports NYION_ERR_NO_DEVICE
instead of computing anything (CPU only)."""
import ctypes as C
import os
import re

import nyion_hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nyion_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    text = re.sub(r"^\s*#.*$", "", text, flags=re.M)  # preprocessor lines
    names = re.findall(r"\b([A-Za-z_]\w*)\s*\(([^;{]*?)\)\s*;", text)
    return sorted({n for n, _ in names if n not in ("sizeof",)})


def test_header_parses_to_known_symbols():
    names = declared_functions()
    assert len(names) >= 30
    assert set(names) == set(nyion_hip.SIGNATURES), set(names) ^ set(nyion_hip.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = C.CDLL(nyion_hip.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_no_device_is_reported_not_faked():
    import torch

    if torch.cuda.is_available():  # only meaningful on a host without a GPU
        return
    L = nyion_hip.load()
    assert L.nyion_device_count() == 0
    assert L.nyion_init(0) == nyion_hip.ERR_NO_DEVICE
    rc = L.nyion_paged_decode_attention(None, None, None, None, 1, None, None, 1, 32, 4, 64, 16, 1,
                                        0, 0, 0, 128, 0.0, None, None, 0, None)
    assert rc == nyion_hip.ERR_NO_DEVICE and "device" in nyion_hip.last_error()
    assert L.nyion_attention_node(None, None, None, None, None, 32, 4, 128, 64, 128, 0,
                                  None) == nyion_hip.ERR_NO_DEVICE
    assert L.nyion_prefill_attention_bf16(None, None, None, 1, 1, 1, 128, 1, 0.0, None, None,
                                          None, None, 16, 0, 0, 0, None) == nyion_hip.ERR_NO_DEVICE
    assert L.nyion_prefill_attention_bf16_ctx(None, None, None, None, None, 0, 1, 1, 1, 128, 1,
                                              0.0, None, None, None, None, 16, 0, 0, 0,
                                              None) == nyion_hip.ERR_NO_DEVICE
    assert L.nyion_kv_gather_bf16(None, None, 16, 1, 1, 64, 0, 1, None,
                                  None) == nyion_hip.ERR_NO_DEVICE
    assert L.nyion_gemv_q6k(None, None, None, 1, 256, None) == nyion_hip.ERR_NO_DEVICE
    spec = nyion_hip.GemvSpec(256, 512, 1024, 1, 256, 210, 0)  # never dereferenced
    assert L.nyion_gemv_specs(C.byref(spec), 1, None) == nyion_hip.ERR_NO_DEVICE
    assert L.gpu_attention_device(None, None, None, None, 32, 4, 128, 64, 128) == -1
    assert L.mojo_stokes_init(64) is None


def test_workspace_sizes_are_host_only():
    L = nyion_hip.load()
    # 64 sequences up to 32K tokens needs split-K partials
    ws = L.nyion_paged_decode_workspace_size(64, 32, 4, 64, 32768, 0, 0)
    assert ws > 0
    # a single short sequence runs in one partition per head group: no workspace
    assert L.nyion_paged_decode_workspace_size(1, 32, 4, 64, 16, 0, 0) == 0
    assert L.nyion_paged_decode_workspace_size(1, 30, 4, 64, 16, 0, 0) == 0  # invalid heads


def test_node_scratch_fits_the_reference_scores_buffer():
    """The node uses at most the n_heads*seq_len floats any reference caller
    gives its scores buffer (fused_attention.cu:206; ScratchBuffers
    n_heads*window_size, lib.rs:317): planned on the host for a spread of
    shapes, including lengths where split-K pays."""
    L = nyion_hip.load()
    seen_split = False
    for hq, hkv in ((32, 4), (32, 8), (8, 8), (64, 4), (40, 8), (4, 1)):
        for d in (64, 128):
            for n in (1, 15, 16, 17, 128, 129, 1000, 2048, 4096, 4097, 16384, 65536, 131071):
                used = nyion_hip.node_scratch_bytes(hq, hkv, n, d)
                assert used <= 4 * hq * n, (hq, hkv, d, n, used)
                seen_split |= used > 0
    assert seen_split
    assert L.nyion_attention_node_scratch_bytes(30, 4, 128, 64) == 0  # invalid heads
