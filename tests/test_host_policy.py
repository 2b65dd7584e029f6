"""Host-side Fugu attention policy (FuguOrchestrator::decide_attention,
swamp-engine/src/fugu.rs:129-170) through the C ABI; no device needed.

Expected strategies are enumerated by hand from fugu.rs:129-170 (threshold
512 with a strict '>', 256 under predictive throttle with saturating
subtraction, window 256 halved under throttle, DSPark when the accept rate
is positive and seq_len > 2048 with num_dspark = clamp(n_heads, 4, 64) and
sentinel stride = head_dim)."""
import pytest

import nyion_hip as nh

FULL, SPARSE, DSPARK = nh.ATTN_FULL, nh.ATTN_SPARSE, nh.ATTN_SPARSE_DSPARK


@pytest.mark.parametrize("kw,expect", [
    (dict(seq_len=100000, is_prefill=True, dspark_accept_rate=0.9), (FULL, 0, 0, 0, 0)),
    (dict(seq_len=512), (FULL, 0, 0, 0, 0)),
    (dict(seq_len=513), (SPARSE, 256, 32, 0, 0)),
    (dict(seq_len=257, predictive_throttle=True), (SPARSE, 128, 32, 0, 0)),
    (dict(seq_len=256, predictive_throttle=True), (FULL, 0, 0, 0, 0)),
    (dict(seq_len=3000, dspark_accept_rate=0.5), (DSPARK, 256, 0, 64, 32)),
    (dict(seq_len=2048, dspark_accept_rate=0.5), (SPARSE, 256, 32, 0, 0)),
    (dict(seq_len=2049, dspark_accept_rate=0.5, predictive_throttle=True), (DSPARK, 128, 0, 64, 32)),
    (dict(seq_len=5000, dspark_accept_rate=0.0), (SPARSE, 256, 32, 0, 0)),
])
def test_decide_attention(kw, expect):
    s = nh.fugu_decide_attention(n_heads=32, head_dim=64, **kw)
    assert (s.kind, s.window, s.num_random, s.sentinel_stride, s.num_dspark) == expect


@pytest.mark.parametrize("n_heads,want", [(2, 4), (4, 4), (32, 32), (64, 64), (100, 64)])
def test_dspark_block_count_clamp(n_heads, want):
    s = nh.fugu_decide_attention(seq_len=4096, n_heads=n_heads, head_dim=128,
                                 dspark_accept_rate=0.1)
    assert s.kind == DSPARK and s.num_dspark == want and s.sentinel_stride == 128


def test_throttle_threshold_saturates():
    cfg = nh.FuguConfig(100, 256, 32, 32, 64)
    assert nh.fugu_decide_attention(1, 32, 64, predictive_throttle=True, cfg=cfg).kind == SPARSE
    assert nh.fugu_decide_attention(100, 32, 64, cfg=cfg).kind == FULL
    assert nh.fugu_decide_attention(101, 32, 64, cfg=cfg).kind == SPARSE
