"""The importance check itself (CPU only).

attention_tracked (swamp-engine/src/ops.rs:283-401) adds, per attended
position, the sum over heads of that head's softmax probability.  The GPU
tests compare it per position with workloads.assert_importance.  These tests
pin that comparison: it must accept the rounding of f32 probabilities and
reject the mistakes a kernel could make with the head and position indices
(one head's probabilities one position off, one head left out at one
position), which a bound on the absolute error of the sum would let through.
The listed-position importance of the oracle is pinned here too: over the full
position set it equals orc_attention's, and float64 brute force agrees.
"""
import numpy as np

import oracle
import workloads as W


def _per_head_probs_f64(pb, b, positions):
    """float64 softmax probabilities [Hq][len(positions)] over the listed positions."""
    t = np.asarray(positions)
    table = pb.tables[b]
    out = np.zeros((pb.n_heads, len(t)))
    group = pb.n_heads // pb.n_kv_heads
    for h in range(pb.n_heads):
        kv = h // group
        k = pb.k_pool[table[t // pb.block_tokens], kv, t % pb.block_tokens].astype(np.float64)
        s = (k @ pb.q[b, h].astype(np.float64)) / np.sqrt(pb.head_dim)
        e = np.exp(s - s.max())
        out[h] = e / e.sum()
    return out


def test_positions_importance_equals_full_importance():
    pb = W.paged_batch([700], seed=41)
    _, full = oracle.attention(pb.q[0], pb.layout(0), 700, 650, 32, 4, 64, importance=True)
    _, listed = oracle.attention_positions(pb.q[0], pb.layout(0), np.arange(651), 32, 4, 64,
                                           importance=True)
    assert np.array_equal(full[:651], listed)
    assert np.all(full[651:] == 0.0)


def test_positions_importance_matches_float64():
    pb = W.paged_batch([3000], seed=42)
    pos = oracle.sparse_positions(3000, 2999, 500, 32)
    _, imp = oracle.attention_positions(pb.q[0], pb.layout(0), pos, 32, 4, 64, importance=True)
    ref = _per_head_probs_f64(pb, 0, pos).sum(axis=0)
    W.assert_importance(imp, ref, "oracle vs float64")
    assert abs(imp.sum() - 32.0) < 1e-5


def test_tolerance_accepts_f32_rounding_and_rejects_index_mistakes():
    pb = W.paged_batch([4096], seed=43)
    pos = np.arange(4096)
    probs = _per_head_probs_f64(pb, 0, pos)
    _, ref = oracle.attention(pb.q[0], pb.layout(0), 4096, 4095, 32, 4, 64, importance=True)
    # f32 probabilities: each head's p rounded to f32 with a few ulp of noise
    rng = np.random.default_rng(44)
    noisy = (probs * (1.0 + 4e-7 * rng.standard_normal(probs.shape))).astype(np.float32)
    W.assert_importance(noisy.astype(np.float64).sum(axis=0), ref, "f32-rounded probabilities")
    for h in (0, 17, 31):
        # head h's probabilities one position off
        shifted = ref - probs[h] + np.roll(probs[h], 1)
        assert np.max(W.importance_excess(shifted, ref)) > 1.0, f"shift of head {h} accepted"
        # head h left out at one position
        for t in (5, 2048, 4095):
            dropped = ref.copy()
            dropped[t] -= probs[h, t]
            assert np.max(W.importance_excess(dropped, ref)) > 1.0, (h, t)
            # the absolute bound 1e-4 * n_heads used before accepts this mistake
            # at most positions: one head's probability is ~2.4e-4 on average
    typical = np.median(probs)
    assert typical < 1e-4 * 32, typical
