"""Zone-geometry host helpers of the HIP library (CPU, no device calls).

nyion_zone_page_id / nyion_zone_page_tokens against the page ids and page
sizes of the reference's own zone test (golden JSON, cache.rs:1000-1029),
and against the golden-pinned oracle over every zone boundary."""
import json
import os

import numpy as np

import nyion_hip
import oracle
import workloads as W

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))


def test_zone_page_ids_golden():
    for pos, pid in GOLD["zone_page_id"]["cases"]:
        assert nyion_hip.zone_page_id(pos) == pid, pos
    for pos, bs in GOLD["zone_block_size"]["cases"]:
        assert nyion_hip.zone_page_tokens(pos) == bs, pos


def test_zone_page_ids_match_oracle_around_boundaries():
    L = oracle.lib()
    big = 1 << 40
    pts = set()
    for edge in (0, 4096, 131072, 1 << 20, (1 << 31) - 1):
        pts.update(range(max(0, edge - 300), edge + 300))
    pts.update(np.random.default_rng(0).integers(0, 1 << 31, 2000).tolist())
    for pos in sorted(pts):
        assert nyion_hip.zone_page_id(pos) == L.orc_zone_page_id(pos, big), pos
        assert nyion_hip.zone_page_tokens(pos) == L.orc_zone_block_size(pos), pos
    assert nyion_hip.zone_page_id(-1) == -1 and nyion_hip.zone_page_tokens(-1) == -1


def test_zone_pool_builder_places_pages_disjointly():
    """The test pools' page placement: pages never overlap, every row offset of
    every layer and head lands inside its own page."""
    zp = W.zone_pool(4300, n_layers=2, n_kv_heads=3, head_dim=64, seed=3)
    L = oracle.lib()
    spans = []
    for p, b in enumerate(zp.page_base):
        bs = L.orc_zone_block_size(W.zone_page_first_position(p))
        spans.append((int(b), int(b) + 2 * 3 * bs * 64))
    spans.sort()
    assert all(a[1] <= b[0] for a, b in zip(spans, spans[1:]))
    for layer in range(2):
        off = W.zone_row_offsets(zp, layer, 4300)
        assert len(np.unique(off)) == off.size
        assert off.min() >= 0 and off.max() + 64 <= zp.k_pool.size
