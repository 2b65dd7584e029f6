"""Seeded synthetic workloads for the attention path (tests and bench.py).

Every tensor is drawn on the host with numpy's PCG64 (default_rng(seed)):
q, k, v ~ N(0, 1) f32, RoPE considered already applied, scale 1/sqrt(D).
Paged caches use 16-token blocks and a shuffled block table
(rng.permutation), one pool shared by all sequences of a batch.

Pool layout: [num_blocks][n_kv_heads][block_tokens][row], row = D f32 or the
Q4-20B bytes of one (token, kv head).
"""
from __future__ import annotations

import dataclasses
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("oracle", "nyion.rs_amd"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)

import oracle  # noqa: E402  (the reference results)


@dataclasses.dataclass
class PagedBatch:
    q: np.ndarray            # [B][Hq][D] f32
    k_pool: np.ndarray       # [NB][Hkv][bt][row] f32, u16 (binary16 bits) or u8 (Q4)
    v_pool: np.ndarray
    tables: np.ndarray       # [B][max_blocks] int32
    ctx_lens: np.ndarray     # [B] int32
    n_heads: int
    n_kv_heads: int
    head_dim: int
    block_tokens: int
    kv_dtype: int
    seed: int

    @property
    def batch(self) -> int:
        return self.q.shape[0]

    def layout(self, b: int):
        return oracle.paged_layout(self.k_pool, self.v_pool, self.tables[b], self.block_tokens,
                                   self.n_kv_heads, self.head_dim, self.kv_dtype)

    def kv_bytes(self, attended=None) -> int:
        """Algorithmic K+V bytes read: every attended (token, kv head) row once."""
        row = {oracle.KV_F32: self.head_dim * 4, oracle.KV_F16: self.head_dim * 2}.get(
            self.kv_dtype, oracle.q4_row_bytes(self.head_dim))
        toks = int(self.ctx_lens.sum()) if attended is None else int(attended)
        return 2 * toks * self.n_kv_heads * row


def _normal(rng, shape):
    return rng.standard_normal(size=shape, dtype=np.float32)


def paged_batch(ctx_lens, n_heads=32, n_kv_heads=4, head_dim=64, block_tokens=16, seed=0,
                kv_dtype=oracle.KV_F32, spare_blocks=0) -> PagedBatch:
    """One shared pool; sequence b owns ceil(ctx_b/bt) blocks at shuffled ids."""
    rng = np.random.default_rng(seed)
    ctx = np.asarray(ctx_lens, dtype=np.int32)
    B = len(ctx)
    nblk = (ctx + block_tokens - 1) // block_tokens
    total = int(nblk.sum()) + spare_blocks
    perm = rng.permutation(total).astype(np.int32)
    max_blocks = int(nblk.max())
    tables = np.zeros((B, max_blocks), dtype=np.int32)
    off = 0
    for b in range(B):
        tables[b, :nblk[b]] = perm[off:off + nblk[b]]
        off += nblk[b]
    q = _normal(rng, (B, n_heads, head_dim))
    k = _normal(rng, (total, n_kv_heads, block_tokens, head_dim))
    v = _normal(rng, (total, n_kv_heads, block_tokens, head_dim))
    if kv_dtype == oracle.KV_Q4:
        k = oracle.q4_quantize_rows(k)
        v = oracle.q4_quantize_rows(v)
    elif kv_dtype == oracle.KV_F16:  # binary16 rows (bits), round to nearest even
        k = k.astype(np.float16).view(np.uint16)
        v = v.astype(np.float16).view(np.uint16)
    return PagedBatch(q, k, v, tables, ctx, n_heads, n_kv_heads, head_dim, block_tokens, kv_dtype,
                      seed)


# ---------------------------------------------------------------- zone pools

@dataclasses.dataclass
class ZonePool:
    """K and V pools laid out as PagedKVCache's zone pages (1-D, in pool units:
    f32, binary16 bits as uint16, or Q4-20B bytes), page_base[p] the offset of
    flat page p in both pools (-1 absent)."""
    k_pool: np.ndarray
    v_pool: np.ndarray
    page_base: np.ndarray  # [n_pages] int64
    n_layers: int
    n_kv_heads: int
    head_dim: int
    kv_dtype: int

    @property
    def row(self) -> int:
        return oracle.q4_row_bytes(self.head_dim) if self.kv_dtype == oracle.KV_Q4 else self.head_dim


def zone_page_first_position(p: int) -> int:
    """First position of flat page p (the inverse of page_id, checked against
    the oracle's golden-pinned orc_zone_page_id by the caller)."""
    if p < 128:
        return 32 * p
    if p < 1120:
        return 4096 + 128 * (p - 128)
    return 131072 + 1024 * (p - 1120)


def zone_pool(n_tokens, n_layers=2, n_kv_heads=2, head_dim=64, kv_dtype=oracle.KV_F32, seed=0,
              present=None, gaps=True) -> ZonePool:
    """Pages covering [0, n_tokens) (only the flat ids in `present` when given),
    placed in shuffled order, with gaps of 0-3 alignment units between them,
    filled with N(0,1) rows (quantised for Q4-20B, rounded for binary16)."""
    L = oracle.lib()
    big = 1 << 40  # max_seq_len argument: beyond every position used
    n_pages = int(L.orc_zone_page_id(n_tokens - 1, big)) + 1
    pages = list(range(n_pages)) if present is None else sorted(set(int(p) for p in present))
    row = oracle.q4_row_bytes(head_dim) if kv_dtype == oracle.KV_Q4 else head_dim
    align = 8 if kv_dtype == oracle.KV_F16 else 4
    rng = np.random.default_rng(seed)
    base = np.full(n_pages, -1, np.int64)
    sizes = {}
    off = 0
    for p in rng.permutation(pages):
        first = zone_page_first_position(int(p))
        assert L.orc_zone_page_id(first, big) == p
        bs = int(L.orc_zone_block_size(first))
        off += align * int(rng.integers(0, 4)) if gaps else 0
        base[p] = off
        sizes[int(p)] = n_layers * n_kv_heads * bs * row
        off += sizes[int(p)]
    dt = {oracle.KV_F32: np.float32, oracle.KV_F16: np.uint16}.get(kv_dtype, np.uint8)
    pools = []
    for _ in range(2):
        pool = np.zeros(off + 64, dt)
        for p, units in sizes.items():
            x = _normal(rng, (units // row, head_dim))
            if kv_dtype == oracle.KV_Q4:
                x = oracle.q4_quantize_rows(x)
            elif kv_dtype == oracle.KV_F16:
                x = x.astype(np.float16).view(np.uint16)
            pool[base[p]:base[p] + units] = x.reshape(-1)
        pools.append(pool)
    return ZonePool(pools[0], pools[1], base, n_layers, n_kv_heads, head_dim, kv_dtype)


def zone_row_offsets(zp: ZonePool, layer: int, n_tokens: int) -> np.ndarray:
    """[Hkv][n_tokens] offsets (pool units) of each row through the oracle's
    zone arithmetic (orc_zone_page_id + orc_zone_f32_offset / _q4_offset),
    -1 where the page is absent."""
    L = oracle.lib()
    big = 1 << 40
    off = np.full((zp.n_kv_heads, n_tokens), -1, np.int64)
    rel = L.orc_zone_q4_offset if zp.kv_dtype == oracle.KV_Q4 else L.orc_zone_f32_offset
    for t in range(n_tokens):
        b = zp.page_base[L.orc_zone_page_id(t, big)]
        if b < 0:
            continue
        for h in range(zp.n_kv_heads):
            off[h, t] = b + rel(layer, h, t, zp.n_kv_heads, zp.head_dim)
    return off


def zone_rows(pool: np.ndarray, offsets: np.ndarray, row: int) -> np.ndarray:
    """[Hkv][n][row] raw rows at `offsets` (zeros where -1)."""
    out = np.zeros(offsets.shape + (row,), pool.dtype)
    ok = offsets >= 0
    out[ok] = pool[offsets[ok][:, None] + np.arange(row)]
    return out


def c1_contiguous(seed=0):
    """Contiguous node: B=1, 32/4 heads, D=64, contiguous f32 KV of 128 positions."""
    rng = np.random.default_rng(seed)
    q = _normal(rng, (32, 64))
    k = _normal(rng, (4, 128, 64))
    v = _normal(rng, (4, 128, 64))
    return q, k, v


def c3_lengths(seed=0, batch=64, lo=512, hi=32768):
    """Continuous batch: per-sequence context lengths ~ U[lo, hi]."""
    rng = np.random.default_rng(seed)
    return rng.integers(lo, hi + 1, size=batch).astype(np.int32)


def reference_decode(pb: PagedBatch, window=0, global_stride=0, q_pos=None, threads=1,
                     batches=None):
    """Oracle output [B][Hq][D] for the batch (ops::attention or its sliding-window form)."""
    out = np.zeros_like(pb.q)
    for b in (range(pb.batch) if batches is None else batches):
        L = int(pb.ctx_lens[b])
        qp = L - 1 if q_pos is None else int(q_pos[b])
        lay = pb.layout(b)
        if window > 0:
            pos = oracle.sparse_positions(L, qp, window, global_stride)
            out[b] = oracle.attention_positions(pb.q[b], lay, pos, pb.n_heads, pb.n_kv_heads,
                                                pb.head_dim, threads).reshape(pb.n_heads, -1)
        else:
            out[b] = oracle.attention(pb.q[b], lay, L, qp, pb.n_heads, pb.n_kv_heads,
                                      pb.head_dim, threads=threads).reshape(pb.n_heads, -1)
    return out


# Importance (attention_tracked's per-position sum over heads of the softmax
# probability, f64) is compared per position against the oracle: f32
# probabilities carry ~1e-7 relative error per head, so 1e-5 of the position's
# own value (plus 1e-7 for positions that hold almost nothing) leaves two
# orders of magnitude of margin, while a head whose probabilities sit one
# position off, or a head left out at one position, moves that position by
# a whole per-head probability (~3 % of the position's importance at 32
# heads): tests/test_importance_tolerance.py checks that such mistakes fail.
IMP_RTOL, IMP_ATOL = 1e-5, 1e-7


def importance_excess(got, ref, rtol=IMP_RTOL, atol=IMP_ATOL):
    """Per-position |got - ref| / (atol + rtol |ref|); above 1 fails."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return np.abs(got - ref) / (atol + rtol * np.abs(ref))


def assert_importance(got, ref, what=""):
    ex = importance_excess(got, ref)
    bad = int(np.sum(~(ex <= 1.0)))
    worst = float(np.nanmax(ex)) if ex.size else 0.0
    assert bad == 0, (f"{what}: importance of {bad} positions outside {IMP_ATOL:g} + "
                      f"{IMP_RTOL:g}*|ref| (worst {worst:.2f}x the bound)")
    return worst


def window_importance(pb: "PagedBatch", b: int, q_pos: int, window: int, global_stride: int,
                      n: int) -> np.ndarray:
    """The oracle's importance of sequence b over a window (with strided
    globals) as an array of n positions, zero outside the attended set."""
    L = int(pb.ctx_lens[b])
    pos = oracle.sparse_positions(L, q_pos, window, global_stride)
    _, imp = oracle.attention_positions(pb.q[b], pb.layout(b), pos, pb.n_heads, pb.n_kv_heads,
                                        pb.head_dim, importance=True)
    full = np.zeros(n, np.float64)
    full[pos] = imp
    return full


def prefill_inputs(n, n_heads=32, n_kv_heads=8, head_dim=128, seed=0):
    """Prefill shapes: fp32 N(0,1) q [n][Hq][D], k, v [n][Hkv][D]."""
    rng = np.random.default_rng(seed)
    q = _normal(rng, (n, n_heads, head_dim))
    k = _normal(rng, (n, n_kv_heads, head_dim))
    v = _normal(rng, (n, n_kv_heads, head_dim))
    return q, k, v


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round f32 to the nearest bf16 (ties to even), returned as f32."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    lsb = (b >> 16) & 1
    r = ((b + 0x7FFF + lsb) & 0xFFFF0000).astype(np.uint32)
    nan = np.isnan(x)
    r[nan] = (b[nan] | 0x00400000) & 0xFFFF0000
    return r.view(np.float32)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def brute_force_attention(q, k, v, valid_end, scale=None):
    """float64 softmax(q K^T * scale) V over keys [0, valid_end]; q [D], k/v [T][D]."""
    q = q.astype(np.float64)
    k = k[:valid_end + 1].astype(np.float64)
    v = v[:valid_end + 1].astype(np.float64)
    s = (k @ q) * (scale if scale is not None else 1.0 / np.sqrt(q.shape[0]))
    s -= s.max()
    p = np.exp(s)
    p /= p.sum()
    return p @ v


# ---------------------------------------------------------------------------
# Q4_K weights (GGUF 144-byte blocks, swamp-kernels/src/fused_gemv_q4k.rs)
# ---------------------------------------------------------------------------

def q4k_pack_scales(scales, mins) -> np.ndarray:
    """Eight 6-bit scales and mins -> the 12 packed bytes (the inverse of
    unpack_scales_q4k, fused_gemv_q4k.rs:30-43)."""
    s = np.asarray(scales, dtype=np.uint8) & 63
    m = np.asarray(mins, dtype=np.uint8) & 63
    out = np.zeros(12, np.uint8)
    out[0:4] = s[0:4] | ((s[4:8] >> 4) << 6)
    out[4:8] = m[0:4] | ((m[4:8] >> 4) << 6)
    out[8:12] = (s[4:8] & 0x0F) | ((m[4:8] & 0x0F) << 4)
    return out


def q4k_block(d, dmin, scales, mins, qs) -> np.ndarray:
    b = np.zeros(144, np.uint8)
    b[0:2] = np.array([d], np.float16).view(np.uint8)
    b[2:4] = np.array([dmin], np.float16).view(np.uint8)
    b[4:16] = q4k_pack_scales(scales, mins)
    b[16:144] = np.asarray(qs, dtype=np.uint8)
    return b


def q4k_random_weights(n_rows, n_cols, seed=0, d_range=(5e-5, 5e-4)) -> np.ndarray:
    """Random Q4_K matrix [n_rows][n_cols/256 * 144] u8 with finite f16
    d, dmin of realistic magnitude and uniform 6-bit scales, mins, nibbles."""
    rng = np.random.default_rng(seed)
    nb = n_rows * (n_cols // 256)
    w = rng.integers(0, 256, size=(nb, 144), dtype=np.uint8)
    d = rng.uniform(*d_range, size=nb).astype(np.float16)
    dmin = rng.uniform(0.0, d_range[1], size=nb).astype(np.float16)
    w[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    w[:, 2:4] = dmin.view(np.uint8).reshape(nb, 2)
    return w.reshape(n_rows, -1)


def q4k_dequant_np(w: np.ndarray, n_rows: int, n_cols: int) -> np.ndarray:
    """numpy restatement of the Q4_K weight formula (f32 products as the
    scalar GEMV rounds them): [n_rows][n_cols] f32."""
    b = np.ascontiguousarray(w, dtype=np.uint8).reshape(-1, 144)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    dmin = b[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]
    sc = b[:, 4:16].astype(np.uint8)
    scales = np.zeros((b.shape[0], 8), np.uint8)
    mins = np.zeros((b.shape[0], 8), np.uint8)
    scales[:, 0:4] = sc[:, 0:4] & 63
    mins[:, 0:4] = sc[:, 4:8] & 63
    scales[:, 4:8] = (sc[:, 8:12] & 0x0F) | ((sc[:, 0:4] >> 6) << 4)
    mins[:, 4:8] = (sc[:, 8:12] >> 4) | ((sc[:, 4:8] >> 6) << 4)
    qs = b[:, 16:144].reshape(-1, 4, 32)
    q = np.zeros((b.shape[0], 8, 32), np.uint8)
    q[:, 0::2, :] = qs & 0x0F
    q[:, 1::2, :] = qs >> 4
    sv = (d[:, None] * scales.astype(np.float32)).astype(np.float32)
    mv = (dmin[:, None] * mins.astype(np.float32)).astype(np.float32)
    wf = (sv[:, :, None] * q.astype(np.float32)).astype(np.float32) - mv[:, :, None]
    return wf.astype(np.float32).reshape(n_rows, n_cols)


def q4k_reference_test_weights(n_rows: int) -> np.ndarray:
    """The weights of the reference's own GEMV tests (fused_gemv_q4k.rs:830-840):
    one block per row, d = 0.5 + 0.1 r, dmin = 0.1 + 0.05 r, every scale
    (r + 1) & 63, every min (r + 2) & 63, every nibble 8."""
    rows = []
    for r in range(n_rows):
        d = np.float32(0.5) + np.float32(r) * np.float32(0.1)
        dm = np.float32(0.1) + np.float32(r) * np.float32(0.05)
        rows.append(q4k_block(d, dm, [(r + 1) & 63] * 8, [(r + 2) & 63] * 8, [8 | (8 << 4)] * 128))
    return np.stack(rows)


def q4k_reference_test_x(n_cols: int) -> np.ndarray:
    """fused_gemv_q4k.rs:842-844: x_i = (i % 100) / 50 - 1."""
    i = np.arange(n_cols)
    return ((i % 100).astype(np.float32) / np.float32(50.0) - np.float32(1.0)).astype(np.float32)


# ---------------------------------------------------------------------------
# Q6_K weights (210-byte blocks, swamp-kernels/src/fused_gemv_q6k.rs)
# ---------------------------------------------------------------------------

def q6k_random_weights(n_rows, n_cols, seed=0, d_range=(7e-5, 5e-4)) -> np.ndarray:
    """Random Q6_K matrix [n_rows][n_cols/256 * 210] u8.  d stays a normal f16:
    the reference converts exponent-0 values (zero, subnormals) to about
    -2e34, which overflows any dot product."""
    rng = np.random.default_rng(seed)
    nb = n_rows * (n_cols // 256)
    w = rng.integers(0, 256, size=(nb, 210), dtype=np.uint8)
    d = rng.uniform(*d_range, size=nb).astype(np.float16)
    w[:, 208:210] = d.view(np.uint8).reshape(nb, 2)
    return w.reshape(n_rows, -1)


def q6k_dequant_np(w: np.ndarray, n_rows: int, n_cols: int) -> np.ndarray:
    """numpy restatement (normal d only): element 128h + l + 32k of a block
    is d * sc[8h + l//16 + 2k] * (q - 32), q from the low (k < 2) or high
    nibble of ql[64h + l + 32(k % 2)] and bits 2k..2k+1 of qh[32h + l]."""
    b = np.ascontiguousarray(w, dtype=np.uint8).reshape(-1, 210)
    d = b[:, 208:210].copy().view(np.float16).astype(np.float32)[:, 0]
    out = np.empty((b.shape[0], 256), np.float32)
    l = np.arange(32)
    for h in range(2):
        ql = b[:, 64 * h:64 * h + 64].astype(np.int32)
        qh = b[:, 128 + 32 * h:128 + 32 * h + 32].astype(np.int32)
        sc = b[:, 192 + 8 * h:200 + 8 * h].view(np.int8).astype(np.float32)
        for k in range(4):
            nib = ql[:, l + 32 * (k % 2)]
            nib = (nib & 0x0F) if k < 2 else (nib >> 4)
            q = nib | (((qh[:, l] >> (2 * k)) & 3) << 4)
            s = sc[:, l // 16 + 2 * k]
            out[:, 128 * h + l + 32 * k] = ((d[:, None] * s).astype(np.float32) *
                                           (q - 32).astype(np.float32)).astype(np.float32)
    return out.reshape(n_rows, n_cols)


def q6k_reference_test_weights(n_rows: int, n_blocks: int) -> np.ndarray:
    """The blocks of the reference's own Q6_K tests (fused_gemv_q6k.rs:329-356)."""
    i128, i64, i16 = np.arange(128), np.arange(64), np.arange(16)
    ql = ((i128 & 0x0F) | (((i128 + 128) & 0x0F) << 4)).astype(np.uint8)
    qh = np.zeros(64, np.uint8)
    for j in range(4):
        qh |= ((((i64 + 64 * j) >> 4) & 3) << (2 * j)).astype(np.uint8)
    rows = []
    for r in range(n_rows):
        blk = np.zeros(210, np.uint8)
        blk[0:128] = ql
        blk[128:192] = qh
        blk[192:208] = ((r * 16 + i16 + 1) & 0x7F).astype(np.uint8)
        blk[208:210] = np.array([0x3800], np.uint16).view(np.uint8)
        rows.append(np.tile(blk, n_blocks))
    return np.stack(rows)
