// decode_attention.hip — batched paged GQA decode attention for gfx950.
//
// One query token per sequence (the executor's decode step,
// swamp-engine/src/executor.rs:739-763).  Semantics follow ops::attention
// (swamp-engine/src/ops.rs:170-278) and ops::attention_sparse (ops.rs:85-168);
// the header states the position sets.
//
// Work decomposition.  A 256-thread workgroup owns one (sequence, kv head,
// group of up to 16 q heads, split-K partition); its four wavefronts take
// consecutive runs of 16-token tiles of that partition.  All q heads of a GQA
// group are processed together, so each K/V byte is read from HBM once.
//
// Per 16-token tile a wavefront runs two MFMA chains on
// v_mfma_f32_16x16x4_f32 (fp32 in, fp32 accumulate):
//   S[16 tok][16 heads] = K_tile[16][D] . Q^T[D][16]       (D/4 MFMAs)
//   O[16 heads][D]     += P[16 heads][16 tok] . V_tile      (D/4 MFMAs)
// The MFMA output layout of S (lane = head + 16*token_quad, reg = token in
// quad) is exactly the A-operand layout P needs in the second product, so the
// probabilities never leave registers.
//
// Memory.  Tiles are aligned to 16 positions, so with blocks of >= 16 tokens
// a tile lies in one block: its block id is one wave-uniform value, read from
// a per-wavefront copy of the block-table slice loaded once.  K rows arrive as
// 128-bit loads (the four token quads of a row read 64 contiguous bytes per
// instruction), V rows as 16 lanes x 16 B = one whole row per instruction.
// The next tile's loads are issued before the current tile's MFMAs (register
// double buffering).  Q4-20B rows stay packed in registers until the tile is
// consumed and are dequantised there, bit-exactly as dequant_block.
//
// Softmax.  Online, in the log2 domain, on the S registers: tile max over the
// 4 registers and the 4 token quads (lane xor 16, 32), rescale, exp2.
//
// Split-K.  The four wavefronts of a workgroup merge through LDS.  When a
// sequence needs several workgroups, each writes one (m, l, O) partial to the
// workspace with device-coherent (write-through) stores, waits for them, and
// counts its arrival with an agent-scope atomic; the last workgroup to arrive
// reads the partials with device-coherent loads, merges them with
// log-sum-exp, writes the output and resets its counter to 0.  No L2
// write-back or invalidate is issued, and one decode call is one launch.
#include <float.h>
#include <math.h>

#include "common.hpp"

namespace nyion {

typedef float floatx4 __attribute__((ext_vector_type(4)));

enum DecodeMode { MODE_FULL = 0, MODE_WINDOW = 1, MODE_LIST = 2 };

struct DecodeArgs {
    const float* q;  // [B][Hq][D]
    const void* k;
    const void* v;
    const int32_t* tables;     // [B][table_stride] or nullptr (contiguous)
    const int32_t* ctx_lens;   // [B] or nullptr (uniform_len)
    const int32_t* q_pos;      // [B] or nullptr (len - 1)
    const int32_t* positions;  // MODE_LIST: [B][pos_stride]
    const int32_t* n_pos;      // MODE_LIST: [B]
    float* out;                // [B][Hq][D]
    float* ws_acc;             // [(b*Hq + head)*max_parts + p][D]
    float2* ws_ml;             // [(b*Hq + head)*max_parts + p] = (m log2, l)
    int* counters;             // [B][Hkv][n_hg], zero between calls
    long long block_stride;
    long long head_stride;
    int table_stride;
    int pos_stride;
    int uniform_len;
    int n_heads;
    int n_kv_heads;
    int group;  // q heads per kv head
    int n_hg;   // ceil(group / 16)
    int token_stride;
    int bt_log2;
    int num_blocks;
    int window;
    int global_stride;
    int mode;
    int tpw;        // tiles per wavefront per partition
    int max_parts;  // workgroup partitions per (sequence, kv head, head group): grid.x
    int max_len;    // host bound on attended positions per sequence
    float scale_log2;  // scale * log2(e)
};

// Attended positions of one sequence.
//  aligned path (FULL/WINDOW, blocks >= 16 tokens): the contiguous range
//    [lo, hi] walked in 16-aligned tiles from lo & ~15, plus n_glob strided
//    globals (stride*g) in one extra partition;
//  gather path: L virtual positions (the same sets, or an explicit list).
struct Extent {
    int lo, hi, n_glob, L;
    int main_tiles;  // aligned: tiles over [lo & ~15, hi]
    int np_main;     // partitions over the main tiles (aligned) or all tiles (gather)
    int np;          // total partitions
};

template <bool ALIGNED>
__device__ __forceinline__ Extent extent(const DecodeArgs& a, int b) {
    Extent e{0, -1, 0, 0, 0, 0, 0};
    const int per_part = 4 * a.tpw;  // tiles per workgroup partition
    // per-sequence values are wave-uniform: keep them (and everything derived
    // from them) in scalar registers so tile loops branch uniformly
    if (a.mode == MODE_LIST) {
        e.L = min(max(__builtin_amdgcn_readfirstlane(a.n_pos[b]), 0), a.max_len);
    } else {
        const int len = a.ctx_lens ? __builtin_amdgcn_readfirstlane(a.ctx_lens[b]) : a.uniform_len;
        const int qp = a.q_pos ? __builtin_amdgcn_readfirstlane(a.q_pos[b]) : len - 1;
        if (len <= 0 || qp < 0) return e;
        const int ve = min(qp, len - 1);  // ops.rs:183
        int lo = 0;
        if (a.mode == MODE_WINDOW) {
            lo = ve > a.window ? ve - a.window + 1 : 0;  // strict '>' (ops.rs:100)
            e.n_glob = a.global_stride > 0 ? min(lo / a.global_stride, 128) : 0;
        }
        e.lo = lo;
        e.hi = min(ve, lo + a.max_len - 1);
        e.L = e.n_glob + (e.hi - lo + 1);
    }
    if (ALIGNED) {
        if (e.hi < e.lo) return e;
        e.main_tiles = (e.hi - (e.lo & ~15)) / 16 + 1;
        e.np_main = (e.main_tiles + per_part - 1) / per_part;
        e.np = min(e.np_main + (e.n_glob > 0 ? 1 : 0), a.max_parts);
    } else {
        const int tiles = (e.L + 15) / 16;
        e.np_main = (tiles + per_part - 1) / per_part;
        e.np = min(e.np_main, a.max_parts);
    }
    return e;
}

// Virtual index -> position, gather path (and the globals of the aligned path).
__device__ __forceinline__ int virt_to_pos(const DecodeArgs& a, const Extent& e, int b, int v) {
    if (a.mode == MODE_FULL) return v;
    if (a.mode == MODE_WINDOW) return v < e.n_glob ? v * a.global_stride : e.lo + (v - e.n_glob);
    return a.positions[(long long)b * a.pos_stride + v];
}

// ---------------------------------------------------------------- tiles
// K operand of lane (row i, quad kq): NC = D/4 values, one per QK MFMA.
//   f32: call c = 4x+y holds dim 16x + 4kq + y  (per x, the 4 quads of a row
//        read 64 contiguous bytes)
//   Q4 : call c holds dim kq*D/4 + c            (contiguous nibbles)
// The Q operand uses the same map (qk_dim).  V operand of lane (col j, quad
// kq), row 4kq+r: DPL = D/16 consecutive dims from DPL*j.
template <int D, int KVT>
__device__ __forceinline__ int qk_dim(int c, int kq) {
    if constexpr (KVT == NYION_KV_F32)
        return 16 * (c >> 2) + 4 * kq + (c & 3);
    else
        return kq * (D / 4) + c;
}

// Raw (undecoded) registers of one tile for one lane.
template <int D, int KVT>
struct Tile;

template <int D>
struct Tile<D, NYION_KV_F32> {
    float4 k[D / 16];         // K row j: dims 16x + 4kq .. +3
    float4 v[4][D / 64];      // V rows 4kq+r: dims DPL*j .. +DPL
};

template <int D>
struct Tile<D, NYION_KV_Q4_20B> {
    uint32_t khdr;            // f16 d | f16 dmin << 16 of the lane's K group
    uint32_t k[D / 32];       // D/4 nibbles of K row j
    uint32_t vhdr[4];
    uint32_t v[4];            // D/16 nibbles of V row 4kq+r (low 16 bits when D = 64)
};

// Loads are unconditional (an invalid row reads offset 0 of the pool, which is
// valid memory) so that the compiler keeps them in flight across the MFMA
// chain of the previous tile; invalid rows are masked when the tile is consumed.
template <int D, int KVT>
__device__ __forceinline__ void load_tile(Tile<D, KVT>& t, const void* kb, const void* vb,
                                          long long koff, const long long* voff, int j, int kq) {
    if constexpr (KVT == NYION_KV_F32) {
        const float* kr = (const float*)kb + koff;
#pragma unroll
        for (int x = 0; x < D / 16; x++) t.k[x] = *(const float4*)(kr + 16 * x + 4 * kq);
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float* vr = (const float*)vb + voff[r] + (D / 16) * j;
#pragma unroll
            for (int x = 0; x < D / 64; x++) t.v[r][x] = *(const float4*)(vr + 4 * x);
        }
    } else {
        const int ke0 = kq * (D / 4);
        const uint8_t* kr = (const uint8_t*)kb + koff + kQ4GroupBytes * (ke0 >> 5);
        t.khdr = *(const uint32_t*)kr;
        const uint32_t* kn = (const uint32_t*)(kr + 4 + ((ke0 & 31) >> 1));
#pragma unroll
        for (int w = 0; w < D / 32; w++) t.k[w] = kn[w];
        const int ve0 = (D / 16) * j;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const uint8_t* vr = (const uint8_t*)vb + voff[r] + kQ4GroupBytes * (ve0 >> 5);
            t.vhdr[r] = *(const uint32_t*)vr;
            const uint8_t* vn = vr + 4 + ((ve0 & 31) >> 1);
            if constexpr (D == 64)
                t.v[r] = (uint32_t)(*(const uint16_t*)vn);
            else
                t.v[r] = *(const uint32_t*)vn;
        }
    }
}

template <int D, int KVT>
__device__ __forceinline__ void decode_k(const Tile<D, KVT>& t, float* kv) {
    if constexpr (KVT == NYION_KV_F32) {
#pragma unroll
        for (int x = 0; x < D / 16; x++) {
            kv[4 * x + 0] = t.k[x].x;
            kv[4 * x + 1] = t.k[x].y;
            kv[4 * x + 2] = t.k[x].z;
            kv[4 * x + 3] = t.k[x].w;
        }
    } else {
        const float d = f16_bits_to_f32(t.khdr), dmin = f16_bits_to_f32(t.khdr >> 16);
#pragma unroll
        for (int w = 0; w < D / 32; w++) q4_dequant8(t.k[w], d, dmin, kv + 8 * w);
    }
}

template <int D, int KVT>
__device__ __forceinline__ void decode_v(const Tile<D, KVT>& t, int r, float* vv) {
    if constexpr (KVT == NYION_KV_F32) {
#pragma unroll
        for (int x = 0; x < D / 64; x++) {
            vv[4 * x + 0] = t.v[r][x].x;
            vv[4 * x + 1] = t.v[r][x].y;
            vv[4 * x + 2] = t.v[r][x].z;
            vv[4 * x + 3] = t.v[r][x].w;
        }
    } else {
        const float d = f16_bits_to_f32(t.vhdr[r]), dmin = f16_bits_to_f32(t.vhdr[r] >> 16);
        if constexpr (D == 64)
            q4_dequant4(t.v[r], d, dmin, vv);
        else
            q4_dequant8(t.v[r], d, dmin, vv);
    }
}

// Running state of one wavefront: O (reg r of acc[t] = head 4kq+r, dim
// DPL*j+t), per-head max (log2) and this lane's share of the denominator.
template <int D>
struct State {
    floatx4 acc[D / 16];
    float m;
    float l;
};

// Rescale threshold of the online softmax, log2 units.  The running max of a
// head is only moved when a tile's max exceeds it by more than this, so
// exp2(s - m) <= 2^8 and the O rescale is rare after the first tiles.
constexpr float kRescaleLog2 = 8.0f;

// One tile: bit i of `mask` (wave-uniform) marks row i of the 16 valid;
// MASKED = false is the all-valid fast path.
template <int D, int KVT, bool MASKED>
__device__ __forceinline__ void consume_tile(State<D>& st, const Tile<D, KVT>& t, const float* qv,
                                             uint32_t mask, int kq, float scale_log2) {
    constexpr int NC = D / 4;
    constexpr int DPL = D / 16;
    float kv[NC];
    decode_k<D, KVT>(t, kv);
    floatx4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NC; c++) s = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[c], qv[c], s, 0, 0, 0);

    float sv[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        sv[r] = s[r] * scale_log2;
        if (MASKED) sv[r] = ((mask >> (4 * kq + r)) & 1u) ? sv[r] : -1e30f;
    }
    float mt = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
    mt = fmaxf(mt, __shfl_xor(mt, 16));
    mt = fmaxf(mt, __shfl_xor(mt, 32));
    if (__any(mt > st.m + kRescaleLog2)) {  // wave-uniform; first tile always
        const float mnew = fmaxf(st.m, mt);
        const float alpha = __builtin_amdgcn_exp2f(st.m - mnew);
        st.l *= alpha;
        st.m = mnew;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float ar = __shfl(alpha, 4 * kq + r);
#pragma unroll
            for (int x = 0; x < DPL; x++) st.acc[x][r] *= ar;
        }
    }
    float pr[4];
#pragma unroll
    for (int r = 0; r < 4; r++) pr[r] = __builtin_amdgcn_exp2f(sv[r] - st.m);
    st.l += (pr[0] + pr[1]) + (pr[2] + pr[3]);
#pragma unroll
    for (int r = 0; r < 4; r++) {
        float vv[DPL];
        decode_v<D, KVT>(t, r, vv);
        if (MASKED) {  // masked rows may hold uninitialised slots: keep NaN out
            const bool ok = (mask >> (4 * kq + r)) & 1u;
#pragma unroll
            for (int x = 0; x < DPL; x++) vv[x] = ok ? vv[x] : 0.f;
        }
#pragma unroll
        for (int x = 0; x < DPL; x++)
            st.acc[x] = __builtin_amdgcn_mfma_f32_16x16x4f32(pr[r], vv[x], st.acc[x], 0, 0, 0);
    }
}

template <int D, int KVT>
__device__ __forceinline__ void consume(State<D>& st, const Tile<D, KVT>& t, const float* qv,
                                        uint32_t mask, int kq, float scale_log2) {
    if (mask == 0xffffu)
        consume_tile<D, KVT, false>(st, t, qv, mask, kq, scale_log2);
    else if (mask)
        consume_tile<D, KVT, true>(st, t, qv, mask, kq, scale_log2);
}

// Row offsets of tile `tile` on the aligned path: positions t0 .. t0+15 of
// one block; valid rows [vlo, vhi].
struct AlignedWalk {
    int base;        // lo & ~15
    int lo, hi;
    int bi_first;    // first block index of this wavefront's tiles
    int tblv;        // lane l: block id of block index bi_first + l (or -1)
    long long head_off;
};

template <int D, int KVT>
__device__ __forceinline__ uint32_t aligned_offsets(const DecodeArgs& a, const AlignedWalk& w,
                                                    int tile, int j, int kq, long long& koff,
                                                    long long* voff) {
    const int t0 = w.base + 16 * tile;
    int blk = 0;
    if (a.tables) blk = __builtin_amdgcn_readlane(w.tblv, (t0 >> a.bt_log2) - w.bi_first);
    const int vlo = max(w.lo - t0, 0);
    const int vhi = min(w.hi - t0, 15);
    uint32_t mask = (vhi >= vlo) ? (((2u << vhi) - 1u) & ~((1u << vlo) - 1u)) : 0u;
    if (blk < 0) {  // block index past the table or block id out of range
        blk = 0;
        mask = 0;
    }
    // rows of a paged pool are contiguous: the token stride is the row size
    constexpr int TS = KVT == NYION_KV_F32 ? D : q4_row_bytes(D);
    const long long base = (long long)blk * a.block_stride + w.head_off +
                           (long long)(t0 & ((1 << a.bt_log2) - 1)) * TS;
    koff = base + j * TS;
    const long long vbase = base + 4 * kq * TS;
#pragma unroll
    for (int r = 0; r < 4; r++) voff[r] = vbase + r * TS;
    return mask;
}

// Gather path: virtual indices v0 .. v0+15 (< vend), one table lookup per
// row.  Invalid rows point at offset 0 and are masked.
template <int D, int KVT>
__device__ __forceinline__ uint32_t gather_offsets(const DecodeArgs& a, const Extent& e,
                                                   const RowMap& m, int b, int kvh, int v0,
                                                   int vend, bool globals, int j, int kq,
                                                   long long& koff, long long* voff) {
    auto off_of = [&](int v) -> long long {
        if (v >= vend) return -1;
        const int pos = globals ? v * a.global_stride : virt_to_pos(a, e, b, v);
        if (pos < 0) return -1;
        return row_offset(m, pos, kvh);
    };
    koff = off_of(v0 + j);
    const uint32_t mask = (uint32_t)(__ballot(koff >= 0) & 0xffffu);
    koff = koff < 0 ? 0 : koff;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const long long o = off_of(v0 + 4 * kq + r);
        voff[r] = o < 0 ? 0 : o;
    }
    return mask;
}

// Walk `n` tiles with the next tile's loads in flight during each MFMA chain.
// Every step issues exactly one tile of loads (at the end, a repeat of the
// last tile that is never consumed), so the number of loads in flight is the
// same on every path and each tile waits only for its own loads.
template <int D, int KVT, typename Offsets>
__device__ __forceinline__ void walk_tiles(State<D>& st, const DecodeArgs& a, const float* qv, int n,
                                           int j, int kq, Offsets offsets) {
    Tile<D, KVT> ta, tb;
    long long ko, vo[4];
    if (n <= 0) return;
    uint32_t ma = offsets(0, ko, vo);
    load_tile<D, KVT>(ta, a.k, a.v, ko, vo, j, kq);
    for (int i = 0; i < n; i += 2) {
        uint32_t mb = offsets(min(i + 1, n - 1), ko, vo);
        load_tile<D, KVT>(tb, a.k, a.v, ko, vo, j, kq);
        consume<D, KVT>(st, ta, qv, ma, kq, a.scale_log2);
        ma = offsets(min(i + 2, n - 1), ko, vo);
        load_tile<D, KVT>(ta, a.k, a.v, ko, vo, j, kq);
        if (i + 1 < n) consume<D, KVT>(st, tb, qv, mb, kq, a.scale_log2);
    }
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
    return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
    return x;
}

// Log-sum-exp merge of the np partials of one (sequence, q head) by one
// wavefront: lanes over partitions for the weights, lanes over dims for O.
// The partials come from other workgroups, so they are read with
// device-coherent loads, 32 partitions' worth issued before any is used.
template <int D>
__device__ void merge_head(const DecodeArgs& a, long long slot0, int np, float* out, int lane) {
    constexpr int X = D / 64;  // dims per lane
    constexpr int CH = 32;     // partitions per batch of loads
    const float* mlp = (const float*)(a.ws_ml + slot0);
    float mx = -INFINITY;
    for (int p = lane; p < np; p += 64)
        mx = fmaxf(mx, __hip_atomic_load(mlp + 2 * p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    mx = wave_max(mx);
    float lsum = 0.f;
    float acc[X];
#pragma unroll
    for (int x = 0; x < X; x++) acc[x] = 0.f;
    for (int p0 = 0; p0 < np; p0 += 64) {
        const int p = p0 + lane;
        float w = 0.f;
        if (p < np) {
            const float m_p = __hip_atomic_load(mlp + 2 * p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const float l_p = __hip_atomic_load(mlp + 2 * p + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            w = m_p == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_p - mx);
            lsum = __builtin_fmaf(l_p, w, lsum);
        }
        const int cnt = min(64, np - p0);
        for (int q0 = 0; q0 < cnt; q0 += CH) {
            const float* src = a.ws_acc + (slot0 + p0 + q0) * D + lane;
            float v[CH][X];
#pragma unroll
            for (int q = 0; q < CH; q++)
#pragma unroll
                for (int x = 0; x < X; x++)
                    v[q][x] = (q0 + q < cnt) ? __hip_atomic_load(src + (long long)q * D + 64 * x,
                                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                             : 0.f;
#pragma unroll
            for (int q = 0; q < CH; q++) {
                const float wq = __shfl(w, q0 + q);
#pragma unroll
                for (int x = 0; x < X; x++) acc[x] = __builtin_fmaf(wq, v[q][x], acc[x]);
            }
        }
    }
    lsum = wave_sum(lsum);
    const float inv = 1.0f / lsum;
#pragma unroll
    for (int x = 0; x < X; x++) out[lane + 64 * x] = acc[x] * inv;
}

// ---------------------------------------------------------------- kernel

template <int D, int KVT, bool ALIGNED>
__global__ __launch_bounds__(256) void decode_kernel(DecodeArgs a) {
    constexpr int NC = D / 4;
    constexpr int DPL = D / 16;
    __shared__ floatx4 sm_acc[3][DPL][64];
    __shared__ float sm_m[4][16];
    __shared__ float sm_l[4][16];
    __shared__ int sm_last;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int j = lane & 15;
    const int kq = lane >> 4;
    const int kvh = blockIdx.y / a.n_hg;
    const int hg = blockIdx.y - kvh * a.n_hg;
    const int b = blockIdx.z;
    const int wgp = blockIdx.x;
    const int g_local = min(16, a.group - hg * 16);
    const int head0 = kvh * a.group + hg * 16;

    const Extent e = extent<ALIGNED>(a, b);
    if (e.np == 0) {  // nothing to attend to (ctx_len <= 0 or q_pos < 0): zeros
        if (wgp == 0)
            for (int i = threadIdx.x; i < g_local * D; i += 256)
                a.out[((long long)b * a.n_heads + head0) * D + i] = 0.f;
        return;
    }
    if (wgp >= e.np) return;  // uniform over the workgroup

    // Q operand (B of the QK product): head j, dims by qk_dim.
    float qv[NC];
    {
        const float* qrow = a.q + ((long long)b * a.n_heads + head0 + min(j, g_local - 1)) * D;
        const bool ok = j < g_local;
#pragma unroll
        for (int c = 0; c < NC; c++) qv[c] = ok ? qrow[qk_dim<D, KVT>(c, kq)] : 0.f;
    }

    State<D> st;
#pragma unroll
    for (int x = 0; x < DPL; x++) st.acc[x] = floatx4{0.f, 0.f, 0.f, 0.f};
    st.m = -INFINITY;
    st.l = 0.f;

    RowMap m;
    m.table = a.tables ? a.tables + (long long)b * a.table_stride : nullptr;
    m.block_stride = a.block_stride;
    m.head_stride = a.head_stride;
    m.token_stride = a.token_stride;
    m.bt_log2 = a.bt_log2;
    m.num_blocks = a.num_blocks;
    m.table_len = a.table_stride;

    const int per_part = 4 * a.tpw;
    if (ALIGNED && wgp < e.np_main) {
        const int first = wgp * per_part + wave * a.tpw;
        const int n = max(0, min(first + a.tpw, e.main_tiles) - first);
        AlignedWalk w;
        w.base = e.lo & ~15;
        w.lo = e.lo;
        w.hi = e.hi;
        w.head_off = (long long)kvh * a.head_stride;
        w.bi_first = (w.base + 16 * first) >> a.bt_log2;
        w.tblv = 0;
        if (a.tables && n > 0) {
            const int bi = w.bi_first + lane;
            const int bi_last = (w.base + 16 * (first + n) - 1) >> a.bt_log2;
            int blk = -1;
            if (bi <= bi_last && bi < a.table_stride) {
                blk = m.table[bi];
                if ((unsigned)blk >= (unsigned)a.num_blocks) blk = -1;
            }
            w.tblv = blk;
        }
        walk_tiles<D, KVT>(st, a, qv, n, j, kq, [&](int i, long long& ko, long long* vo) {
            return aligned_offsets<D, KVT>(a, w, first + i, j, kq, ko, vo);
        });
    } else {
        // gather: the explicit/virtual position list, or the aligned path's globals
        const bool globals = ALIGNED;
        const int vend = globals ? e.n_glob : e.L;
        const int first = globals ? wave : wgp * per_part + wave * a.tpw;
        const int step = globals ? 4 : 1;
        const int ntiles = (vend + 15) / 16;
        const int n = globals ? max(0, (ntiles - first + 3) / 4)
                              : max(0, min(first + a.tpw, ntiles) - first);
        walk_tiles<D, KVT>(st, a, qv, n, j, kq, [&](int i, long long& ko, long long* vo) {
            return gather_offsets<D, KVT>(a, e, m, b, kvh, 16 * (first + i * step), vend, globals,
                                          j, kq, ko, vo);
        });
    }

    // ---- merge the four wavefronts through LDS (wave 0 keeps the result)
    float lt = st.l + __shfl_xor(st.l, 16);
    lt += __shfl_xor(lt, 32);
    if (wave > 0) {
#pragma unroll
        for (int x = 0; x < DPL; x++) sm_acc[wave - 1][x][lane] = st.acc[x];
    }
    if (kq == 0) {
        sm_m[wave][j] = st.m;
        sm_l[wave][j] = lt;
    }
    __syncthreads();
    const int slot_base = ((b * a.n_kv_heads + kvh) * a.n_hg + hg);
    if (wave == 0) {
        float mh[4], lh[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int hh = 4 * kq + r;
            float M = fmaxf(fmaxf(sm_m[0][hh], sm_m[1][hh]), fmaxf(sm_m[2][hh], sm_m[3][hh]));
            float sw[4], L = 0.f;
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const float mw = sm_m[w][hh];
                sw[w] = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - M);
                L = __builtin_fmaf(sm_l[w][hh], sw[w], L);
            }
#pragma unroll
            for (int x = 0; x < DPL; x++) {
                float v = st.acc[x][r] * sw[0];
#pragma unroll
                for (int w = 1; w < 4; w++) v = __builtin_fmaf(sm_acc[w - 1][x][lane][r], sw[w], v);
                st.acc[x][r] = v;
            }
            mh[r] = M;
            lh[r] = L;
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int hh = 4 * kq + r;
            if (hh >= g_local) continue;
            const long long head = head0 + hh;
            if (e.np == 1) {
                const float inv = 1.0f / lh[r];
                float* o = a.out + ((long long)b * a.n_heads + head) * D + DPL * j;
#pragma unroll
                for (int x = 0; x < DPL / 4; x++)
                    *(float4*)(o + 4 * x) = float4{st.acc[4 * x + 0][r] * inv, st.acc[4 * x + 1][r] * inv,
                                                   st.acc[4 * x + 2][r] * inv, st.acc[4 * x + 3][r] * inv};
            } else {
                // device-coherent (write-through) stores: the merging workgroup
                // may run on another XCD, whose L2 does not see this one's
                const long long slot = ((long long)b * a.n_heads + head) * a.max_parts + wgp;
                float* o = a.ws_acc + slot * D + DPL * j;
#pragma unroll
                for (int x = 0; x < DPL; x++)
                    __hip_atomic_store(o + x, st.acc[x][r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (j == 0) {
                    float* ml = (float*)(a.ws_ml + slot);
                    __hip_atomic_store(ml, mh[r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(ml + 1, lh[r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
        if (e.np > 1) {
            // publish: the write-through stores complete before the arrival is
            // counted; the last workgroup to arrive merges
            __builtin_amdgcn_s_waitcnt(0);
            int old = 0;
            if (lane == 0)
                old = __hip_atomic_fetch_add(a.counters + slot_base, 1, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
            old = __shfl(old, 0);
            if (lane == 0) sm_last = (old == e.np - 1);
        }
    }
    if (e.np == 1) return;
    __syncthreads();
    if (!sm_last) return;
    for (int hh = wave; hh < g_local; hh += 4) {
        const long long head = head0 + hh;
        merge_head<D>(a, ((long long)b * a.n_heads + head) * a.max_parts, e.np,
                      a.out + ((long long)b * a.n_heads + head) * D, lane);
    }
    if (threadIdx.x == 0)
        __hip_atomic_store(a.counters + slot_base, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ void fill_zero_kernel(int* p, long long n) {
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n;
         i += (long long)gridDim.x * blockDim.x)
        p[i] = 0;
}

// ---------------------------------------------------------------- host side

static int g_tpw_override = 0;

// Tiles per wavefront per partition.  Enough workgroups to fill 256 CUs
// about four deep, each wavefront streaming as many 16-token tiles as that
// allows (at most 64, one block-table slice per lane), so the partial
// write-back and merge stay small next to the K/V bytes.
static int pick_tpw(int batch, int units, int max_len) {
    if (g_tpw_override > 0) return g_tpw_override;
    const long long tiles = (long long)batch * units * ((max_len + 15) / 16);
    const long long target_wg = 1024;
    int t = 1;
    while (t < 64 && 4LL * t * target_wg < tiles) t <<= 1;
    return t;
}

struct DecodePlan {
    DecodeArgs a;
    dim3 grid;
    size_t ws_bytes;
    int head_dim;
    int kvt;
    bool aligned;
    int batch;
};

static size_t ws_layout(int batch, int n_heads, int n_kv_heads, int n_hg, int head_dim,
                        int max_parts, size_t* ml_off, size_t* ctr_off) {
    if (max_parts <= 1) return 0;
    const size_t slots = (size_t)batch * n_heads * max_parts;
    size_t acc = (slots * head_dim * sizeof(float) + 255) & ~(size_t)255;
    size_t ml = (slots * sizeof(float2) + 255) & ~(size_t)255;
    size_t ctr = ((size_t)batch * n_kv_heads * n_hg * sizeof(int) + 255) & ~(size_t)255;
    if (ml_off) *ml_off = acc;
    if (ctr_off) *ctr_off = acc + ml;
    return acc + ml + ctr;
}

// max_main: host bound on the contiguous main range; globals: whether an
// extra partition of strided globals may exist.
static int plan_common(DecodePlan& pl, int batch, int n_heads, int n_kv_heads, int head_dim,
                       int kvt, int max_main, bool globals, bool aligned_path, float scale) {
    if (batch <= 0 || n_heads <= 0 || n_kv_heads <= 0)
        return set_error(NYION_ERR_INVALID, "decode: batch/heads must be positive");
    if (n_heads % n_kv_heads)
        return set_error(NYION_ERR_INVALID, "decode: n_heads %d not a multiple of n_kv_heads %d",
                         n_heads, n_kv_heads);
    if (head_dim != 64 && head_dim != 128)
        return set_error(NYION_ERR_UNSUPPORTED, "decode: head_dim %d (supported: 64, 128)", head_dim);
    if (kvt != NYION_KV_F32 && kvt != NYION_KV_Q4_20B)
        return set_error(NYION_ERR_INVALID, "decode: kv_dtype %d", kvt);
    if (max_main <= 0) return set_error(NYION_ERR_INVALID, "decode: max_ctx must be positive");
    if (batch > 65535) return set_error(NYION_ERR_UNSUPPORTED, "decode: batch %d > 65535", batch);
    DecodeArgs& a = pl.a;
    a = DecodeArgs{};
    a.n_heads = n_heads;
    a.n_kv_heads = n_kv_heads;
    a.group = n_heads / n_kv_heads;
    a.n_hg = (a.group + 15) / 16;
    if (n_kv_heads * a.n_hg > 65535) return set_error(NYION_ERR_UNSUPPORTED, "decode: too many heads");
    const float sc = scale > 0.f ? scale : 1.0f / sqrtf((float)head_dim);
    a.scale_log2 = sc * 1.4426950408889634f;
    // the gather path walks the globals too, so its bound includes them
    const int max_len = aligned_path ? max_main : max_main + (globals ? 128 : 0);
    a.max_len = max_main;
    a.tpw = pick_tpw(batch, n_kv_heads * a.n_hg, max_len);
    const int per_part = 4 * a.tpw;
    const int tiles = (max_len + 15) / 16 + (aligned_path ? 1 : 0);
    a.max_parts = (tiles + per_part - 1) / per_part + (aligned_path && globals ? 1 : 0);
    pl.head_dim = head_dim;
    pl.kvt = kvt;
    pl.aligned = aligned_path;
    pl.batch = batch;
    pl.grid = dim3(a.max_parts, n_kv_heads * a.n_hg, batch);
    pl.ws_bytes = ws_layout(batch, n_heads, n_kv_heads, a.n_hg, head_dim, a.max_parts, nullptr, nullptr);
    return NYION_OK;
}

static int attach_workspace(DecodePlan& pl, void* ws, size_t ws_bytes) {
    if (pl.ws_bytes == 0) return NYION_OK;
    if (!ws || ws_bytes < pl.ws_bytes)
        return set_error(NYION_ERR_WORKSPACE, "decode: workspace %zu bytes < required %zu", ws_bytes,
                         pl.ws_bytes);
    if (!aligned(ws, 256)) return set_error(NYION_ERR_INVALID, "decode: workspace not 256-byte aligned");
    size_t ml_off = 0, ctr_off = 0;
    ws_layout(pl.batch, pl.a.n_heads, pl.a.n_kv_heads, pl.a.n_hg, pl.head_dim, pl.a.max_parts, &ml_off,
              &ctr_off);
    pl.a.ws_acc = (float*)ws;
    pl.a.ws_ml = (float2*)((char*)ws + ml_off);
    pl.a.counters = (int*)((char*)ws + ctr_off);
    return NYION_OK;
}

template <int D, int KVT>
static void launch_dk(const DecodePlan& pl, hipStream_t stream) {
    if (pl.aligned)
        hipLaunchKernelGGL((decode_kernel<D, KVT, true>), pl.grid, dim3(256), 0, stream, pl.a);
    else
        hipLaunchKernelGGL((decode_kernel<D, KVT, false>), pl.grid, dim3(256), 0, stream, pl.a);
}

static int launch_plan(const DecodePlan& pl, hipStream_t stream) {
    if (pl.head_dim == 64 && pl.kvt == NYION_KV_F32)
        launch_dk<64, NYION_KV_F32>(pl, stream);
    else if (pl.head_dim == 64)
        launch_dk<64, NYION_KV_Q4_20B>(pl, stream);
    else if (pl.kvt == NYION_KV_F32)
        launch_dk<128, NYION_KV_F32>(pl, stream);
    else
        launch_dk<128, NYION_KV_Q4_20B>(pl, stream);
    return check_launch("decode");
}

static long long row_elems(int head_dim, int kvt) {
    return kvt == NYION_KV_F32 ? head_dim : q4_row_bytes(head_dim);
}

static int check_pool_ptrs(const void* k, const void* v, int kvt) {
    if (!k || !v) return set_error(NYION_ERR_INVALID, "decode: null K/V pool");
    const size_t al = kvt == NYION_KV_F32 ? 16 : 4;
    if (!aligned(k, al) || !aligned(v, al))
        return set_error(NYION_ERR_INVALID, "decode: K/V pools must be %zu-byte aligned", al);
    return NYION_OK;
}

static int window_main_len(int max_ctx, int window) {
    if (window <= 0) return max_ctx;
    return (int)((long long)window + 1 < max_ctx ? (long long)window + 1 : max_ctx);
}

}  // namespace nyion

using namespace nyion;

extern "C" {

int nyion_set_decode_partition_tokens(int tokens) {
    if (tokens != 0 && (tokens < 64 || tokens > 4096 || !is_pow2(tokens)))
        return set_error(NYION_ERR_INVALID,
                         "partition tokens %d: power of two in [64, 4096] (4 wavefronts x 16-token "
                         "tiles) or 0", tokens);
    g_tpw_override = tokens / 64;
    return NYION_OK;
}

int nyion_get_decode_partition_tokens(int batch, int n_kv_heads, int head_dim, int max_len) {
    (void)head_dim;
    return 64 * pick_tpw(batch, n_kv_heads, max_len);
}

size_t nyion_paged_decode_workspace_size(int batch, int n_heads, int n_kv_heads, int head_dim,
                                         int max_ctx, int window, int global_stride) {
    DecodePlan pl;
    if (plan_common(pl, batch, n_heads, n_kv_heads, head_dim, NYION_KV_F32,
                    window_main_len(max_ctx, window), window > 0 && global_stride > 0, true,
                    0.f) != NYION_OK)
        return 0;
    // the gather path (block_tokens < 16) may need more partitions
    DecodePlan pg;
    if (plan_common(pg, batch, n_heads, n_kv_heads, head_dim, NYION_KV_F32,
                    window_main_len(max_ctx, window), window > 0 && global_stride > 0, false,
                    0.f) != NYION_OK)
        return 0;
    return pl.ws_bytes > pg.ws_bytes ? pl.ws_bytes : pg.ws_bytes;
}

int nyion_decode_workspace_init(void* d_workspace, size_t workspace_bytes, nyion_stream_t stream) {
    clear_error();
    int rc;
    if ((rc = require_device()) != NYION_OK) return rc;
    if (!d_workspace || workspace_bytes == 0) return NYION_OK;
    if (!aligned(d_workspace, 4)) return set_error(NYION_ERR_INVALID, "workspace init: alignment");
    const long long n = (long long)(workspace_bytes / sizeof(int));
    long long g = (n + 255) / 256;
    if (g > 4096) g = 4096;
    hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)g), dim3(256), 0, (hipStream_t)stream,
                       (int*)d_workspace, n);
    return check_launch("workspace init");
}

int nyion_paged_decode_attention(const float* d_q, const void* k_pool, const void* v_pool,
                                 const int32_t* block_tables, int max_blocks_per_seq,
                                 const int32_t* ctx_lens, const int32_t* q_pos, int batch,
                                 int n_heads, int n_kv_heads, int head_dim, int block_tokens,
                                 int num_blocks, int kv_dtype, int window, int global_stride,
                                 int max_ctx, float scale, float* d_out, void* d_workspace,
                                 size_t workspace_bytes, nyion_stream_t stream) {
    clear_error();
    int rc;
    if ((rc = require_device()) != NYION_OK) return rc;
    if (!d_q || !d_out || !block_tables || !ctx_lens)
        return set_error(NYION_ERR_INVALID, "paged decode: null q/out/block_tables/ctx_lens");
    if (!aligned(d_q, 16) || !aligned(d_out, 16))
        return set_error(NYION_ERR_INVALID, "paged decode: q/out must be 16-byte aligned");
    if ((rc = check_pool_ptrs(k_pool, v_pool, kv_dtype)) != NYION_OK) return rc;
    if (!is_pow2(block_tokens) || block_tokens > (1 << 20))
        return set_error(NYION_ERR_INVALID, "paged decode: block_tokens %d not a power of two",
                         block_tokens);
    if (num_blocks <= 0 || max_blocks_per_seq <= 0)
        return set_error(NYION_ERR_INVALID, "paged decode: num_blocks/max_blocks_per_seq");
    if (max_ctx <= 0 || (long long)max_ctx > (long long)max_blocks_per_seq * block_tokens)
        return set_error(NYION_ERR_INVALID,
                         "paged decode: max_ctx %d must be in [1, max_blocks_per_seq*block_tokens]",
                         max_ctx);
    const bool aligned_path = block_tokens >= 16;
    DecodePlan pl;
    if ((rc = plan_common(pl, batch, n_heads, n_kv_heads, head_dim, kv_dtype,
                          window_main_len(max_ctx, window), window > 0 && global_stride > 0,
                          aligned_path, scale)) != NYION_OK)
        return rc;
    if ((rc = attach_workspace(pl, d_workspace, workspace_bytes)) != NYION_OK) return rc;
    DecodeArgs& a = pl.a;
    const long long row = row_elems(head_dim, kv_dtype);
    a.q = d_q;
    a.k = k_pool;
    a.v = v_pool;
    a.tables = block_tables;
    a.table_stride = max_blocks_per_seq;
    a.ctx_lens = ctx_lens;
    a.q_pos = q_pos;
    a.out = d_out;
    a.token_stride = (int)row;
    a.head_stride = (long long)block_tokens * row;
    a.block_stride = (long long)n_kv_heads * block_tokens * row;
    a.bt_log2 = ilog2(block_tokens);
    a.num_blocks = num_blocks;
    a.mode = window > 0 ? MODE_WINDOW : MODE_FULL;
    a.window = window;
    a.global_stride = global_stride;
    return launch_plan(pl, (hipStream_t)stream);
}

size_t nyion_paged_decode_positions_workspace_size(int batch, int n_heads, int n_kv_heads,
                                                   int head_dim, int max_positions) {
    DecodePlan pl;
    if (plan_common(pl, batch, n_heads, n_kv_heads, head_dim, NYION_KV_F32, max_positions, false,
                    false, 0.f) != NYION_OK)
        return 0;
    return pl.ws_bytes;
}

int nyion_paged_decode_attention_positions(
    const float* d_q, const void* k_pool, const void* v_pool, const int32_t* block_tables,
    int max_blocks_per_seq, const int32_t* positions, const int32_t* n_positions, int max_positions,
    int batch, int n_heads, int n_kv_heads, int head_dim, int block_tokens, int num_blocks,
    int kv_dtype, float scale, float* d_out, void* d_workspace, size_t workspace_bytes,
    nyion_stream_t stream) {
    clear_error();
    int rc;
    if ((rc = require_device()) != NYION_OK) return rc;
    if (!d_q || !d_out || !block_tables || !positions || !n_positions)
        return set_error(NYION_ERR_INVALID, "positions decode: null argument");
    if (!aligned(d_q, 16) || !aligned(d_out, 16))
        return set_error(NYION_ERR_INVALID, "positions decode: q/out must be 16-byte aligned");
    if ((rc = check_pool_ptrs(k_pool, v_pool, kv_dtype)) != NYION_OK) return rc;
    if (!is_pow2(block_tokens) || block_tokens > (1 << 20))
        return set_error(NYION_ERR_INVALID, "positions decode: block_tokens %d not a power of two",
                         block_tokens);
    if (num_blocks <= 0 || max_blocks_per_seq <= 0 || max_positions <= 0)
        return set_error(NYION_ERR_INVALID, "positions decode: sizes must be positive");
    DecodePlan pl;
    if ((rc = plan_common(pl, batch, n_heads, n_kv_heads, head_dim, kv_dtype, max_positions, false,
                          false, scale)) != NYION_OK)
        return rc;
    if ((rc = attach_workspace(pl, d_workspace, workspace_bytes)) != NYION_OK) return rc;
    DecodeArgs& a = pl.a;
    const long long row = row_elems(head_dim, kv_dtype);
    a.q = d_q;
    a.k = k_pool;
    a.v = v_pool;
    a.tables = block_tables;
    a.table_stride = max_blocks_per_seq;
    a.positions = positions;
    a.n_pos = n_positions;
    a.pos_stride = max_positions;
    a.out = d_out;
    a.token_stride = (int)row;
    a.head_stride = (long long)block_tokens * row;
    a.block_stride = (long long)n_kv_heads * block_tokens * row;
    a.bt_log2 = ilog2(block_tokens);
    a.num_blocks = num_blocks;
    a.mode = MODE_LIST;
    return launch_plan(pl, (hipStream_t)stream);
}

int nyion_attention_node(const float* d_q, const void* d_k, const void* d_v, float* d_scores,
                         float* d_out, uint32_t n_heads, uint32_t n_kv_heads, uint32_t seq_len,
                         uint32_t head_dim, uint32_t kv_stride, int kv_dtype,
                         nyion_stream_t stream) {
    clear_error();
    int rc;
    if ((rc = require_device()) != NYION_OK) return rc;
    if (!d_q || !d_out) return set_error(NYION_ERR_INVALID, "attention node: null q/out");
    if (!aligned(d_q, 16) || !aligned(d_out, 16))
        return set_error(NYION_ERR_INVALID, "attention node: q/out must be 16-byte aligned");
    if ((rc = check_pool_ptrs(d_k, d_v, kv_dtype)) != NYION_OK) return rc;
    if (seq_len == 0 || seq_len > kv_stride || kv_stride > (1u << 30))
        return set_error(NYION_ERR_INVALID, "attention node: need 0 < seq_len (%u) <= kv_stride (%u)",
                         seq_len, kv_stride);
    if (n_heads > 4096 || n_kv_heads == 0)
        return set_error(NYION_ERR_INVALID, "attention node: head counts");
    DecodePlan pl;
    if ((rc = plan_common(pl, 1, (int)n_heads, (int)n_kv_heads, (int)head_dim, kv_dtype,
                          (int)seq_len, false, true, 0.f)) != NYION_OK)
        return rc;
    // The node's scores buffer (n_heads*kv_stride floats, the reference's
    // ScratchBuffers::d_scores) holds the split-K partials; without it, or
    // when it is too small, use longer partitions until one workgroup covers
    // the sequence.
    DecodeArgs& a = pl.a;
    const size_t scores_bytes =
        d_scores && aligned(d_scores, 256) ? (size_t)n_heads * kv_stride * sizeof(float) : 0;
    while (pl.ws_bytes > scores_bytes) {
        a.tpw *= 2;
        const int per_part = 4 * a.tpw;
        const int tiles = ((int)seq_len + 15) / 16 + 1;
        a.max_parts = (tiles + per_part - 1) / per_part;
        pl.grid = dim3(a.max_parts, a.n_kv_heads * a.n_hg, 1);
        pl.ws_bytes = ws_layout(1, a.n_heads, a.n_kv_heads, a.n_hg, (int)head_dim, a.max_parts,
                                nullptr, nullptr);
    }
    if ((rc = attach_workspace(pl, d_scores, scores_bytes)) != NYION_OK) return rc;
    const long long row = row_elems((int)head_dim, kv_dtype);
    a.q = d_q;
    a.k = d_k;
    a.v = d_v;
    a.tables = nullptr;
    a.uniform_len = (int)seq_len;
    a.out = d_out;
    a.token_stride = (int)row;
    a.head_stride = (long long)kv_stride * row;
    a.block_stride = 0;
    a.bt_log2 = 30;
    a.num_blocks = 1;
    a.mode = MODE_FULL;
    if (pl.ws_bytes) {  // the scores buffer is caller scratch: clear the counters each call
        const long long n = (long long)a.n_kv_heads * a.n_hg;
        hipLaunchKernelGGL(fill_zero_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, a.counters, n);
        if ((rc = check_launch("attention node counters")) != NYION_OK) return rc;
    }
    return launch_plan(pl, (hipStream_t)stream);
}

int gpu_attention_streamed(const float* d_q, const float* d_k_cache, const float* d_v_cache,
                           float* d_output, int n_heads, int n_kv_heads, int seq_len, int head_dim,
                           int kv_stride, nyion_stream_t stream) {
    if (n_heads <= 0 || n_kv_heads <= 0 || seq_len <= 0 || head_dim <= 0 || kv_stride <= 0) {
        set_error(NYION_ERR_INVALID, "gpu_attention_streamed: non-positive size");
        return -1;
    }
    const int rc = nyion_attention_node(d_q, d_k_cache, d_v_cache, nullptr, d_output,
                                        (uint32_t)n_heads, (uint32_t)n_kv_heads, (uint32_t)seq_len,
                                        (uint32_t)head_dim, (uint32_t)kv_stride, NYION_KV_F32, stream);
    return rc == NYION_OK ? 0 : -1;
}

int gpu_attention_device(const float* d_q, const float* d_k_cache, const float* d_v_cache,
                         float* d_output, int n_heads, int n_kv_heads, int seq_len, int head_dim,
                         int kv_stride) {
    return gpu_attention_streamed(d_q, d_k_cache, d_v_cache, d_output, n_heads, n_kv_heads, seq_len,
                                  head_dim, kv_stride, nullptr);
}

}  // extern "C"
