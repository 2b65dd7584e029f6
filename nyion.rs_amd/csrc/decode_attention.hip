// decode_attention.hip — batched paged GQA decode attention for gfx950.
//
// One query token per sequence (the executor's decode step,
// swamp-engine/src/executor.rs:739-763).  Semantics follow ops::attention
// (swamp-engine/src/ops.rs:170-278) and ops::attention_sparse (ops.rs:85-168);
// the header states the position sets.
//
// Work decomposition (stream-K).  A segment is one (sequence, kv head, group
// of up to 16 q heads); its attended positions form a list of 16-token tiles.
// The segments' tile lists are laid end to end and a grid sized to the
// resident capacity of the chip cuts that list into equal ranges, one per
// 256-thread workgroup, whatever the spread of context lengths.  A workgroup
// walks its range segment by segment; its four wavefronts split each piece.
// All q heads of a GQA group are processed together, so each K/V byte is read
// from HBM once.
//
// Per 16-token tile a wavefront runs two MFMA chains on
// v_mfma_f32_16x16x4_f32 (fp32 in, fp32 accumulate):
//   S[16 tok][16 heads] = K_tile[16][D] . Q^T[D][16]       (D/4 MFMAs)
//   O[16 heads][D]     += P[16 heads][16 tok] . V_tile      (D/4 MFMAs)
// The MFMA output layout of S (lane = head + 16*token_quad, reg = token in
// quad) is exactly the A-operand layout P needs in the second product, so the
// probabilities never leave registers.  Binary16 rows use
// v_mfma_f32_16x16x16_f16 for both products instead: K as stored against q
// split into binary16 high and low parts, P rounded to binary16 against V as
// stored (a quarter of the f32 MFMA cycles; half the bytes per tile would
// otherwise leave the chain, not HBM, as the limit).
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
// Split-K.  The four wavefronts of a workgroup merge through LDS.  A segment
// covered by one workgroup is written out directly.  Otherwise each workgroup
// holding a piece of it writes one (m, l, O) partial to the workspace with
// device-coherent (write-through) stores, waits for them, and counts its
// arrival with an agent-scope atomic; the last one to arrive reads the
// partials with device-coherent loads, merges them with log-sum-exp, writes
// the output and resets the counter to 0.  Pieces of a segment are held by
// consecutive workgroups g, so partial slot g + segment is unique.  No L2
// write-back or invalidate is issued, and one decode call is one launch.
#include <float.h>
#include <math.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <type_traits>
#include <utility>

#include "common.hpp"

namespace nyion {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef _Float16 halfx2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 halfx4 __attribute__((ext_vector_type(4)));
typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));
// 16 bytes at 8-byte alignment (binary16 rows): one dwordx4 load
typedef uint32_t u32x4a __attribute__((ext_vector_type(4), aligned(8)));
typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));


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
    float* ws_acc;             // partial slot p: [p][16 heads][D]
    float2* ws_ml;             // [p][16 heads] = (m log2, l)
    int* counters;             // [segment], zero between calls
    float* scores;             // tracked decode: [B][Hq][scores_stride] scaled scores (log2)
    int scores_stride;         // >= attended positions + 2; the row ends hold (m, l)
    long long block_stride;
    long long head_stride;
    int table_stride;
    int pos_stride;
    int uniform_len;
    int batch;  // sequences of this launch (<= kMaxLaunchBatch)
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
    int max_len;    // host bound on attended positions per sequence
    float scale_log2;  // scale * log2(e)
    unsigned* status;  // the device's range-status word (binary16 q overflow)
    int direct;        // > 0: direct partition, pieces per segment (else stream-K)
    int seg_tiles;     // direct: host bound on the tiles of one segment
    int spec_len;      // window mode: the host's max_ctx, whose window start a
                       // walk's block-table loads may assume before the
                       // length arrives (0: none)
    // zone geometry (gather path): sequence b's page offsets at
    // page_bases + b * zone.n_pages; zone.page_base unused
    const int64_t* page_bases;
    ZoneMap zone;
    int decode_grid;   // workgroups of the decode itself (the launch may add more)
    // tracked decode, pipelined: the workgroups past decode_grid sum the
    // importance of the previous call's scores (same sequences and lengths),
    // imp_nx position blocks x imp_ny sequence strides over imp_batch sequences
    const float* imp_scores;
    double* imp_out;
    int imp_stride;
    int imp_nx, imp_ny, imp_batch;
};

// Sequences per launch: the per-sequence tile prefix sums live in LDS.
constexpr int kMaxLaunchBatch = 2048;

// Attended positions of one sequence.
//  aligned path (FULL/WINDOW, blocks >= 16 tokens): the contiguous range
//    [lo, hi] walked in 16-aligned tiles from lo & ~15 (main tiles), then
//    n_glob strided globals (stride*g) gathered 16 per tile;
//  gather path: L virtual positions (the same sets, or an explicit list).
struct Extent {
    int lo, hi, n_glob, L;
    int main_tiles;  // aligned: tiles over [lo & ~15, hi]
    int tiles;       // all tiles of one segment of this sequence
};

// len / qp / npos: the sequence's ctx_len, q_pos and list length as loaded.
template <bool ALIGNED>
__device__ __forceinline__ Extent seq_extent(const DecodeArgs& a, int len, int qp, int npos) {
    Extent e{0, -1, 0, 0, 0, 0};
    if (a.mode == MODE_LIST) {
        e.L = min(max(npos, 0), a.max_len);
    } else {
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
        e.tiles = e.main_tiles + (e.n_glob + 15) / 16;
    } else {
        e.tiles = (e.L + 15) / 16;
    }
    return e;
}

// The per-sequence values an extent needs: (ctx_len, q_pos), or the list
// length in MODE_LIST (as len).
__device__ __forceinline__ int2 seq_values(const DecodeArgs& a, int b) {
    if (a.mode == MODE_LIST) return int2{a.n_pos[b], 0};
    const int len = a.ctx_lens ? a.ctx_lens[b] : a.uniform_len;
    return int2{len, a.q_pos ? a.q_pos[b] : len - 1};
}

template <bool ALIGNED>
__device__ __forceinline__ Extent extent_of(const DecodeArgs& a, int2 v) {
    return a.mode == MODE_LIST ? seq_extent<ALIGNED>(a, 0, 0, v.x) : seq_extent<ALIGNED>(a, v.x, v.y, 0);
}

// Extent of sequence b as seen by one thread (no uniformity assumed).
template <bool ALIGNED>
__device__ __forceinline__ Extent lane_extent(const DecodeArgs& a, int b) {
    return extent_of<ALIGNED>(a, seq_values(a, b));
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
//   f16: value c = 8x+4e+y (binary16 MFMA 2x+e, element y) holds dim
//        32x + 8kq + 4e + y  (per x, the 4 quads of a row read 64 contiguous
//        bytes)
//   Q4 : per 32-element group g, the lane's four nibble bytes 4kq .. 4kq+3
//        (elements 8kq .. 8kq+7, element 2i in the low nibble of byte i) as
//        the eight values of a 16x16x32 binary16 MFMA: class a, elements
//        8kq + {0, 4, 2, 6}, then class b, elements 8kq + {1, 5, 3, 7}
//        (q_operand_q4)
// The Q operand uses the same map (qk_dim; q_operand_q4 for Q4).  V operand
// of lane (col j, quad kq), row 4kq+r: DPL = D/16 consecutive dims from
// DPL*j.
template <int D, int KVT>
__device__ __forceinline__ int qk_dim(int c, int kq) {
    if constexpr (KVT == NYION_KV_F16)
        return 32 * (c >> 3) + 8 * kq + 4 * ((c >> 2) & 1) + (c & 3);
    else
        return 16 * (c >> 2) + 4 * kq + (c & 3);  // f32 and Q4-20B
}

// Raw (undecoded) registers of one tile for one lane.
template <int D, int KVT>
struct Tile;

template <int D>
struct Tile<D, NYION_KV_F32> {
    floatx4 k[D / 16];        // K row j: dims 16x + 4kq .. +3
    floatx4 v[4][D / 64];     // V rows 4kq+r: dims DPL*j .. +DPL
};

template <int D>
struct Tile<D, NYION_KV_F16> {
    u32x4a k[D / 32];         // K row j: dims 32x + 8kq .. +7, eight binary16 values
    uint32_t v[4][D / 32];    // V rows 4kq+r: dims DPL*j .. +DPL-1, two per word
};

template <int D>
struct Tile<D, NYION_KV_Q4_20B> {
    uint32_t kn[D / 32];      // K row j, group g: nibble bytes 4kq .. 4kq+3
    uint32_t khdr;            // K row j, group kq % (D/32): f16 d | f16 dmin << 16
    uint32_t vhdr[4];
    uint32_t v[4];            // D/16 nibbles of V row 4kq+r (low 16 bits when D = 64)
};

// Loads are unconditional (an invalid row reads offset 0 of the pool, which is
// valid memory) so that the compiler keeps them in flight across the MFMA
// chain of the previous tile; invalid rows are masked when the tile is consumed.
template <int D, int KVT>
__device__ __forceinline__ void load_tile(Tile<D, KVT>& t, const void* kb, const void* vb,
                                          long long koff, const long long* voff, int j, int kq) {
    if constexpr (KVT == NYION_KV_F16) {
        const uint16_t* kr = (const uint16_t*)kb + koff;
#pragma unroll
        for (int x = 0; x < D / 32; x++)
            t.k[x] = __builtin_nontemporal_load((const u32x4a*)(kr + 32 * x + 8 * kq));
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const uint16_t* vr = (const uint16_t*)vb + voff[r] + (D / 16) * j;
            if constexpr (D == 64) {
                const u32x2 w = __builtin_nontemporal_load((const u32x2*)vr);
                t.v[r][0] = w[0];
                t.v[r][1] = w[1];
            } else {
                const u32x4a w = __builtin_nontemporal_load((const u32x4a*)vr);
#pragma unroll
                for (int i = 0; i < 4; i++) t.v[r][i] = w[i];
            }
        }
    } else if constexpr (KVT == NYION_KV_F32) {
        const float* kr = (const float*)kb + koff;
#pragma unroll
        for (int x = 0; x < D / 16; x++)
            t.k[x] = __builtin_nontemporal_load((const floatx4*)(kr + 16 * x + 4 * kq));
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float* vr = (const float*)vb + voff[r] + (D / 16) * j;
#pragma unroll
            for (int x = 0; x < D / 64; x++)
                t.v[r][x] = __builtin_nontemporal_load((const floatx4*)(vr + 4 * x));
        }
    } else {
        // K row j: nibble bytes 4kq .. 4kq+3 of every group; and the header
        // of group kq % (D/32) (lane 16g + i then holds row i's header of
        // group g)
        const uint8_t* kr = (const uint8_t*)kb + koff;
#pragma unroll
        for (int g = 0; g < D / 32; g++)
            t.kn[g] = __builtin_nontemporal_load((const uint32_t*)(kr + kQ4GroupBytes * g + 4 + 4 * kq));
        t.khdr = __builtin_nontemporal_load((const uint32_t*)(kr + kQ4GroupBytes * (kq % (D / 32))));
        const int ve0 = (D / 16) * j;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const uint8_t* vr = (const uint8_t*)vb + voff[r] + kQ4GroupBytes * (ve0 >> 5);
            t.vhdr[r] = __builtin_nontemporal_load((const uint32_t*)vr);
            const uint8_t* vn = vr + 4 + ((ve0 & 31) >> 1);
            if constexpr (D == 64)
                t.v[r] = (uint32_t)__builtin_nontemporal_load((const uint16_t*)vn);
            else
                t.v[r] = __builtin_nontemporal_load((const uint32_t*)vn);
        }
    }
}

template <int D, int KVT>
__device__ __forceinline__ void decode_k(const Tile<D, KVT>& t, float* kv) {
#pragma unroll
    for (int x = 0; x < D / 16; x++) {
        kv[4 * x + 0] = t.k[x].x;
        kv[4 * x + 1] = t.k[x].y;
        kv[4 * x + 2] = t.k[x].z;
        kv[4 * x + 3] = t.k[x].w;
    }
}

template <int D, int KVT>
__device__ __forceinline__ void decode_v(const Tile<D, KVT>& t, int r, float* vv) {
#pragma unroll
    for (int x = 0; x < D / 64; x++) {
        vv[4 * x + 0] = t.v[r][x].x;
        vv[4 * x + 1] = t.v[r][x].y;
        vv[4 * x + 2] = t.v[r][x].z;
        vv[4 * x + 3] = t.v[r][x].w;
    }
}

// Running state of one wavefront: O (reg r of acc[t] = head 4kq+r, dim
// DPL*j+t), per-head max (log2) and this lane's share of the denominator.
template <int D>
struct State {
    floatx4 acc[D / 16];
    floatx4 acc_m;  // Q4-20B: sum of p * dmin/32 (the same for every dim of a lane's column)
    float m;
    float l;
    // Q4-20B: 0x64006400 held in a register (opaque to the compiler), so that
    // mask-and-insert of the nibbles is one v_and_or_b32 (gfx9 VOP3 takes no
    // literal and one scalar operand)
    uint32_t k6464;
};

// Max over lanes l, l ^ 16, l ^ 32 and l ^ 48 (the four quads of one column)
// with gfx950's lane swaps: permlane16_swap(v, v) pairs each lane with its
// partner in the neighbouring row of 16, permlane32_swap(v, v) with its
// partner in the other half; no LDS round trip.
__device__ __forceinline__ float max_across_quads(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// max_across_quads with v_max_f32 applied to the swapped words as they are:
// fmaxf first quiets its operands (two canonicalising maxes per step, the
// lane swap's results not being known canonical); for scores, which hold
// no signalling NaN, the result is the same
__device__ __forceinline__ float max_across_quads_raw(float x) {
    auto vmax = [](uint32_t p, uint32_t q) {
        float r;
        asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(__uint_as_float(p)), "v"(__uint_as_float(q)));
        return r;
    };
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = vmax(a[0], a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return vmax(b[0], b[1]);
}

// Four values as binary16 (two words) and their binary16 residuals (two
// more): hi + lo carries 22 significant bits of each value.
__device__ __forceinline__ void pack_hi_lo(const float* v, float* w) {
    const halfx4 hi = {(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
    const halfx4 lo = {(_Float16)(v[0] - (float)hi[0]), (_Float16)(v[1] - (float)hi[1]),
                       (_Float16)(v[2] - (float)hi[2]), (_Float16)(v[3] - (float)hi[3])};
    const floatx2 hw = __builtin_bit_cast(floatx2, hi), lw = __builtin_bit_cast(floatx2, lo);
    w[0] = hw[0];
    w[1] = hw[1];
    w[2] = lw[0];
    w[3] = lw[1];
}

// Q operand of the Q4-20B QK product for lane (head j, quad kq), the B side
// of the K tile's 16x16x32 MFMAs (eight binary16 values per lane: class a,
// elements 32g + 8kq + {0, 4, 2, 6}, then class b, elements 32g + 8kq +
// {1, 5, 3, 7} divided by 16): per group g, words 8g .. 8g+3 = the eight
// values rounded to binary16, words 8g+4 .. 8g+7 = their binary16
// residuals; word D/4 + g = 2^-24 times the sum of the head's q over group
// g.  ok = false (a pad head) gives zeros.  Returns whether some |q| >=
// 65520, whose binary16 high part rounds to infinity.
template <int D>
__device__ __forceinline__ bool q_operand_q4(const float* qrow, bool ok, int kq, float* qv) {
    bool big = false;
#pragma unroll
    for (int g = 0; g < D / 32; g++) {
        const float4 z = {0.f, 0.f, 0.f, 0.f};
        const float4 u = ok ? *(const float4*)(qrow + 32 * g + 8 * kq) : z;
        const float4 w = ok ? *(const float4*)(qrow + 32 * g + 8 * kq + 4) : z;
        const float e[8] = {u.x, u.y, u.z, u.w, w.x, w.y, w.z, w.w};
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            sum += e[i];
            big |= fabsf(e[i]) >= 65520.f;
        }
        sum += __shfl_xor(sum, 16);
        sum += __shfl_xor(sum, 32);
        qv[D / 4 + g] = sum * 0x1p-24f;
        const float ca[4] = {e[0], e[4], e[2], e[6]};
        const float cb[4] = {e[1] * 0.0625f, e[5] * 0.0625f, e[3] * 0.0625f, e[7] * 0.0625f};
        float wa[4], wb[4];
        pack_hi_lo(ca, wa);
        pack_hi_lo(cb, wb);
        qv[8 * g + 0] = wa[0];
        qv[8 * g + 1] = wa[1];
        qv[8 * g + 2] = wb[0];
        qv[8 * g + 3] = wb[1];
        qv[8 * g + 4] = wa[2];
        qv[8 * g + 5] = wa[3];
        qv[8 * g + 6] = wb[2];
        qv[8 * g + 7] = wb[3];
    }
    return big;
}

// Headers of rows 4kq .. 4kq+3 of a gathered Q4-20B tile (khr[g][r]) come
// from the lanes that loaded them (lane 16g + i holds row i's header of
// group g) through a per-wavefront LDS slot [group][row]: one write and one
// 16-byte read per group.  The wavefront's LDS operations complete in order,
// so the slot needs no barrier.
template <int D>
__device__ __forceinline__ uint32_t (*q4_header_slot())[16] {
    __shared__ __attribute__((aligned(16))) uint32_t sm_khdr[4][D / 32][16];
    return sm_khdr[threadIdx.x >> 6];
}

template <int D>
__device__ __forceinline__ void q4_headers_put(const Tile<D, NYION_KV_Q4_20B>& t, int kq) {
    if (kq < D / 32) q4_header_slot<D>()[kq][threadIdx.x & 15] = t.khdr;
}

template <int D>
__device__ __forceinline__ void q4_headers_get(int kq, uint32_t (*khr)[4]) {
    uint32_t(*hs)[16] = q4_header_slot<D>();
#pragma unroll
    for (int g = 0; g < D / 32; g++) {
        const u32x4 h4 = *(const u32x4*)&hs[g][4 * kq];
#pragma unroll
        for (int r = 0; r < 4; r++) khr[g][r] = h4[r];
    }
}

// Rescale threshold of the online softmax, log2 units.  The running max of a
// head is only moved when a tile's max exceeds it by more than this, so
// exp2(s - m) <= 2^8 and the O rescale is rare after the first tiles.
constexpr float kRescaleLog2 = 8.0f;

// One 16x16x32 MFMA per group and q part: the lane's eight values are class
// a then class b (q_operand_q4 orders q the same way); sg[g] = nib.q of
// group g, scaled by 2^-24.
template <int D>
__device__ __forceinline__ void q4_tile_mfma(const Tile<D, NYION_KV_Q4_20B>& t, const float* qv, floatx4* sg) {
#pragma unroll
    for (int g = 0; g < D / 32; g++) {
        const uint32_t w = t.kn[g], w8 = w >> 8;
        const halfx8 kab = __builtin_bit_cast(
            halfx8, u32x4{w & 0x000f000fu, w8 & 0x000f000fu, w & 0x00f000f0u, w8 & 0x00f000f0u});
        const float* qg = qv + 8 * g;
        sg[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
            kab, __builtin_bit_cast(halfx8, floatx4{qg[0], qg[1], qg[2], qg[3]}), floatx4{0.f, 0.f, 0.f, 0.f},
            0, 0, 0);
        sg[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
            kab, __builtin_bit_cast(halfx8, floatx4{qg[4], qg[5], qg[6], qg[7]}), sg[g], 0, 0, 0);
    }
}

// Row r's score from the group products: fma(d, S_g, fma(dmin, qsum_g, acc))
// over g in order (khr[g][r]: the header of row 4kq+r, group g; qv[D/4 + g]:
// 2^-24 times head j's q summed over group g).  The four rows' chains are
// formed step by step side by side, so that consecutive FMAs do not depend
// on each other.
template <int D>
__device__ __forceinline__ floatx4 q4_tile_combine(const floatx4* sg, const float* qv, const uint32_t (*khr)[4]) {
    constexpr int NC = D / 4;
    floatx4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < D / 32; g++) {
#pragma unroll
        for (int r = 0; r < 4; r++) s[r] = __builtin_fmaf(f16_bits_to_f32(khr[g][r] >> 16), qv[NC + g], s[r]);
#pragma unroll
        for (int r = 0; r < 4; r++) s[r] = __builtin_fmaf(f16_bits_to_f32(khr[g][r]), sg[g][r], s[r]);
    }
    return s;
}

// S of one Q4-20B tile for lane (head j, quad kq): rows 4kq+r, scaled by
// 2^-24.  khr: the K headers of rows 4kq+r (null for a gathered tile:
// exchanged through LDS).
//
// k = d*nib + dmin per 32-element group g, so q.k = sum_g d*(nib.q)_g +
// dmin*sum(q_g): the nibbles are exact binary16 operands against q split
// into binary16 high and low parts (q_operand_q4; qv[D/4 + g] = 2^-24 times
// the sum of head j's q over group g), one accumulator per group, then each
// row's d and dmin (khr[g][r]: the header of row 4kq+r, group g).  A nibble
// masked in place is a binary16 denormal: bits e (elements 8kq + {0, 4, 2,
// 6}, class a) or 16e (elements 8kq + {1, 5, 3, 7}, class b, whose q carries
// 1/16), times 2^-24; the MFMA takes denormal inputs exactly, so the scores
// come out scaled by 2^-24 (undone with the softmax scale).  khr null (a
// gathered tile): the headers come from the lanes that loaded them, written
// to the exchange slot before the MFMAs and read after.
template <int D>
__device__ __forceinline__ floatx4 q4_tile_scores(const Tile<D, NYION_KV_Q4_20B>& t, const float* qv, int kq,
                                                  const uint32_t (*khr)[4]) {
    if (!khr) q4_headers_put<D>(t, kq);
    floatx4 sg[D / 32];
    q4_tile_mfma<D>(t, qv, sg);
    uint32_t hx[D / 32][4];
    if (!khr) {
        q4_headers_get<D>(kq, hx);
        khr = hx;
    }
    return q4_tile_combine<D>(sg, qv, khr);
}

// Log2-unit scores of one tile (masked rows -1e30); TRACK: stored into srow
// at positions pos[r] (rows 4kq+r of this lane's head).
template <int KVT, bool MASKED, bool TRACK>
__device__ __forceinline__ void tile_logits(const floatx4& s, float scale_log2, uint32_t mask, int kq,
                                            float* srow, const int* pos, float* sv) {
    // Q4-20B scores come out of the MFMAs scaled by 2^-24 (exact: a power of two)
    const float sc = KVT == NYION_KV_Q4_20B ? scale_log2 * 16777216.f : scale_log2;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        sv[r] = s[r] * sc;
        if (MASKED) sv[r] = ((mask >> (4 * kq + r)) & 1u) ? sv[r] : -1e30f;
    }
    if (TRACK && srow) {
        const uint32_t mq = (mask >> (4 * kq)) & 0xfu;
        if (mq == 0xfu && pos[3] == pos[0] + 3) {
            // four consecutive positions: one store (dword alignment suffices)
            typedef float floatx4u __attribute__((ext_vector_type(4), aligned(4)));
            *(floatx4u*)(srow + pos[0]) = floatx4u{sv[0], sv[1], sv[2], sv[3]};
        } else {
#pragma unroll
            for (int r = 0; r < 4; r++)
                if ((mq >> r) & 1u) srow[pos[r]] = sv[r];
        }
    }
}

// Online-softmax step over the lane's N scores (N / 4 tiles; score i is row
// 4kq + (i & 3) of its tile): the running max moves, with the O rescale, only
// when the scores' max exceeds it by more than kRescaleLog2 (wave-uniform;
// always on the first step).  pr = exp2(s - m) (Q4-20B: 32 exp2(s - m), the
// P.V operand, l accumulated in units of 32).
template <int D, int KVT, int N>
__device__ __forceinline__ void softmax_step(State<D>& st, const float* sv, int kq, float* pr) {
    constexpr int DPL = D / 16;
    float mx = sv[0];
#pragma unroll
    for (int i = 1; i < N; i++) mx = fmaxf(mx, sv[i]);
    const float mt = max_across_quads(mx);
    if (__any(mt > st.m + kRescaleLog2)) {
        const float mnew = fmaxf(st.m, mt);
        const float alpha = __builtin_amdgcn_exp2f(st.m - mnew);
        st.l *= alpha;
        st.m = mnew;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float ar = __shfl(alpha, 4 * kq + r);
#pragma unroll
            for (int x = 0; x < DPL; x++) st.acc[x][r] *= ar;
            if constexpr (KVT == NYION_KV_Q4_20B) st.acc_m[r] *= ar;
        }
    }
    const float mp = KVT == NYION_KV_Q4_20B ? st.m - 5.f : st.m;
#pragma unroll
    for (int i = 0; i < N; i++) pr[i] = __builtin_amdgcn_exp2f(sv[i] - mp);
    float ls = (pr[0] + pr[1]) + (pr[2] + pr[3]);
#pragma unroll
    for (int i = 4; i < N; i += 4) ls += (pr[i] + pr[i + 1]) + (pr[i + 2] + pr[i + 3]);
    st.l += ls;
}

// The online-softmax step of an unmasked, untracked pair of 4-bit tiles from
// their raw scores x (log2 units times 1/sc; sc > 0): the max is taken on x
// and scaled once (scaling by sc > 0 is monotonic, so max(x) * sc is the
// max of the scaled scores), and each weight is 32 exp2(x sc - m) with the
// scale and the shift in one FMA.  Otherwise as softmax_step.
template <int D, int N>
__device__ __forceinline__ void softmax_step_raw(State<D>& st, const float* x, float sc, int kq, float* pr) {
    constexpr int DPL = D / 16;
    float mx = x[0];
#pragma unroll
    for (int i = 1; i < N; i++) mx = fmaxf(mx, x[i]);
    const float mt = max_across_quads_raw(mx) * sc;
    if (__any(mt > st.m + kRescaleLog2)) {
        const float mnew = fmaxf(st.m, mt);
        const float alpha = __builtin_amdgcn_exp2f(st.m - mnew);
        st.l *= alpha;
        st.m = mnew;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float ar = __shfl(alpha, 4 * kq + r);
#pragma unroll
            for (int xx = 0; xx < DPL; xx++) st.acc[xx][r] *= ar;
            st.acc_m[r] *= ar;
        }
    }
    const float nmp = 5.f - st.m;  // -(m - 5): weights in units of 1/32
#pragma unroll
    for (int i = 0; i < N; i++) pr[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(x[i], sc, nmp));
    float ls = (pr[0] + pr[1]) + (pr[2] + pr[3]);
#pragma unroll
    for (int i = 4; i < N; i += 4) ls += (pr[i] + pr[i + 1]) + (pr[i + 2] + pr[i + 3]);
    st.l += ls;
}

// B operands of one Q4-20B tile's P.V product for lane (col j, quad kq):
// v/32 = (d/32) nib + dmin/32 as three exact binary16 terms: hi = (d/32) nib
// rounded, lo = fma(d/32, nib, -hi) (exact: the product has at most 15
// significant bits), and dmin/32, whose product with P is the same for every
// element of the lane's column (acc_m).  d/32 and dmin/32 are exact for |d|,
// |dmin| >= 2^-9 (below, the scaled header rounds by at most 2^-25), and
// d/32 * 15 stays inside binary16 range.  Words hold rows (0, 1) and (2, 3):
// hi[z], lo[z] for output dim DPL*j + z, mm the dmin/32 terms.
template <int D>
struct Q4VOperands {
    uint32_t hi[D / 16][2], lo[D / 16][2], mm[2];
};

template <int D, bool MASKED>
__device__ __forceinline__ Q4VOperands<D> q4_v_operands(const Tile<D, NYION_KV_Q4_20B>& t, uint32_t mask,
                                                        int kq, uint32_t k6464) {
    constexpr int DPL = D / 16;
    Q4VOperands<D> o;
    const halfx2 s32 = {(_Float16)0.03125f, (_Float16)0.03125f};
    uint32_t d01 = __builtin_amdgcn_perm(t.vhdr[1], t.vhdr[0], 0x05040100u);
    uint32_t d23 = __builtin_amdgcn_perm(t.vhdr[3], t.vhdr[2], 0x05040100u);
    uint32_t m01 = __builtin_amdgcn_perm(t.vhdr[1], t.vhdr[0], 0x07060302u);
    uint32_t m23 = __builtin_amdgcn_perm(t.vhdr[3], t.vhdr[2], 0x07060302u);
    if (MASKED) {  // masked rows may hold uninitialised slots: their terms are 0
        const uint32_t q = (mask >> (4 * kq)) & 0xfu;
        const uint32_t k01 = ((q & 1u) ? 0xffffu : 0u) | ((q & 2u) ? 0xffff0000u : 0u);
        const uint32_t k23 = ((q & 4u) ? 0xffffu : 0u) | ((q & 8u) ? 0xffff0000u : 0u);
        d01 &= k01;
        m01 &= k01;
        d23 &= k23;
        m23 &= k23;
    }
    const halfx2 dd01 = __builtin_bit_cast(halfx2, d01) * s32, dd23 = __builtin_bit_cast(halfx2, d23) * s32;
    o.mm[0] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(halfx2, m01) * s32);
    o.mm[1] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(halfx2, m23) * s32);
    // byte b of the nibble words of rows 2p and 2p+1 side by side, [row 2p
    // byte b, 0, row 2p+1 byte b, 0] (one permute per pair and byte): its low
    // nibbles are element 2b of the two rows and its high nibbles element
    // 2b + 1, each as binary16 1024 + e after a mask and 0x64 in the high
    // bytes (k6464)
    constexpr int NBY = DPL / 2;  // nibble bytes per row: 2 at head_dim 64, 4 at 128
    const halfx2 k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
    uint32_t pw[2][NBY];
#pragma unroll
    for (int p = 0; p < 2; p++)
#pragma unroll
        for (int b = 0; b < NBY; b++)
            pw[p][b] = __builtin_amdgcn_perm(t.v[2 * p + 1], t.v[2 * p], 0x0c000c00u | ((4u + b) << 16) | (uint32_t)b);
#pragma unroll
    for (int z = 0; z < DPL; z++) {  // element z: nibble z of the lane's word
        const int b = z >> 1;
        const uint32_t n01 = (((z & 1) ? pw[0][b] >> 4 : pw[0][b]) & 0x000f000fu) | k6464;
        const uint32_t n23 = (((z & 1) ? pw[1][b] >> 4 : pw[1][b]) & 0x000f000fu) | k6464;
        const halfx2 e01 = __builtin_bit_cast(halfx2, n01) - k1024;
        const halfx2 e23 = __builtin_bit_cast(halfx2, n23) - k1024;
        const halfx2 h01 = dd01 * e01, h23 = dd23 * e23;
        o.hi[z][0] = __builtin_bit_cast(uint32_t, h01);
        o.hi[z][1] = __builtin_bit_cast(uint32_t, h23);
        o.lo[z][0] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(dd01, e01, -h01));
        o.lo[z][1] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(dd23, e23, -h23));
    }
    return o;
}

// f32 and binary16 KV: one tile, scores through the online softmax to P.V.
template <int D, int KVT, bool MASKED, bool TRACK>
__device__ __forceinline__ void consume_tile_fh(State<D>& st, const Tile<D, KVT>& t, const float* qv,
                                             uint32_t mask, int kq, float scale_log2, float* srow,
                                             const int* pos) {
    constexpr int NC = D / 4;
    constexpr int DPL = D / 16;
    floatx4 s = {0.f, 0.f, 0.f, 0.f};
    if constexpr (KVT == NYION_KV_F16) {
        // binary16 K as stored against q split into binary16 high and low
        // parts (qv words 4x, 4x+1 and 4x+2, 4x+3): the products are exact in
        // f32, so S keeps f32 accuracy at a quarter of the f32 MFMA cycles.
        // Call x takes words 2(x&1), +1 of K load x/2 (dims 32(x/2) + 8kq +
        // 4(x&1) .. +3).  The words are copied to scalars first: this
        // compiler's __builtin_bit_cast of a vector element yields the bits
        // of element 0.
#pragma unroll
        for (int x = 0; x < D / 16; x++) {
            const uint32_t k0 = t.k[x >> 1][2 * (x & 1)], k1 = t.k[x >> 1][2 * (x & 1) + 1];
            const halfx4 kx = __builtin_bit_cast(halfx4, u32x2{k0, k1});
            const halfx4 qh = __builtin_bit_cast(halfx4, floatx2{qv[4 * x], qv[4 * x + 1]});
            const halfx4 ql = __builtin_bit_cast(halfx4, floatx2{qv[4 * x + 2], qv[4 * x + 3]});
            s = __builtin_amdgcn_mfma_f32_16x16x16f16(kx, qh, s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_16x16x16f16(kx, ql, s, 0, 0, 0);
        }
    } else {
        float kv[NC];
        decode_k<D, KVT>(t, kv);
#pragma unroll
        for (int c = 0; c < NC; c++) s = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[c], qv[c], s, 0, 0, 0);
    }

    const float sc = scale_log2;
    float sv[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        sv[r] = s[r] * sc;
        if (MASKED) sv[r] = ((mask >> (4 * kq + r)) & 1u) ? sv[r] : -1e30f;
    }
    if (TRACK && srow) {
        const uint32_t mq = (mask >> (4 * kq)) & 0xfu;
        if (mq == 0xfu && pos[3] == pos[0] + 3) {
            // four consecutive positions: one store (dword alignment suffices)
            typedef float floatx4u __attribute__((ext_vector_type(4), aligned(4)));
            *(floatx4u*)(srow + pos[0]) = floatx4u{sv[0], sv[1], sv[2], sv[3]};
        } else {
#pragma unroll
            for (int r = 0; r < 4; r++)
                if ((mq >> r) & 1u) srow[pos[r]] = sv[r];
        }
    }
    const float mt = max_across_quads(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])));
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
    if constexpr (KVT == NYION_KV_F16) {
        // O += P.V on binary16 MFMAs: A = this lane's four p (tokens 4kq..+3
        // of head j), rounded to binary16 (relative error <= 2^-12, p <= 2^8);
        // B of output dim DPL*j + z = the four rows' value of that dim, one
        // 16-bit half of each row's word (z/2)
        const halfx4 pa = {(_Float16)pr[0], (_Float16)pr[1], (_Float16)pr[2], (_Float16)pr[3]};
        uint32_t vw[4][DPL / 2];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const bool ok = !MASKED || ((mask >> (4 * kq + r)) & 1u);
#pragma unroll
            for (int w = 0; w < DPL / 2; w++)
                vw[r][w] = ok ? t.v[r][w] : 0u;  // masked rows may hold uninitialised slots
        }
#pragma unroll
        for (int z = 0; z < DPL; z++) {
            const int w = z >> 1;
            const uint32_t b01 = (z & 1) ? (vw[0][w] >> 16) | (vw[1][w] & 0xffff0000u)
                                         : (vw[0][w] & 0xffffu) | (vw[1][w] << 16);
            const uint32_t b23 = (z & 1) ? (vw[2][w] >> 16) | (vw[3][w] & 0xffff0000u)
                                         : (vw[2][w] & 0xffffu) | (vw[3][w] << 16);
            st.acc[z] = __builtin_amdgcn_mfma_f32_16x16x16f16(
                pa, __builtin_bit_cast(halfx4, u32x2{b01, b23}), st.acc[z], 0, 0, 0);
        }
    } else {
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
}

// One tile: bit i of `mask` (wave-uniform) marks row i of the 16 valid;
// MASKED = false is the all-valid fast path.  TRACK: also store the scaled
// scores of this lane's head (rows 4kq+r, at positions pos[r]) into srow.
template <int D, int KVT, bool MASKED, bool TRACK>
__device__ __forceinline__ void consume_tile(State<D>& st, const Tile<D, KVT>& t, const float* qv,
                                             uint32_t mask, int kq, float scale_log2, float* srow,
                                             const int* pos, const uint32_t (*khr)[4]) {
    constexpr int DPL = D / 16;
    if constexpr (KVT != NYION_KV_Q4_20B) {
        consume_tile_fh<D, KVT, MASKED, TRACK>(st, t, qv, mask, kq, scale_log2, srow, pos);
    } else {
        float sv[4], pr[4];
        tile_logits<KVT, MASKED, TRACK>(q4_tile_scores<D>(t, qv, kq, khr), scale_log2, mask, kq, srow, pos, sv);
        softmax_step<D, KVT, 4>(st, sv, kq, pr);
        // O += P.V on binary16 MFMAs: A = 32p rounded to binary16 (pr is 32p;
        // as for binary16 KV; 32p <= 2^13), B = V/32 as q4_v_operands (V
        // dequantised exactly as dequant_block, then scaled by 2^-5, which is
        // exact and keeps d*15 + dmin <= 2^20 inside binary16 range)
        const halfx4 pa = {(_Float16)pr[0], (_Float16)pr[1], (_Float16)pr[2], (_Float16)pr[3]};
        const Q4VOperands<D> o = q4_v_operands<D, MASKED>(t, mask, kq, st.k6464);
        st.acc_m = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, __builtin_bit_cast(halfx4, u32x2{o.mm[0], o.mm[1]}),
                                                         st.acc_m, 0, 0, 0);
#pragma unroll
        for (int z = 0; z < DPL; z++) {
            st.acc[z] = __builtin_amdgcn_mfma_f32_16x16x16f16(
                pa, __builtin_bit_cast(halfx4, u32x2{o.hi[z][0], o.hi[z][1]}), st.acc[z], 0, 0, 0);
            st.acc[z] = __builtin_amdgcn_mfma_f32_16x16x16f16(
                pa, __builtin_bit_cast(halfx4, u32x2{o.lo[z][0], o.lo[z][1]}), st.acc[z], 0, 0, 0);
        }
    }
}

template <int D, int KVT, bool TRACK>
__device__ __forceinline__ void consume(State<D>& st, const Tile<D, KVT>& t, const float* qv,
                                        uint32_t mask, int kq, float scale_log2, float* srow,
                                        const int* pos, const uint32_t (*khr)[4] = nullptr) {
    if (mask == 0xffffu)
        consume_tile<D, KVT, false, TRACK>(st, t, qv, mask, kq, scale_log2, srow, pos, khr);
    else if (mask)
        consume_tile<D, KVT, true, TRACK>(st, t, qv, mask, kq, scale_log2, srow, pos, khr);
}

// Two consecutive Q4-20B tiles as one 32-token step: one max reduction and
// rescale check, and P.V on 16x16x32 MFMAs whose eight values per lane are
// the lane's four rows of tile a then of tile b (the same order for P and
// V).  Masks as consume_tile (a tile past the walk has mask 0).
template <int D, bool MASKED, bool TRACK>
__device__ __forceinline__ void consume_pair_tiles(State<D>& st, const Tile<D, NYION_KV_Q4_20B>& ta,
                                                   const Tile<D, NYION_KV_Q4_20B>& tb, const float* qv,
                                                   uint32_t ma, uint32_t mb, int kq, float scale_log2,
                                                   float* srow, const int* pa_pos, const int* pb_pos,
                                                   const uint32_t (*khra)[4], const uint32_t (*khrb)[4]) {
    constexpr int KVT = NYION_KV_Q4_20B;
    constexpr int DPL = D / 16;
    float sv[8], pr[8];
    // both tiles' MFMAs before either combine (span tiles: headers in khr)
    floatx4 sga[D / 32], sgb[D / 32];
    // the scores through the softmax at raised issue priority: of two
    // wavefronts on a SIMD, the one in this stretch of MFMAs, exchanges and
    // exponentials goes first while the other builds V operands and runs
    // its P.V products (64 sequences of 512-32768 tokens: 115.5 -> 110.0 us;
    // 8 windows of 4096 tokens, one wavefront per SIMD: 14.8 -> 15.0 us)
    __builtin_amdgcn_s_setprio(1);
    q4_tile_mfma<D>(ta, qv, sga);
    q4_tile_mfma<D>(tb, qv, sgb);
    const floatx4 xa = q4_tile_combine<D>(sga, qv, khra), xb = q4_tile_combine<D>(sgb, qv, khrb);
    if constexpr (!MASKED && !TRACK) {
        // the scores come out of the MFMAs scaled by 2^-24 (exact)
        const float x[8] = {xa[0], xa[1], xa[2], xa[3], xb[0], xb[1], xb[2], xb[3]};
        softmax_step_raw<D, 8>(st, x, scale_log2 * 16777216.f, kq, pr);
    } else {
        tile_logits<KVT, MASKED, TRACK>(xa, scale_log2, ma, kq, srow, pa_pos, sv);
        tile_logits<KVT, MASKED, TRACK>(xb, scale_log2, mb, kq, srow, pb_pos, sv + 4);
        softmax_step<D, KVT, 8>(st, sv, kq, pr);
    }
    const halfx8 pa = {(_Float16)pr[0], (_Float16)pr[1], (_Float16)pr[2], (_Float16)pr[3],
                       (_Float16)pr[4], (_Float16)pr[5], (_Float16)pr[6], (_Float16)pr[7]};
    __builtin_amdgcn_s_setprio(0);
    const Q4VOperands<D> oa = q4_v_operands<D, MASKED>(ta, ma, kq, st.k6464);
    const Q4VOperands<D> ob = q4_v_operands<D, MASKED>(tb, mb, kq, st.k6464);
    st.acc_m = __builtin_amdgcn_mfma_f32_16x16x32_f16(
        pa, __builtin_bit_cast(halfx8, u32x4{oa.mm[0], oa.mm[1], ob.mm[0], ob.mm[1]}), st.acc_m, 0, 0, 0);
#pragma unroll
    for (int z = 0; z < DPL; z++) {
        st.acc[z] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
            pa, __builtin_bit_cast(halfx8, u32x4{oa.hi[z][0], oa.hi[z][1], ob.hi[z][0], ob.hi[z][1]}), st.acc[z],
            0, 0, 0);
        st.acc[z] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
            pa, __builtin_bit_cast(halfx8, u32x4{oa.lo[z][0], oa.lo[z][1], ob.lo[z][0], ob.lo[z][1]}), st.acc[z],
            0, 0, 0);
    }
}

// A Q4-20B tile of a contiguous walk (aligned blocks of >= 16 tokens, zone
// units of 32) at head_dim 64: its 16 K rows and its 16 V rows are each one
// span of 16 * 40 bytes, together 80 chunks of 16 bytes.  Lane l takes chunk
// l of K then V (lanes 0-39 the K chunks, 40-63 the first 24 V chunks) with
// one 16-byte load, and bytes 384 + 4l of the V span with one 4-byte load:
// five registers a tile, every byte loaded once.
template <int D>
struct SpanTile {
    static_assert(D == 64, "span tiles: head_dim 64");
    static constexpr int TS = q4_row_bytes(D);
    static constexpr int KCH = TS;                // 16-byte chunks of a span
    static constexpr int VTAIL = 16 * (64 - KCH);  // V bytes in the 16-byte loads
    u32x4a c;
    uint32_t w;
};

template <int D>
__device__ __forceinline__ void load_span(SpanTile<D>& t, const void* kb, const void* vb, long long base,
                                          int lane) {
    constexpr int KCH = SpanTile<D>::KCH, VTAIL = SpanTile<D>::VTAIL;
    const uint8_t* p = lane < KCH ? (const uint8_t*)kb + 16 * lane : (const uint8_t*)vb + 16 * (lane - KCH);
    t.c = __builtin_nontemporal_load((const u32x4a*)(p + base));
    t.w = __builtin_nontemporal_load((const uint32_t*)((const uint8_t*)vb + VTAIL + 4 * lane + base));
}

// Operands of a span tile: the chunks go to one of the wavefront's two LDS
// slots (rows at TS-byte strides, K then V), from which each lane reads the
// words the tile layout gives it (Tile<D, Q4-20B>: K row j's nibble words, V
// rows 4kq+r's header and nibbles) and the K headers of rows 4kq+r
// (khr[g][r]).  The wavefront's LDS operations complete in order: a later
// tile's writes to the slot come after these reads.
template <int D>
__device__ __forceinline__ void stage_span(const SpanTile<D>& sp, Tile<D, NYION_KV_Q4_20B>& t,
                                           uint32_t (*khr)[4], int j, int kq, int slot = 0) {
    constexpr int TS = SpanTile<D>::TS, DPL = D / 16;
    // K at bytes 0 .. 16 TS - 1 of the slot, V after it
    __shared__ u32x4 sm_span[4][2][2 * SpanTile<D>::KCH];
    const int lane = threadIdx.x & 63;
    u32x4* sb = sm_span[threadIdx.x >> 6][slot];
    sb[lane] = sp.c;                         // bytes 0 .. 1023: K, then V bytes 0 .. 383
    ((uint32_t*)(sb + 64))[lane] = sp.w;     // V bytes 384 + 4 lane
    const uint8_t* kr = (const uint8_t*)sb;
    const uint8_t* vr = kr + 16 * TS;
#pragma unroll
    for (int g = 0; g < D / 32; g++) {
        t.kn[g] = *(const uint32_t*)(kr + TS * j + kQ4GroupBytes * g + 4 + 4 * kq);
#pragma unroll
        for (int r = 0; r < 4; r++) khr[g][r] = *(const uint32_t*)(kr + TS * (4 * kq + r) + kQ4GroupBytes * g);
    }
    const int gv = (DPL * j) >> 5;                  // the group of the lane's V dims
    const int nv = 4 + (((DPL * j) & 31) >> 1);     // their first nibble byte in the group
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const uint8_t* row = vr + TS * (4 * kq + r) + kQ4GroupBytes * gv;
        t.vhdr[r] = *(const uint32_t*)row;
        t.v[r] = *(const uint16_t*)(row + nv);  // head_dim 64: four dims, two bytes
    }
}

// A run of an aligned walk: tiles of positions t0 .. t0+15 within one block;
// valid rows [lo, hi].  Lane l holds a 64-bit row offset, low word in tblv,
// high in tblh (-1: no rows): 4-bit paged walks, the first row of run tile l
// in this kv head; other paged walks, the first row of this kv head in the
// block of block index bi_first + l; ZONE, the blocks are 32-token units of
// zone pages (every zone page is a whole number of them, and a unit's rows
// of one (layer, kv head) are consecutive), the offset of row (layer, kv
// head 0) of unit bi_first + l.
struct AlignedWalk {
    int base;        // lo & ~15
    int lo, hi;
    int f;           // the run's first tile (tile t starts at base + 16 t)
    int ia, nint;    // tile tables: run tiles ia .. ia + nint - 1 are interior
                     // (16 valid rows, block present); 0 if any is absent
    int bi_first;    // block tables: the run's first block index (ZONE: unit)
    int tblv;        // lane l: low word of the row offset of run tile l (tile
    int tblh;        // tables) or of block bi_first + l; high word
    int kvh;         // ZONE: the kv head
    long long head_off;
};

constexpr int kZoneUnitLog2 = 5;  // zone walks: 32-token units

// Paged walks of 4-bit rows keep a lane table of tile row offsets (lane l:
// run tile l), so a tile's offset is one lane read and an interior tile's
// mask an index compare; f32 and binary16 walks keep a table of block row
// offsets (lane l: block bi_first + l), whose per-tile arithmetic is
// scalar work their tiles amortise (a tile table ran the f32 head_dim-64
// layer 1.5 % slower).
template <int KVT, bool ZONE>
constexpr bool tile_table() {
    return KVT == NYION_KV_Q4_20B && !ZONE;
}

// Offsets of run tile i (i < 64, wave-uniform) of an aligned walk.
template <int D, int KVT, bool ZONE = false>
__device__ __forceinline__ uint32_t aligned_offsets(const DecodeArgs& a, const AlignedWalk& w,
                                                    int i, int j, int kq, long long& koff,
                                                    long long* voff, int* pos) {
    const int t0 = w.base + 16 * (w.f + i);
#pragma unroll
    for (int r = 0; r < 4; r++) pos[r] = t0 + 4 * kq + r;
    auto edge_mask = [&]() -> uint32_t {
        const int vlo = max(w.lo - t0, 0);
        const int vhi = min(w.hi - t0, 15);
        return (vhi >= vlo) ? (((2u << vhi) - 1u) & ~((1u << vlo) - 1u)) : 0u;
    };
    // rows of a paged pool are contiguous: the token stride is the row size
    constexpr int TS = KVT == NYION_KV_Q4_20B ? q4_row_bytes(D) : D;
    uint32_t mask = 0xffffu;  // interior tiles: all valid
    long long base;
    if constexpr (ZONE) {
        if (__builtin_expect(t0 < w.lo || t0 + 15 > w.hi, 0)) mask = edge_mask();
        const int idx = (t0 >> kZoneUnitLog2) - w.bi_first;
        const long long row = ((long long)__builtin_amdgcn_readlane(w.tblh, idx) << 32) |
                              (uint32_t)__builtin_amdgcn_readlane(w.tblv, idx);
        const int lg = zone_pos(t0).page_log2;  // uniform: a tile lies in one page
        base = row + (long long)w.kvh * ((long long)TS << lg) + (long long)(t0 & 31) * TS;
        if (row < 0) {  // page absent, misaligned or outside the pool: the
            base = 0;   // loads read the pool's first rows (the host keeps at
            mask = 0;   // least 32), and the tile is masked
        }
    } else if constexpr (tile_table<KVT, ZONE>()) {
        // the tile's first row in this kv head, precomputed per run; the
        // edge tiles and runs with an absent block take the full test
        base = ((long long)__builtin_amdgcn_readlane(w.tblh, i) << 32) |
               (uint32_t)__builtin_amdgcn_readlane(w.tblv, i);
        if (__builtin_expect((unsigned)(i - w.ia) >= (unsigned)w.nint, 0)) {
            mask = edge_mask();
            if (base < 0) {  // block index past the table or block id out of range
                base = 0;
                mask = 0;
            }
        }
    } else {
        if (__builtin_expect(t0 < w.lo || t0 + 15 > w.hi, 0)) mask = edge_mask();
        // the block's first row of this kv head, precomputed per run
        const int idx = (t0 >> a.bt_log2) - w.bi_first;
        const long long row = ((long long)__builtin_amdgcn_readlane(w.tblh, idx) << 32) |
                              (uint32_t)__builtin_amdgcn_readlane(w.tblv, idx);
        base = row + (long long)(t0 & ((1 << a.bt_log2) - 1)) * TS;
        if (row < 0) {  // block index past the table or block id out of range
            base = 0;
            mask = 0;
        }
    }
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
                                                   long long& koff, long long* voff, int* pos) {
    auto pos_of = [&](int v) -> int {
        if (v >= vend) return -1;
        return globals ? v * a.global_stride : virt_to_pos(a, e, b, v);
    };
    auto off_of = [&](int p) -> long long { return p < 0 ? -1 : row_offset(m, p, kvh); };
    koff = off_of(pos_of(v0 + j));
    const uint32_t mask = (uint32_t)(__ballot(koff >= 0) & 0xffffu);
    koff = koff < 0 ? 0 : koff;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        pos[r] = pos_of(v0 + 4 * kq + r);
        const long long o = off_of(pos[r]);
        voff[r] = o < 0 ? 0 : o;
    }
    return mask;
}

// Block ids of the strided globals one wavefront gathers (virtual indices
// v0 .. v0 + 127; a sequence has at most 128), loaded in one batch so that
// each gathered tile costs one round trip instead of a table load followed
// by its row loads: lane l holds those of v0 + l and v0 + 64 + l, -1 past the
// list, past the table or outside [0, num_blocks) (row_offset's rules).
struct GlobalBlocks {
    int b[2];
};

__device__ __forceinline__ GlobalBlocks load_global_blocks(const DecodeArgs& a, const Extent& e,
                                                           const RowMap& m, int v0, int lane) {
    GlobalBlocks g;
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const int v = v0 + 64 * k + lane;
        int blk = -1;
        if (v < e.n_glob) {
            const int t = v * a.global_stride;
            if (!m.table) {
                blk = 0;
            } else if ((t >> m.bt_log2) < m.table_len) {
                blk = m.table[t >> m.bt_log2];
                if ((unsigned)blk >= (unsigned)m.num_blocks) blk = -1;
            }
        }
        g.b[k] = blk;
    }
    return g;
}

// Offsets of gathered global tile i (virtual indices v0 + 16i .. +15, i < 8)
// from the preloaded block ids: the same rows, positions and mask as
// gather_offsets with globals = true.  Invalid rows point at offset 0 and are
// masked.
__device__ __forceinline__ uint32_t global_offsets(const DecodeArgs& a, const Extent& e,
                                                   const RowMap& m, const GlobalBlocks& g, int kvh,
                                                   int v0, int i, int j, int kq, long long& koff,
                                                   long long* voff, int* pos) {
    const int src = i < 4 ? g.b[0] : g.b[1];  // i is wave-uniform
    auto row = [&](int rel, int& p) -> long long {
        const int blk = __shfl(src, rel & 63);  // every lane takes part
        const int v = v0 + rel;
        p = v < e.n_glob ? v * a.global_stride : -1;
        if (p < 0 || blk < 0) return -1;
        return (long long)blk * m.block_stride + (long long)kvh * m.head_stride +
               (long long)(p & ((1 << m.bt_log2) - 1)) * m.token_stride;
    };
    int pk;
    koff = row(16 * i + j, pk);
    const uint32_t mask = (uint32_t)(__ballot(koff >= 0) & 0xffffu);
    koff = koff < 0 ? 0 : koff;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const long long o = row(16 * i + 4 * kq + r, pos[r]);
        voff[r] = o < 0 ? 0 : o;
    }
    return mask;
}

// Contiguous walks load Q4-20B tiles as spans at head_dim 64; head_dim 128
// keeps per-row loads (twice the bytes per load; its span tiles and staged
// operands exceed the register budget).
template <int D, int KVT>
constexpr bool span_tiles() {
    return KVT == NYION_KV_Q4_20B && D == 64;
}

// Tiles whose loads a wavefront keeps in flight: the one being consumed and
// NB - 1 ahead.  A Q4-20B span tile (head_dim 64) is 1280 bytes, a sixth of
// an f32 tile, so it takes a ring of four.  Gathered tiles (position lists,
// strided globals) keep two: their walks are short, and the extra tiles
// loaded past a walk's end cost more than the deeper ring gains.
template <int D, int KVT, bool SPAN>
constexpr int tile_ring() {
    return SPAN ? 4 : 2;
}

// Walk `n` tiles with the next NB - 1 tiles' loads in flight during each MFMA
// chain.  The ring is unrolled NB times so that every slot is a fixed set of
// registers (no copies between slots).  Every step issues exactly one tile of
// loads (at the end, repeats of the last tile that are never consumed), so the
// number of loads in flight is the same on every path and each tile waits
// only for its own loads.  CONTIG: the offsets describe tiles of 16
// consecutive rows, and span tiles (span_tiles) are loaded as such, koff
// being the tile's first row.
template <int D, int KVT, bool TRACK, typename Offsets, bool CONTIG = false>
__device__ __forceinline__ void walk_tiles(State<D>& st, const DecodeArgs& a, const float* qv, int n,
                                           int j, int kq, float* srow, Offsets offsets) {
    constexpr bool SPAN = CONTIG && span_tiles<D, KVT>();
    // untracked span tiles go in pairs (the tracked form's score positions
    // leave no registers for the second staged tile)
    constexpr bool PAIRS = SPAN && !TRACK;
    constexpr int NB = tile_ring<D, KVT, SPAN>();
    static_assert(!PAIRS || NB % 2 == 0, "pairs take slots 2i, 2i+1");
    using RingTile = typename std::conditional<SPAN, SpanTile<D>, Tile<D, KVT>>::type;
    RingTile t[NB];
    uint32_t msk[NB];
    long long ko, vo[4];
    int pos[NB][4];  // positions of this lane's score rows (used when TRACK)
    const int lane = threadIdx.x & 63;
    auto load = [&](RingTile& x) {
        if constexpr (SPAN)
            load_span<D>(x, a.k, a.v, ko, lane);
        else
            load_tile<D, KVT>(x, a.k, a.v, ko, vo, j, kq);
    };
    if (n <= 0) return;
#pragma unroll
    for (int k = 0; k < NB - 1; k++) {
        msk[k] = offsets(min(k, n - 1), ko, vo, pos[k]);
        load(t[k]);
    }
    if constexpr (PAIRS) {
        // span tiles go in pairs (32-token steps): slots k-1 and k at odd k,
        // before that step's load refills slot k-1
        auto eat_pair = [&](const RingTile& x, const RingTile& y, uint32_t ma, uint32_t mb, const int* pa,
                            const int* pb) {
            Tile<D, KVT> ya, yb;
            uint32_t khra[D / 32][4], khrb[D / 32][4];
            stage_span<D>(x, ya, khra, j, kq, 0);
            stage_span<D>(y, yb, khrb, j, kq, 1);
            if ((ma & mb) == 0xffffu)
                consume_pair_tiles<D, false, TRACK>(st, ya, yb, qv, ma, mb, kq, a.scale_log2, srow, pa, pb, khra,
                                                    khrb);
            else
                consume_pair_tiles<D, true, TRACK>(st, ya, yb, qv, ma, mb, kq, a.scale_log2, srow, pa, pb, khra,
                                                   khrb);
        };
        // whole ring iterations, every tile within the walk: a pair with no
        // valid row (absent blocks) takes the masked path rather than a
        // branch around it, which would make the compiler copy the running
        // state on every pair; its scores are -1e30 and its V rows zero, so
        // it adds nothing once the running max is finite, and a wavefront
        // that has seen no valid row yet is left with m = -1e30 and a
        // nonzero l, which the first valid tile multiplies away exactly
        // (alpha = exp2(-1e30 - m) = 0) and which otherwise yields the same
        // zero output as an empty walk
        int i = 0;
        for (; i + NB <= n; i += NB) {
#pragma unroll
            for (int k = 0; k < NB; k++) {
                const int s = (k + NB - 1) % NB;
                if (k & 1) eat_pair(t[k - 1], t[k], msk[k - 1], msk[k], pos[k - 1], pos[k]);
                // the refill's offsets and loads at the highest priority the
                // walk uses, so its requests leave ahead of the other
                // wavefront's arithmetic (the 64-sequence 4-bit batch
                // 111.0 -> 109.6 us, the 4096-token windows 15.06 -> 14.95 us)
                __builtin_amdgcn_s_setprio(2);
                msk[s] = offsets(min(i + k + NB - 1, n - 1), ko, vo, pos[s]);
                load(t[s]);
                __builtin_amdgcn_s_setprio(0);
            }
        }
        // the last, partial iteration: its tiles are in slots 0 .. n-i-1,
        // loaded by the steps before; no further loads
        if (i < n) {
#pragma unroll
            for (int k = 1; k < NB; k += 2) {
                const uint32_t ma = i + k - 1 < n ? msk[k - 1] : 0u;
                const uint32_t mb = i + k < n ? msk[k] : 0u;
                if (ma | mb) eat_pair(t[k - 1], t[k], ma, mb, pos[k - 1], pos[k]);
            }
        }
    } else {
        for (int i = 0; i < n; i += NB) {
#pragma unroll
            for (int k = 0; k < NB; k++) {
                const int s = (k + NB - 1) % NB;  // the slot consumed NB - 1 steps from now
                // 4-bit tiles: the refill at the top priority, as in the pair
                // walk (the windows' gathered globals 14.96 -> 14.83 us; the
                // f32 and binary16 walks gained nothing, binary16 lost 0.5 %)
                if constexpr (KVT == NYION_KV_Q4_20B) __builtin_amdgcn_s_setprio(2);
                msk[s] = offsets(min(i + k + NB - 1, n - 1), ko, vo, pos[s]);
                load(t[s]);
                if constexpr (KVT == NYION_KV_Q4_20B) __builtin_amdgcn_s_setprio(0);
                if ((k == 0 || i + k < n) && msk[k]) {
                    if constexpr (SPAN) {
                        Tile<D, KVT> y;
                        uint32_t khr[D / 32][4];
                        stage_span<D>(t[k], y, khr, j, kq);
                        consume<D, KVT, TRACK>(st, y, qv, msk[k], kq, a.scale_log2, srow, pos[k], khr);
                    } else {
                        consume<D, KVT, TRACK>(st, t[k], qv, msk[k], kq, a.scale_log2, srow, pos[k]);
                    }
                }
            }
        }
    }
}

// Online log-sum-exp merge state of one (head, 4-dim quad).
struct MergeAcc {
    float m, l, o[4];
};

__device__ __forceinline__ void merge_into(MergeAcc& x, float m, float l, const float* o) {
    const float mn = fmaxf(x.m, m);
    if (mn == -INFINITY) return;  // nothing attended on either side
    const float sx = x.m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(x.m - mn);
    const float sy = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mn);
    x.l = __builtin_fmaf(l, sy, x.l * sx);
#pragma unroll
    for (int i = 0; i < 4; i++) x.o[i] = __builtin_fmaf(o[i], sy, x.o[i] * sx);
    x.m = mn;
}

// Log-sum-exp merge of the np partials of one segment by the whole
// workgroup.  Partial p of head hh sits at acc0 + (p*16 + hh)*D and
// ml0[p*16 + hh].  A thread owns one (head, 4-dim quad) item; when there are
// fewer items than threads, R replicas of each item take partials
// r, r+R, ... and combine through LDS, so up to CH*R partials need one
// round of loads.  The partials come from other workgroups, so they are read
// with sc1 loads, CH partials' worth (m, l and O quads) issued before any is
// used.  `lds` holds 6 floats per thread; the function begins and ends with
// a barrier.
template <int D, int CH>
__device__ void merge_segment(const float* acc0, const float2* ml0, int np, int g_local, float* out,
                              int tid, float* score_rows, int scores_stride, float* lds) {
    constexpr int QPH = D / 4;  // quads per head
    const int items = g_local * QPH;
    const int R = items >= 256 ? 1 : 256 / items;
    const int nthr = items >= 256 ? 256 : R * items;
    const int r = tid / (items >= 256 ? 256 : items);
    const __amdgpu_buffer_rsrc_t racc = partial_rsrc(acc0, (uint32_t)np * 16 * D * 4);
    const __amdgpu_buffer_rsrc_t rml = partial_rsrc(ml0, (uint32_t)np * 16 * 8);
    __syncthreads();
    for (int base = 0; base < items; base += 256) {
        const int item = items >= 256 ? base + tid : tid % items;
        const bool active = tid < nthr && item < items;
        MergeAcc x{-INFINITY, 0.f, {0.f, 0.f, 0.f, 0.f}};
        const int hh = item / QPH;
        const int dq = item - hh * QPH;
        if (active) {
            for (int p0 = r; p0 < np; p0 += CH * R) {
                u32x2 mlv[CH];
                u32x4 av[CH];
#pragma unroll
                for (int q = 0; q < CH; q++) {
                    const int pq = p0 + q * R;
                    if (pq < np) {
                        const int e = pq * 16 + hh;
                        mlv[q] = __builtin_amdgcn_raw_buffer_load_b64(rml, e * 8, 0, kSc1);
                        av[q] = __builtin_amdgcn_raw_buffer_load_b128(racc, (e * D + 4 * dq) * 4, 0, kSc1);
                    } else {
                        mlv[q] = u32x2{__float_as_uint(-INFINITY), 0u};  // m = -inf, l = 0
                        av[q] = u32x4{0u, 0u, 0u, 0u};
                    }
                }
                float mc = -INFINITY;
#pragma unroll
                for (int q = 0; q < CH; q++) mc = fmaxf(mc, __uint_as_float(mlv[q][0]));
                MergeAcc c{mc, 0.f, {0.f, 0.f, 0.f, 0.f}};
                if (mc != -INFINITY) {
#pragma unroll
                    for (int q = 0; q < CH; q++) {
                        const float mq = __uint_as_float(mlv[q][0]);
                        const float w = mq == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mq - mc);
                        c.l = __builtin_fmaf(w, __uint_as_float(mlv[q][1]), c.l);
#pragma unroll
                        for (int i = 0; i < 4; i++) c.o[i] = __builtin_fmaf(w, __uint_as_float(av[q][i]), c.o[i]);
                    }
                }
                merge_into(x, c.m, c.l, c.o);
            }
        }
        if (R > 1) {  // replicas -> replica 0 through LDS
            if (active) {
                float* d = lds + 6 * tid;
                d[0] = x.m;
                d[1] = x.l;
#pragma unroll
                for (int i = 0; i < 4; i++) d[2 + i] = x.o[i];
            }
            __syncthreads();
            if (active && r == 0)
                for (int k = 1; k < R; k++) {
                    const float* d = lds + 6 * (k * items + item);
                    merge_into(x, d[0], d[1], d + 2);
                }
        }
        if (active && r == 0) {
            const float inv = x.l > 0.f ? 1.0f / x.l : 0.f;  // nothing attended: zeros
            *(float4*)(out + hh * D + 4 * dq) =
                float4{x.o[0] * inv, x.o[1] * inv, x.o[2] * inv, x.o[3] * inv};
            if (score_rows && dq == 0) {  // final (m, l) of the head: end of its score row
                float* sr = score_rows + (long long)hh * scores_stride;
                sr[scores_stride - 2] = x.m;
                sr[scores_stride - 1] = x.l;
            }
        }
    }
    __syncthreads();
}

// ---------------------------------------------------------------- kernel

// Main tiles [first, first + n) of one segment on the aligned path, in runs of
// at most 64 tiles (blocks of >= 16 tokens: a tile lies in one block, and a
// run spans at most 64 blocks).  Lane l's block id for the run [f, f + nc)
// from position base: TILES, that of the block holding run tile l; else that
// of the run's l-th block (-1 past the run, past the table or out of
// [0, num_blocks)).
template <bool TILES>
__device__ __forceinline__ int run_table_entry(const DecodeArgs& a, const int32_t* table, int base,
                                               int f, int nc, int lane) {
    const int bi = TILES ? (base + 16 * (f + lane)) >> a.bt_log2 : ((base + 16 * f) >> a.bt_log2) + lane;
    const bool in_run = TILES ? lane < nc : bi <= (base + 16 * (f + nc) - 1) >> a.bt_log2;
    int blk = -1;
    if (in_run && bi < a.table_stride) {
        blk = table[bi];
        if ((unsigned)blk >= (unsigned)a.num_blocks) blk = -1;
    }
    return blk;
}

template <int D, int KVT, bool TRACK, bool ZONE = false>
__device__ __forceinline__ void walk_main(State<D>& st, const DecodeArgs& a, const float* qv,
                                          const Extent& e, const int32_t* table, long long head_off,
                                          int first, int n, int lane, int j, int kq, float* srow,
                                          bool have_pref = false, int tbl_pref = -1,
                                          const ZoneMap* zone = nullptr, int kvh = 0) {
    for (int c0 = 0; c0 < n; c0 += 64) {
        const int f = first + c0;
        const int nc = min(64, n - c0);
        AlignedWalk w;
        w.base = e.lo & ~15;
        w.lo = e.lo;
        w.hi = e.hi;
        w.head_off = head_off;
        w.f = f;
        w.bi_first = (w.base + 16 * f) >> a.bt_log2;  // zone walks: 32-token units
        w.tblv = 0;
        // the first run's entries may have been loaded ahead (a superset of
        // the run from the same first block index: entries past the run are
        // never read)
        w.tblh = 0;
        w.kvh = kvh;
        if constexpr (ZONE) {
            // this run's 32-token units, one per lane
            constexpr int TS = KVT == NYION_KV_Q4_20B ? q4_row_bytes(D) : D;
            const int u = w.bi_first + lane;
            const int u_last = (w.base + 16 * (f + nc) - 1) >> kZoneUnitLog2;
            const long long row = u <= u_last ? zone_row_offset(*zone, u << kZoneUnitLog2, 0, TS) : -1;
            w.tblv = (int)(uint32_t)row;
            w.tblh = (int)(row >> 32);
        } else if constexpr (tile_table<KVT, ZONE>()) {
            // lane l: the first row of run tile l in this kv head (-1: past
            // the table or an invalid block id)
            constexpr int TS = q4_row_bytes(D);
            const int blk = !table ? 0
                            : (have_pref && c0 == 0) ? tbl_pref
                                                     : run_table_entry<true>(a, table, w.base, f, nc, lane);
            const int t = w.base + 16 * (f + lane);
            const long long row =
                blk < 0 ? -1
                        : (long long)blk * a.block_stride + head_off + (long long)(t & ((1 << a.bt_log2) - 1)) * TS;
            w.tblv = (int)(uint32_t)row;
            w.tblh = (int)(row >> 32);
            // interior tiles: from base + 16 t >= lo to base + 16 t + 15 <= hi
            const int ta = (e.lo & 15) != 0;
            const int tb = (e.hi - w.base + 1) >> 4;
            const bool absent = __ballot(lane < nc && blk < 0) != 0;
            w.ia = ta - f;
            w.nint = absent ? 0 : max(tb - ta, 0);
        } else {
            // lane l: the first row of this kv head in the block of block index
            // bi_first + l (-1: past the table or an invalid block id)
            const int blk = !table ? 0
                            : (have_pref && c0 == 0) ? tbl_pref
                                                     : run_table_entry<false>(a, table, w.base, f, nc, lane);
            const long long row = blk < 0 ? -1 : (long long)blk * a.block_stride + head_off;
            w.tblv = (int)(uint32_t)row;
            w.tblh = (int)(row >> 32);
        }
        // span tiles take the tile's first row (row 0 for every lane: a
        // wave-uniform offset)
        constexpr bool SPAN = span_tiles<D, KVT>();
        auto offs = [&](int i, long long& ko, long long* vo, int* pos) {
            return aligned_offsets<D, KVT, ZONE>(a, w, i, SPAN ? 0 : j, kq, ko, vo, pos);
        };
        walk_tiles<D, KVT, TRACK, decltype(offs), true>(st, a, qv, nc, j, kq, srow, offs);
    }
}

__device__ __forceinline__ int sload(const int* p) { return __builtin_amdgcn_readfirstlane(*p); }

// Occupancy target, which bounds the registers the compiler may use: two
// workgroups (8 wavefronts) per CU, except f32 KV at head_dim 128, whose two
// register-resident 16-token tiles alone take 128 VGPRs per lane (one), and
// the smaller binary16 tiles at head_dim 64 (three).  Two tiles of loads in
// flight per wavefront at this occupancy keep ~32 MB of f32 reads
// outstanding, more than HBM latency x bandwidth.  The 4-bit kernels keep
// two: at three their binary16 products spill, and the 131072-token window
// runs 10 % faster at two.
template <int D, int KVT>
constexpr int decode_waves_per_eu() {
    return (D == 128 && KVT == NYION_KV_F32) ? 1 : (D == 64 && KVT == NYION_KV_F16) ? 3 : 2;
}

// Tracked decode, second pass: importance[b][t] += sum over q heads of the
// normalised probability of position t (ops::attention_tracked,
// ops.rs:303-368: p in f32, accumulated in f64), for every attended t.
// A workgroup takes 64 positions of one sequence; wavefront w sums heads
// w, w+4, w+8, ... for its lane's position (so a thread evaluates n_heads/4
// exponentials, each times the head's 1/l, staged once per workgroup), and
// the four partial sums are added in a fixed order through LDS.
constexpr int kImpPositions = 64;
// Sequence stride of the importance workgroups a pipelined decode launch
// adds (each takes every kImpMaxSeqStride-th sequence).
constexpr int kImpMaxSeqStride = 64;

// One workgroup's share: positions bx*64 .. +63 of sequences by0, by0 + by_step,
// ...; sml and part are LDS of 256 float2 and 4 x 64 double.
__device__ __forceinline__ void importance_body(const DecodeArgs& a, double* imp, int imp_stride,
                                                int bx, int by0, int by_step, float2* sml,
                                                double (*part)[kImpPositions]) {
    constexpr int HB = 8;  // score loads issued together per thread
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int t = bx * kImpPositions + lane;
    const int tt = min(t, a.scores_stride - 3);  // in-row address for any thread
    for (int b = by0; b < a.batch; b += by_step) {
        const float* rows = a.scores + (long long)b * a.n_heads * a.scores_stride;
        const Extent e = lane_extent<true>(a, b);
        double* dst = imp + (long long)b * imp_stride + min(t, imp_stride - 1);
        const double prev = w == 0 ? *dst : 0.0;  // requested with the other loads
        double acc = 0.0;
        const bool in_window = t >= e.lo && t <= e.hi;
        const bool global = e.n_glob > 0 && t < e.n_glob * a.global_stride && t % a.global_stride == 0;
        const bool active = in_window || global;
        for (int h0 = 0; h0 < a.n_heads; h0 += 256) {
            const int hn = min(256, a.n_heads - h0);
            // (m, l) of this chunk's heads staged in LDS by vector loads
            float2 ml = float2{0.f, 1.f};
            if ((int)threadIdx.x < hn) {
                const float* row = rows + (long long)(h0 + threadIdx.x) * a.scores_stride;
                ml = float2{row[a.scores_stride - 2], 1.0f / row[a.scores_stride - 1]};
            }
            float sv[HB];
#pragma unroll
            for (int k = 0; k < HB; k++)
                sv[k] = rows[(long long)(h0 + min(w + 4 * k, hn - 1)) * a.scores_stride + tt];
            __syncthreads();  // the previous chunk's readers are done
            if ((int)threadIdx.x < hn) sml[threadIdx.x] = ml;
            __syncthreads();
            for (int k0 = 0; 4 * k0 < hn; k0 += HB) {
                if (k0 > 0) {
#pragma unroll
                    for (int k = 0; k < HB; k++)
                        sv[k] = rows[(long long)(h0 + min(w + 4 * (k0 + k), hn - 1)) * a.scores_stride + tt];
                }
#pragma unroll
                for (int k = 0; k < HB; k++) {
                    const int hh = w + 4 * (k0 + k);
                    if (active && hh < hn) {
                        const float2 m = sml[hh];
                        acc += (double)(__builtin_amdgcn_exp2f(sv[k] - m.x) * m.y);
                    }
                }
            }
        }
        part[w][lane] = acc;
        __syncthreads();
        if (w == 0 && active) *dst = prev + ((part[0][lane] + part[1][lane]) + (part[2][lane] + part[3][lane]));
        __syncthreads();  // part[] is reused by the next sequence
    }
}

__global__ __launch_bounds__(256) void importance_kernel(DecodeArgs a, double* imp, int imp_stride) {
    __shared__ float2 sml[256];
    __shared__ double part[4][kImpPositions];
    importance_body(a, imp, imp_stride, blockIdx.x, blockIdx.y, gridDim.y, sml, part);
}

template <int D, int KVT, bool ALIGNED, bool TRACK, bool ZONE = false>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(decode_waves_per_eu<D, KVT>())))
void decode_kernel(DecodeArgs a) {
    constexpr int NC = D / 4;
    constexpr int DPL = D / 16;
    __shared__ floatx4 sm_acc[3][DPL][64];
    __shared__ float sm_m[4][16];
    __shared__ float sm_l[4][16];
    __shared__ int sm_pref[kMaxLaunchBatch + 1];  // tiles per segment, exclusive prefix
    __shared__ int2 sm_seq[kMaxLaunchBatch];       // (ctx_len, q_pos) or (list length, 0)
    __shared__ int sm_wsum[4];
    __shared__ int sm_last;

    if constexpr (TRACK) {
        if ((int)blockIdx.x >= a.decode_grid) {
            // pipelined tracked decode: the previous call's importance sum
            // (its scores are final, launches on one stream run in order)
            // on workgroups past the decode's, in the merge buffer's LDS
            const int k = (int)blockIdx.x - a.decode_grid;
            DecodeArgs ia = a;
            ia.scores = const_cast<float*>(a.imp_scores);
            ia.batch = a.imp_batch;
            float2* sml = reinterpret_cast<float2*>(&sm_acc[0][0][0]);
            importance_body(ia, a.imp_out, a.imp_stride, k % a.imp_nx, k / a.imp_nx, a.imp_ny, sml,
                            reinterpret_cast<double(*)[kImpPositions]>(sml + 256));
            return;
        }
    }
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int j = lane & 15;
    const int kq = lane >> 4;
    const int U = a.n_kv_heads * a.n_hg;  // segments per sequence

    // Each iteration runs one piece of segment (b, u) -- its wavefronts take
    // tiles [wa, wb) -- and ends with a merge: `whole` when the piece is the
    // segment; otherwise its partial goes to slot `slot`, the segment's
    // `pieces` partials sit in slots slot0 .. slot0 + pieces - 1 and the last
    // to arrive merges them.  pref: this wavefront's first block-table
    // entries were loaded ahead (tbl_pref).
    //
    // Direct partition (few segments, a.direct > 0): workgroup = piece
    // `piece` of segment s, pieces of c tiles of the host's bound on a
    // segment's tiles, one iteration, no per-workgroup prefix sums; with full
    // context a tile's positions do not depend on the length, so this
    // wavefront's block-table entries are requested before the length
    // arrives.  Stream-K (otherwise): the segments' tile lists laid end to
    // end and cut into equal ranges, one per workgroup, possibly spanning
    // several segments.
    const bool direct = a.direct > 0;
    int g1 = 0, c = 1, pos = 0, b = 0;
    if (!direct) {
        // tiles of one segment of each sequence, prefix-summed into LDS
        int carry = 0;
        if (threadIdx.x == 0) sm_pref[0] = 0;
        for (int c0 = 0; c0 < a.batch; c0 += 256) {
            const int bb = c0 + threadIdx.x;
            int t = 0;
            if (bb < a.batch) {
                const int2 v = seq_values(a, bb);
                sm_seq[bb] = v;
                t = extent_of<ALIGNED>(a, v).tiles;
            }
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int y = __shfl_up(t, o);
                if (lane >= o) t += y;
            }
            if (lane == 63) sm_wsum[wave] = t;
            __syncthreads();
            int off = carry;
            for (int w = 0; w < wave; w++) off += sm_wsum[w];
            if (bb < a.batch) sm_pref[bb + 1] = off + t;
            carry += sm_wsum[0] + sm_wsum[1] + sm_wsum[2] + sm_wsum[3];
            __syncthreads();
        }
        // the host keeps batch * U * (tiles of the longest segment) below 2^31
        const int T = __builtin_amdgcn_readfirstlane(carry) * U;
        c = (T + a.decode_grid - 1) / a.decode_grid;  // tiles per workgroup
        const int g0 = min((int)blockIdx.x * c, T);
        g1 = min(g0 + c, T);

        // sequences with nothing to attend to (ctx_len <= 0, q_pos < 0, empty list)
        for (int bb = blockIdx.x; bb < a.batch; bb += a.decode_grid) {
            if (sload(&sm_pref[bb + 1]) != sload(&sm_pref[bb])) continue;
            float* o = a.out + (long long)bb * a.n_heads * D;
            for (int i = threadIdx.x; i < a.n_heads * D; i += 256) o[i] = 0.f;
        }
        if (g0 >= g1) return;

        // first sequence of the range: the largest b with U * prefix[b] <= g0
        int hi = a.batch - 1;
        while (b < hi) {
            const int mid = (b + hi + 1) >> 1;
            if (U * sload(&sm_pref[mid]) <= g0) b = mid;
            else hi = mid - 1;
        }
        pos = g0;
    }
    for (;;) {
        int u, wa, wb, pieces, slot;
        long long slot0;
        bool whole, pref = false;
        int tbl_pref = -1;
        Extent e;
        if (direct) {
            const int P = a.direct;
            const int s = (int)blockIdx.x / P;
            const int piece = (int)blockIdx.x - s * P;
            b = s / U;
            u = s - b * U;
            const int cd = (a.seg_tiles + P - 1) / P;
            const int t0 = piece * cd;
            const int wa0 = t0 + (wave * cd) / 4, wb0 = t0 + ((wave + 1) * cd) / 4;
            pref = ALIGNED && a.mode == MODE_FULL && a.tables && wb0 > wa0;
            // untracked 4-bit span walks of paged windows: the walk of a
            // sequence at the host's max_ctx (q at its end) starts at block
            // position pref_base; its entries are requested with the length,
            // kept if the extent confirms that start
            constexpr bool kSpec = tile_table<KVT, ZONE>() && span_tiles<D, KVT>() && !TRACK;
            int pref_base = 0;
            if (kSpec && ALIGNED && a.mode == MODE_WINDOW && a.spec_len > 0 && a.tables && wb0 > wa0) {
                const int ve = a.spec_len - 1;
                pref_base = (ve > a.window ? ve - a.window + 1 : 0) & ~15;
                pref = true;
            }
            if (pref)
                tbl_pref = run_table_entry<tile_table<KVT, ZONE>()>(
                    a, a.tables + (long long)b * a.table_stride, pref_base, wa0, min(64, wb0 - wa0), lane);
            const int len = a.ctx_lens ? sload(a.ctx_lens + b) : a.uniform_len;
            const int qp = a.q_pos ? sload(a.q_pos + b) : len - 1;
            e = extent_of<ALIGNED>(a, int2{len, qp});
            wa = min(wa0, e.tiles);
            wb = min(wb0, e.tiles);
            if (KVT == NYION_KV_Q4_20B && ALIGNED && e.n_glob > 0 && e.main_tiles > t0 &&
                e.main_tiles < t0 + cd) {
                // no wavefront walks both sides of the boundary between the
                // contiguous tiles and the globals (two serial chains of round
                // trips): the piece's inner wave boundary nearest to it moves
                // onto it when its neighbours enclose it; the piece's tiles
                // are the same, two wavefronts trade a few.  4-bit kernels
                // only: in the f32 and binary16 ones the extra scalar state
                // spills scalar registers inside the walk loops.
                const int mt = e.main_tiles;
                const int kb = min(3, max(1, (8 * (mt - t0) + cd) / (2 * cd)));
                if (t0 + ((kb - 1) * cd) / 4 <= mt && mt <= t0 + ((kb + 1) * cd) / 4) {
                    if (wave == kb - 1) wb = mt;
                    if (wave == kb) wa = mt;
                }
            }
            // (the entries cover tiles wa0 .. wb0 - 1: a walk start moved or
            // an end moved past wb0 by the re-cut above loads its own)
            if (kSpec && pref && ((e.lo & ~15) != pref_base || wa != wa0 || wb > wb0)) pref = false;
            whole = P == 1;
            pieces = P;
            slot = (int)blockIdx.x;
            slot0 = (long long)s * P;
        } else {
            while (U * sload(&sm_pref[b + 1]) <= pos) b++;
            const int pb = sload(&sm_pref[b]);
            const int Tb = sload(&sm_pref[b + 1]) - pb;
            u = (pos - U * pb) / Tb;
            const int seg0 = U * pb + u * Tb;  // first global tile of segment (b, u)
            const int t0 = pos - seg0;
            const int t1 = min(Tb, t0 + (g1 - pos));
            pos += t1 - t0;
            // the sequence's values from LDS, in scalar registers, so that
            // tile loop bounds and masks derived from them branch uniformly
            e = extent_of<ALIGNED>(a, int2{sload(&sm_seq[b].x), sload(&sm_seq[b].y)});
            const int n = t1 - t0;
            wa = t0 + (wave * n) / 4;
            wb = t0 + ((wave + 1) * n) / 4;
            whole = n == Tb;
            const int gf = seg0 / c;
            pieces = (seg0 + Tb - 1) / c - gf + 1;
            slot = (int)blockIdx.x + b * U + u;
            slot0 = (long long)gf + b * U + u;
        }

        const int kvh = u / a.n_hg;
        const int hg = u - kvh * a.n_hg;
        const int g_local = min(16, a.group - hg * 16);
        const int head0 = kvh * a.group + hg * 16;

        // Q operand (B of the QK product): head j, dims by qk_dim (Q4-20B:
        // q_operand_q4, NC words and then the D/32 scaled group sums)
        float qv[KVT == NYION_KV_Q4_20B ? NC + D / 32 : NC];
        {
            const float* qrow = a.q + ((long long)b * a.n_heads + head0 + min(j, g_local - 1)) * D;
            const bool ok = j < g_local;
            if constexpr (KVT == NYION_KV_Q4_20B) {
                report_range(a.status, q_operand_q4<D>(qrow, ok, kq, qv), kRangeDecodeQ);
            } else {
                // the lane's dims come in runs of four (qk_dim(4i..4i+3)
                // consecutive): one 16-byte load per run
#pragma unroll
                for (int i = 0; i < NC / 4; i++) {
                    const float4 r4 =
                        ok ? *(const float4*)(qrow + qk_dim<D, KVT>(4 * i, kq)) : float4{0.f, 0.f, 0.f, 0.f};
                    qv[4 * i] = r4.x;
                    qv[4 * i + 1] = r4.y;
                    qv[4 * i + 2] = r4.z;
                    qv[4 * i + 3] = r4.w;
                }
            }
            if constexpr (KVT == NYION_KV_F16) {
                // words 4x, 4x+1: the four values as binary16; 4x+2, 4x+3: the
                // binary16 residuals.  |q| >= 65520 rounds the high part to
                // infinity: reported through the status word.
                bool big = false;
#pragma unroll
                for (int cc = 0; cc < NC; cc++) big |= fabsf(qv[cc]) >= 65520.f;
                report_range(a.status, big, kRangeDecodeQ);
#pragma unroll
                for (int x = 0; x < D / 16; x++) pack_hi_lo(qv + 4 * x, qv + 4 * x);
            }
        }

        State<D> st;
#pragma unroll
        for (int x = 0; x < DPL; x++) st.acc[x] = floatx4{0.f, 0.f, 0.f, 0.f};
        st.acc_m = floatx4{0.f, 0.f, 0.f, 0.f};
        st.m = -INFINITY;
        st.l = 0.f;
        st.k6464 = 0x64006400u;
        asm volatile("" : "+v"(st.k6464));

        // TRACK: this lane's head's row of the score buffer (pad heads: none)
        float* srow = nullptr;
        if (TRACK && j < g_local)
            srow = a.scores + ((long long)b * a.n_heads + head0 + j) * a.scores_stride;

        RowMap m;
        m.table = a.tables ? a.tables + (long long)b * a.table_stride : nullptr;
        m.block_stride = a.block_stride;
        m.head_stride = a.head_stride;
        m.token_stride = a.token_stride;
        m.bt_log2 = a.bt_log2;
        m.num_blocks = a.num_blocks;
        m.table_len = a.table_stride;
        m.zone = a.zone;
        m.zone.page_base = a.page_bases ? a.page_bases + (long long)b * a.zone.n_pages : nullptr;

        if (ALIGNED) {
            const int mt = e.main_tiles;
            const int me = min(wb, mt);
            if (wa < me)
                walk_main<D, KVT, TRACK, ZONE>(st, a, qv, e, m.table, (long long)kvh * a.head_stride, wa,
                                               me - wa, lane, j, kq, srow, pref, tbl_pref, &m.zone, kvh);
            const int ga = max(wa, mt) - mt;
            const int gb = wb - mt;
            if (ZONE && ga < gb) {
                // zone pages: each global row through the zone arithmetic
                walk_tiles<D, KVT, TRACK>(st, a, qv, gb - ga, j, kq, srow,
                                          [&](int i, long long& ko, long long* vo, int* pos) {
                                              return gather_offsets<D, KVT>(a, e, m, b, kvh, 16 * (ga + i),
                                                                            e.n_glob, true, j, kq, ko, vo, pos);
                                          });
            } else if (ga < gb) {
                // the block ids of all this wavefront's globals in one batch
                const GlobalBlocks gbk = load_global_blocks(a, e, m, 16 * ga, lane);
                walk_tiles<D, KVT, TRACK>(st, a, qv, gb - ga, j, kq, srow,
                                          [&](int i, long long& ko, long long* vo, int* pos) {
                                              return global_offsets(a, e, m, gbk, kvh, 16 * ga, i, j,
                                                                    kq, ko, vo, pos);
                                          });
            }
        } else {
            walk_tiles<D, KVT, TRACK>(st, a, qv, wb - wa, j, kq, srow,
                                      [&](int i, long long& ko, long long* vo, int* pos) {
                                          return gather_offsets<D, KVT>(a, e, m, b, kvh, 16 * (wa + i),
                                                                        e.L, false, j, kq, ko, vo, pos);
                                      });
        }

        if constexpr (KVT == NYION_KV_Q4_20B) {  // the dmin/32 term belongs to every dim
#pragma unroll
            for (int x = 0; x < DPL; x++) st.acc[x] += st.acc_m;
            st.l *= 0.03125f;  // accumulated in units of 32 (exact)
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
        const int s = b * U + u;
        if (wave == 0) {
            // this piece's partial slot (used when !whole)
            const __amdgpu_buffer_rsrc_t racc = partial_rsrc(a.ws_acc + (long long)slot * 16 * D, 16 * D * 4);
            const __amdgpu_buffer_rsrc_t rml = partial_rsrc(a.ws_ml + (long long)slot * 16, 16 * 8);
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
            // span walks: the store offsets are formed here, from a copy of kq
            // the compiler cannot see through; hoisted out of the piece loop
            // they would be held across the walk, where registers are short
            int kqs = kq;
            if constexpr (span_tiles<D, KVT>()) asm volatile("" : "+v"(kqs));
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int hh = 4 * kqs + r;
                if (hh >= g_local) continue;
                if (TRACK && whole && j == 0) {  // final (m, l) of the head: row end
                    float* sr = a.scores + ((long long)b * a.n_heads + head0 + hh) * a.scores_stride;
                    sr[a.scores_stride - 2] = mh[r];
                    sr[a.scores_stride - 1] = lh[r];
                }
                if (whole) {
                    const float inv = lh[r] > 0.f ? 1.0f / lh[r] : 0.f;  // nothing attended: zeros
                    float* o = a.out + ((long long)b * a.n_heads + head0 + hh) * D + DPL * j;
#pragma unroll
                    for (int x = 0; x < DPL / 4; x++)
                        *(float4*)(o + 4 * x) = float4{st.acc[4 * x + 0][r] * inv, st.acc[4 * x + 1][r] * inv,
                                                       st.acc[4 * x + 2][r] * inv, st.acc[4 * x + 3][r] * inv};
                } else {
#pragma unroll
                    for (int x = 0; x < DPL / 4; x++) {
                        const u32x4 d = {__float_as_uint(st.acc[4 * x + 0][r]), __float_as_uint(st.acc[4 * x + 1][r]),
                                         __float_as_uint(st.acc[4 * x + 2][r]), __float_as_uint(st.acc[4 * x + 3][r])};
                        __builtin_amdgcn_raw_buffer_store_b128(d, racc, (hh * D + DPL * j + 4 * x) * 4, 0, kSc1);
                    }
                    if (j == 0)
                        __builtin_amdgcn_raw_buffer_store_b64(u32x2{__float_as_uint(mh[r]), __float_as_uint(lh[r])},
                                                              rml, hh * 8, 0, kSc1);
                }
            }
            if (!whole) {
                // publish: the write-through stores complete before the arrival is
                // counted (the fence keeps the compiler from moving them past the
                // wait); the last of the segment's pieces to arrive merges
                __atomic_signal_fence(__ATOMIC_SEQ_CST);
                __builtin_amdgcn_s_waitcnt(0);
                int old = 0;
                if (lane == 0)
                    old = __hip_atomic_fetch_add(a.counters + s, 1, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
                old = __shfl(old, 0);
                if (lane == 0) sm_last = (old == pieces - 1);
            }
        }
        __syncthreads();  // also: LDS is free for the next piece
        if (!whole && sm_last) {
            // partials per batch of loads: 16, or 8 in kernels with three
            // wavefronts per SIMD (168 VGPRs), where 16 would spill
            constexpr int kMergeBatch = decode_waves_per_eu<D, KVT>() >= 3 ? 8 : 16;
            merge_segment<D, kMergeBatch>(a.ws_acc + slot0 * 16 * D, a.ws_ml + slot0 * 16, pieces, g_local,
                             a.out + ((long long)b * a.n_heads + head0) * D, threadIdx.x,
                             TRACK ? a.scores + ((long long)b * a.n_heads + head0) * a.scores_stride
                                   : nullptr,
                             a.scores_stride, (float*)&sm_acc[0][0][0]);
            if (threadIdx.x == 0)
                __hip_atomic_store(a.counters + s, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (direct || pos >= g1) break;
    }
}

__global__ void fill_zero_kernel(int* p, long long n) {
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n;
         i += (long long)gridDim.x * blockDim.x)
        p[i] = 0;
}

// ---------------------------------------------------------------- host side

// Tiles per workgroup the grid is sized for: small enough to spread a short
// context over many CUs, large enough that each wavefront pipelines a few
// tiles.  By default the launch's tiles divided by the CU count, within
// [kSmallWgTiles, kDefaultWgTiles] (a single 4096-token sequence then fills
// every CU with 8-tile ranges; large batches use 16).  Workspace sizes assume
// the smallest allowed value, so tuning never outgrows a workspace.
constexpr int kDefaultWgTiles = 16;
constexpr int kSmallWgTiles = 8;
constexpr int kMinWgTiles = 4;
constexpr int kMaxGrid = 2048;  // workgroups per launch (partial slots are sized for it)
// Tuning override of the tiles per workgroup (0 = default), set by
// nyion_set_decode_partition_tokens for the whole process and read once per
// call; an atomic, so a concurrent change takes effect at a call boundary.
static std::atomic<int> g_wg_tiles_override{0};

struct DecodePlan {
    DecodeArgs a;      // batch field: set per launch
    int batch;         // all sequences
    int chunk;         // sequences per launch
    int tiles_max;     // bound on the tiles of one segment
    int grid_bound;    // workgroups per launch at most (sizes the partial slots)
    size_t ws_bytes;
    int head_dim;
    int kvt;
    bool aligned;
    bool track;
    bool zone;         // zone pages on the aligned walk
    int imp_max_ctx;   // > 0: the first launch also sums the importance of
                       // a.imp_scores (pipelined tracked decode)
};

static size_t ws_layout(int slots, int segments, int head_dim, size_t* ml_off, size_t* ctr_off) {
    const size_t acc = ((size_t)slots * 16 * head_dim * sizeof(float) + 255) & ~(size_t)255;
    const size_t ml = ((size_t)slots * 16 * sizeof(float2) + 255) & ~(size_t)255;
    const size_t ctr = ((size_t)segments * sizeof(int) + 255) & ~(size_t)255;
    if (ml_off) *ml_off = acc;
    if (ctr_off) *ctr_off = acc + ml;
    return acc + ml + ctr;
}

static int grid_for(long long tiles, int wg_tiles, int cap) {
    long long g = (tiles + wg_tiles - 1) / wg_tiles;
    if (g > cap) g = cap;
    return g < 1 ? 1 : (int)g;
}

// max_main: host bound on the contiguous main range; globals: whether
// strided globals may exist.
static int plan_common(DecodePlan& pl, int batch, int n_heads, int n_kv_heads, int head_dim,
                       int kvt, int max_main, bool globals, bool aligned_path, float scale) {
    if (batch <= 0 || n_heads <= 0 || n_kv_heads <= 0)
        return set_error(NYION_ERR_INVALID, "decode: batch/heads must be positive");
    if (n_heads % n_kv_heads)
        return set_error(NYION_ERR_INVALID, "decode: n_heads %d not a multiple of n_kv_heads %d",
                         n_heads, n_kv_heads);
    if (head_dim != 64 && head_dim != 128)
        return set_error(NYION_ERR_UNSUPPORTED, "decode: head_dim %d (supported: 64, 128)", head_dim);
    if (kvt != NYION_KV_F32 && kvt != NYION_KV_Q4_20B && kvt != NYION_KV_F16)
        return set_error(NYION_ERR_INVALID, "decode: kv_dtype %d", kvt);
    if (max_main <= 0) return set_error(NYION_ERR_INVALID, "decode: max_ctx must be positive");
    DecodeArgs& a = pl.a;
    a = DecodeArgs{};
    a.n_heads = n_heads;
    a.n_kv_heads = n_kv_heads;
    a.group = n_heads / n_kv_heads;
    a.n_hg = (a.group + 15) / 16;
    const float sc = scale > 0.f ? scale : 1.0f / sqrtf((float)head_dim);
    a.scale_log2 = sc * 1.4426950408889634f;
    a.max_len = max_main;
    a.status = device_status_word();
    const long long units = (long long)n_kv_heads * a.n_hg;
    // aligned: main tiles <= max_main/16 + 2, globals (<= 128) <= 8 tiles;
    // gather: the globals are part of the list
    const long long tiles = aligned_path ? max_main / 16 + 2 + (globals ? 8 : 0)
                                         : ((long long)max_main + (globals ? 128 : 0) + 15) / 16;
    const long long per_seq = units * tiles;
    if (per_seq >= (1LL << 31))
        return set_error(NYION_ERR_UNSUPPORTED, "decode: %lld tiles per sequence", per_seq);
    long long chunk = ((1LL << 31) - 1) / per_seq;
    if (chunk > kMaxLaunchBatch) chunk = kMaxLaunchBatch;
    if (chunk > batch) chunk = batch;
    pl.batch = batch;
    pl.chunk = (int)chunk;
    pl.tiles_max = (int)tiles;
    pl.head_dim = head_dim;
    pl.kvt = kvt;
    pl.aligned = aligned_path;
    pl.track = false;
    pl.zone = false;
    pl.imp_max_ctx = 0;
    pl.grid_bound = grid_for(chunk * per_seq, kMinWgTiles, kMaxGrid);
    // one sequence over at most one workgroup per segment: no partials
    if (batch == 1 && pl.grid_bound <= units) {
        pl.grid_bound = (int)units;
        pl.ws_bytes = 0;
    } else {
        pl.ws_bytes = ws_layout(pl.grid_bound + (int)(chunk * units), (int)(chunk * units), head_dim,
                                nullptr, nullptr);
    }
    return NYION_OK;
}

static int attach_workspace(DecodePlan& pl, void* ws, size_t ws_bytes) {
    if (pl.ws_bytes == 0) return NYION_OK;
    if (!ws || ws_bytes < pl.ws_bytes)
        return set_error(NYION_ERR_WORKSPACE, "decode: workspace %zu bytes < required %zu", ws_bytes,
                         pl.ws_bytes);
    if (!aligned(ws, 256)) return set_error(NYION_ERR_INVALID, "decode: workspace not 256-byte aligned");
    const int units = pl.a.n_kv_heads * pl.a.n_hg;
    size_t ml_off = 0, ctr_off = 0;
    ws_layout(pl.grid_bound + pl.chunk * units, pl.chunk * units, pl.head_dim, &ml_off, &ctr_off);
    pl.a.ws_acc = (float*)ws;
    pl.a.ws_ml = (float2*)((char*)ws + ml_off);
    pl.a.counters = (int*)((char*)ws + ctr_off);
    return NYION_OK;
}

// Workgroups of one kernel instance resident on the whole device (per
// device, computed on first use there).
template <int D, int KVT, bool AL, bool TR, bool ZN = false>
static int resident_capacity() {
    static std::atomic<int> cache[kMaxDevices];
    return per_device_value(
        cache,
        [] {
            int per_cu = 0;
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_kernel<D, KVT, AL, TR, ZN>,
                                                             256, 0) != hipSuccess) {
                (void)hipGetLastError();
                return 0;
            }
            return (per_cu > 0 ? per_cu : 1) * device_cu_count();
        },
        256);
}

static int wg_tiles_for(long long total_tiles) {
    const int ov = g_wg_tiles_override.load(std::memory_order_relaxed);
    if (ov > 0) return ov;
    const long long per_cu = total_tiles / device_cu_count();
    return per_cu < kSmallWgTiles ? kSmallWgTiles : per_cu > kDefaultWgTiles ? kDefaultWgTiles : (int)per_cu;
}

// Segments of one launch up to which the direct partition is used: with few
// segments the stream-K prologue (lengths, prefix sums, a search) is a
// dependent round trip and two barriers that the direct form skips.
constexpr int kDirectMaxSegments = 64;
// Direct partition of small tiles (4-bit rows, binary16 at head_dim 64): the
// tiles per workgroup double while a workgroup's K+V bytes stay within
// kDirectWgBytes and the launch keeps kDirectMinGrid workgroups.  Such a
// launch's time is the chain of round trips of its pieces (rows, partial
// stores and their acknowledgement, the arrival atomic, the merge's
// reloads), not their walks, and fewer pieces publish and re-read fewer
// partials.  The pieces are then raised to one workgroup per CU where each
// keeps kDirectMinPieceTiles tiles: with the CUs otherwise idle, the
// shorter walks gain more than the extra partials cost (8 windows of 4096
// tokens, 4 kv heads: 128 -> 256 workgroups, 14.8 -> 13.5 us).  The tuning
// override, when set, is used as it is.
constexpr long long kDirectWgBytes = 96 << 10;
constexpr long long kDirectMinGrid = 128;
constexpr int kDirectMinPieceTiles = 16;

template <int D, int KVT>
static int direct_wg_tiles(int wg, int seg_tiles, long long segs) {
    if (g_wg_tiles_override.load(std::memory_order_relaxed) > 0) return wg;
    constexpr long long tile_bytes =
        32LL * (KVT == NYION_KV_Q4_20B ? q4_row_bytes(D) : KVT == NYION_KV_F16 ? 2 * D : 4 * D);
    while (2 * wg * tile_bytes <= kDirectWgBytes && 2 * wg <= seg_tiles &&
           (seg_tiles + 2LL * wg - 1) / (2LL * wg) * segs >= kDirectMinGrid)
        wg *= 2;
    return wg;
}

template <int D, int KVT, bool AL, bool TR, bool ZN = false>
static void launch_dk(const DecodePlan& pl, hipStream_t stream) {
    const int units = pl.a.n_kv_heads * pl.a.n_hg;
    const int cap = resident_capacity<D, KVT, AL, TR, ZN>();
    for (int b0 = 0; b0 < pl.batch; b0 += pl.chunk) {
        const int nb = pl.batch - b0 < pl.chunk ? pl.batch - b0 : pl.chunk;
        DecodeArgs a = pl.a;
        a.batch = nb;
        const long long qo = (long long)b0 * a.n_heads * D;
        a.q += qo;
        a.out += qo;
        if (a.tables) a.tables += (long long)b0 * a.table_stride;
        if (a.page_bases) a.page_bases += (long long)b0 * a.zone.n_pages;
        if (a.ctx_lens) a.ctx_lens += b0;
        if (a.q_pos) a.q_pos += b0;
        if (a.positions) a.positions += (long long)b0 * a.pos_stride;
        if (a.n_pos) a.n_pos += b0;
        if (a.scores) a.scores += (long long)b0 * a.n_heads * a.scores_stride;
        const long long total = (long long)nb * units * pl.tiles_max;
        const int wg = wg_tiles_for(total);
        int grid = grid_for(total, wg, cap);
        if (grid > pl.grid_bound) grid = pl.grid_bound;
        if (pl.ws_bytes == 0 || (nb == 1 && grid <= units)) grid = units;  // whole segments
        const long long segs = (long long)nb * units;
        if (AL && a.mode != MODE_LIST && segs <= kDirectMaxSegments) {
            // pieces per segment from the tiles per workgroup, within the
            // partial slots the workspace holds (one per workgroup)
            const int seg_tiles = a.mode == MODE_FULL ? (a.max_len + 15) / 16 : pl.tiles_max;
            const int wgd = direct_wg_tiles<D, KVT>(wg, seg_tiles, segs);
            long long P = pl.ws_bytes == 0 ? 1 : (seg_tiles + wgd - 1) / wgd;
            if (pl.ws_bytes != 0 && wgd > wg) {
                // small tiles: at least one workgroup per CU where the pieces
                // keep kDirectMinPieceTiles tiles
                const long long p_cu = std::min<long long>(device_cu_count() / segs, seg_tiles / kDirectMinPieceTiles);
                if (p_cu > P) P = p_cu;
            }
            const long long limit = std::min<long long>(cap, pl.grid_bound);
            if (P * segs > limit) P = std::max<long long>(1, limit / segs);
            if (P > 1 || pl.ws_bytes == 0 || nb == 1) {
                a.direct = (int)P;
                a.seg_tiles = seg_tiles;
                grid = (int)(P * segs);
            }
        }
        a.decode_grid = grid;
        long long launch = grid;
        if (TR && b0 == 0 && pl.imp_max_ctx > 0) {
            // the previous call's importance: all its sequences, from this
            // first launch (its ctx_lens / q_pos are not offset)
            a.imp_nx = (pl.imp_max_ctx + kImpPositions - 1) / kImpPositions;
            a.imp_ny = pl.batch < kImpMaxSeqStride ? pl.batch : kImpMaxSeqStride;
            a.imp_batch = pl.batch;
            launch += (long long)a.imp_nx * a.imp_ny;
        }
        hipLaunchKernelGGL((decode_kernel<D, KVT, AL, TR, ZN>), dim3((unsigned)launch), dim3(256), 0,
                           stream, a);
    }
}

template <int D, int KVT>
static void launch_dkt(const DecodePlan& pl, hipStream_t stream) {
    if (pl.zone) {  // zone pages on the aligned walk (no tracked form)
        launch_dk<D, KVT, true, false, true>(pl, stream);
    } else if (pl.track) {
        if (pl.aligned)
            launch_dk<D, KVT, true, true>(pl, stream);
        else
            launch_dk<D, KVT, false, true>(pl, stream);
    } else if (pl.aligned) {
        launch_dk<D, KVT, true, false>(pl, stream);
    } else {
        launch_dk<D, KVT, false, false>(pl, stream);
    }
}

static int launch_plan(const DecodePlan& pl, hipStream_t stream) {
    if (pl.head_dim == 64 && pl.kvt == NYION_KV_F32)
        launch_dkt<64, NYION_KV_F32>(pl, stream);
    else if (pl.head_dim == 64 && pl.kvt == NYION_KV_F16)
        launch_dkt<64, NYION_KV_F16>(pl, stream);
    else if (pl.head_dim == 64)
        launch_dkt<64, NYION_KV_Q4_20B>(pl, stream);
    else if (pl.kvt == NYION_KV_F32)
        launch_dkt<128, NYION_KV_F32>(pl, stream);
    else if (pl.kvt == NYION_KV_F16)
        launch_dkt<128, NYION_KV_F16>(pl, stream);
    else
        launch_dkt<128, NYION_KV_Q4_20B>(pl, stream);
    return check_launch("decode");
}

// Row size in the pool's own units: f32 or f16 elements, Q4-20B bytes.
static long long row_elems(int head_dim, int kvt) {
    return kvt == NYION_KV_Q4_20B ? q4_row_bytes(head_dim) : head_dim;
}

static int check_pool_ptrs(const void* k, const void* v, int kvt) {
    if (!k || !v) return set_error(NYION_ERR_INVALID, "decode: null K/V pool");
    const size_t al = kvt == NYION_KV_F32 ? 16 : kvt == NYION_KV_F16 ? 8 : 4;
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
    if (tokens != 0 && (tokens < 16 * kMinWgTiles || tokens > 4096 || !is_pow2(tokens)))
        return set_error(NYION_ERR_INVALID,
                         "partition tokens %d: power of two in [%d, 4096] or 0", tokens,
                         16 * kMinWgTiles);
    g_wg_tiles_override.store(tokens / 16, std::memory_order_relaxed);
    return NYION_OK;
}

int nyion_get_decode_partition_tokens(int batch, int n_kv_heads, int head_dim, int max_len) {
    if (batch <= 0 || n_kv_heads <= 0 || max_len <= 0) return 0;
    const long long tiles = (long long)batch * n_kv_heads * (max_len / 16 + 2);
    int cap = kMaxGrid;
    const int ov = g_wg_tiles_override.load(std::memory_order_relaxed);
    int wg_tiles = ov > 0 ? ov : kDefaultWgTiles;
    if (require_device() == NYION_OK) {
        cap = head_dim == 128 ? resident_capacity<128, NYION_KV_F32, true, false>()
                              : resident_capacity<64, NYION_KV_F32, true, false>();
        wg_tiles = wg_tiles_for(tiles);
    }
    clear_error();
    const int grid = grid_for(tiles, wg_tiles, cap);
    return (int)(16 * ((tiles + grid - 1) / grid));
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

}  // extern "C"

// Split-K scratch of nyion_paged_decode_attention_noalloc: a library-owned
// device array (one per device, held until the process ends).  Host code
// never passes the array's name to a kernel (on the host it names a
// stand-in, not device memory): decode_scratch_ptr() gives the device
// address, looked up once per device with that device current.
constexpr size_t kScratchBytes = NYION_DECODE_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace nyion {

void* decode_scratch_ptr() {
    static std::atomic<uintptr_t> cache[kMaxDevices];
    const int dev = current_device();
    if (dev < 0) return nullptr;
    uintptr_t v = cache[dev].load(std::memory_order_relaxed);
    if (v) return (void*)v;
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
        (void)hipGetLastError();
        set_error(NYION_ERR_LAUNCH, "decode scratch: hipGetSymbolAddress failed: %s",
                  hipGetErrorString(e));
        return nullptr;
    }
    cache[dev].store((uintptr_t)ptr, std::memory_order_relaxed);
    return ptr;
}

}  // namespace nyion

// The tracked form's second launch over the scores (and per-row max and
// denominator) the decode stored: `a` carries the attended sets (mode,
// window, globals, lengths) and the scores buffer.
static int launch_importance(const DecodeArgs& a, int batch, int max_ctx, double* d_importance,
                             int importance_stride, hipStream_t stream) {
    DecodeArgs ia = a;
    ia.batch = batch;
    const unsigned gy = batch < 65535 ? (unsigned)batch : 65535u;
    hipLaunchKernelGGL(importance_kernel,
                       dim3((unsigned)((max_ctx + kImpPositions - 1) / kImpPositions), gy), dim3(256), 0,
                       stream, ia, d_importance, importance_stride);
    return check_launch("decode importance");
}

// Shared body of the paged decode entry points; scores/imp non-null selects
// the tracked form; use_scratch takes the split-K workspace from the
// library's scratch array (d_workspace is ignored) and clears its counters.
static int paged_decode_common(const float* d_q, const void* k_pool, const void* v_pool,
                               const int32_t* block_tables, int max_blocks_per_seq,
                               const int32_t* ctx_lens, const int32_t* q_pos, int batch,
                               int n_heads, int n_kv_heads, int head_dim, int block_tokens,
                               int num_blocks, int kv_dtype, int window, int global_stride,
                               int max_ctx, float scale, float* d_out, void* d_workspace,
                               size_t workspace_bytes, float* d_scores, int scores_stride,
                               double* d_importance, int importance_stride, hipStream_t stream,
                               bool use_scratch = false, bool with_importance = true,
                               const float* d_prev_scores = nullptr) {
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
    const bool track = d_scores != nullptr;
    if (track) {
        if (with_importance && !d_importance)
            return set_error(NYION_ERR_INVALID, "tracked decode: null importance");
        if ((long long)scores_stride < (long long)max_ctx + 2 ||
            (with_importance && importance_stride < max_ctx))
            return set_error(NYION_ERR_INVALID,
                             "tracked decode: scores_stride %d must be >= max_ctx + 2 and "
                             "importance_stride %d >= max_ctx (%d)",
                             scores_stride, importance_stride, max_ctx);
        if (!aligned(d_scores, 4) || (with_importance && !aligned(d_importance, 8)))
            return set_error(NYION_ERR_INVALID, "tracked decode: buffer alignment");
        if (d_prev_scores) {
            if (!d_importance || importance_stride < max_ctx)
                return set_error(NYION_ERR_INVALID,
                                 "pipelined tracked decode: the previous call's importance needs "
                                 "d_prev_importance with importance_stride %d >= max_ctx (%d)",
                                 importance_stride, max_ctx);
            if (!aligned(d_prev_scores, 4) || !aligned(d_importance, 8))
                return set_error(NYION_ERR_INVALID, "pipelined tracked decode: buffer alignment");
            if (d_prev_scores == d_scores)
                return set_error(NYION_ERR_INVALID,
                                 "pipelined tracked decode: the previous scores buffer is this "
                                 "call's scores buffer");
        }
    }
    const bool aligned_path = block_tokens >= 16;
    DecodePlan pl;
    if ((rc = plan_common(pl, batch, n_heads, n_kv_heads, head_dim, kv_dtype,
                          window_main_len(max_ctx, window), window > 0 && global_stride > 0,
                          aligned_path, scale)) != NYION_OK)
        return rc;
    if (use_scratch) {
        if (pl.ws_bytes > kScratchBytes)
            return set_error(NYION_ERR_WORKSPACE,
                             "paged decode (no allocation): this call needs %zu bytes of split-K "
                             "workspace, the library's scratch holds %zu; use "
                             "nyion_paged_decode_attention with a workspace",
                             pl.ws_bytes, kScratchBytes);
        d_workspace = pl.ws_bytes ? decode_scratch_ptr() : nullptr;
        if (pl.ws_bytes && !d_workspace) return NYION_ERR_LAUNCH;
        workspace_bytes = kScratchBytes;
    }
    if ((rc = attach_workspace(pl, d_workspace, workspace_bytes)) != NYION_OK) return rc;
    if (use_scratch && pl.ws_bytes) {
        // the scratch keeps the previous call's contents (another layout may
        // have put partials where this call's counters are): clear them
        const long long n = (long long)pl.chunk * pl.a.n_kv_heads * pl.a.n_hg;
        hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)((n + 255) / 256 < 64 ? (n + 255) / 256 : 64)),
                           dim3(256), 0, stream, pl.a.counters, n);
        if ((rc = check_launch("decode scratch counters")) != NYION_OK) return rc;
    }
    pl.track = track;
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
    a.spec_len = window > 0 ? max_ctx : 0;
    a.scores = d_scores;
    a.scores_stride = scores_stride;
    if (track && d_prev_scores) {
        pl.imp_max_ctx = max_ctx;
        a.imp_scores = d_prev_scores;
        a.imp_out = d_importance;
        a.imp_stride = importance_stride;
    }
    if ((rc = launch_plan(pl, stream)) != NYION_OK || !track || !with_importance) return rc;
    return launch_importance(a, batch, max_ctx, d_importance, importance_stride, stream);
}

// Plan of the attention node over scratch_bytes of its scores buffer.  The
// host knows the length: a segment is exactly ceil(seq_len/16) tiles from
// position 0.  When one workgroup's share covers that, the launch runs whole
// segments (grid = units): no partials, no counters, and so no
// counter-clearing launch.  Otherwise the scores buffer holds the split-K
// partials when it is large enough (halving the grid until the partials fit
// it); failing that, one workgroup covers each head group.
static int node_plan(DecodePlan& pl, uint32_t n_heads, uint32_t n_kv_heads, uint32_t seq_len,
                     uint32_t head_dim, int kv_dtype, size_t scratch_bytes) {
    int rc;
    if ((rc = plan_common(pl, 1, (int)n_heads, (int)n_kv_heads, (int)head_dim, kv_dtype, (int)seq_len,
                          false, true, 0.f)) != NYION_OK)
        return rc;
    DecodeArgs& a = pl.a;
    pl.tiles_max = (int)((seq_len + 15) / 16);
    if (pl.tiles_max <= wg_tiles_for((long long)a.n_kv_heads * a.n_hg * pl.tiles_max)) pl.ws_bytes = 0;
    const int units = a.n_kv_heads * a.n_hg;
    while (pl.ws_bytes > scratch_bytes && pl.grid_bound > units) {
        pl.grid_bound = pl.grid_bound / 2 > units ? pl.grid_bound / 2 : units;
        pl.ws_bytes = ws_layout(pl.grid_bound + units, units, (int)head_dim, nullptr, nullptr);
    }
    if (pl.ws_bytes > scratch_bytes) pl.ws_bytes = 0;  // whole segments: grid = units
    return NYION_OK;
}

extern "C" {

int nyion_paged_decode_attention(const float* d_q, const void* k_pool, const void* v_pool,
                                 const int32_t* block_tables, int max_blocks_per_seq,
                                 const int32_t* ctx_lens, const int32_t* q_pos, int batch,
                                 int n_heads, int n_kv_heads, int head_dim, int block_tokens,
                                 int num_blocks, int kv_dtype, int window, int global_stride,
                                 int max_ctx, float scale, float* d_out, void* d_workspace,
                                 size_t workspace_bytes, nyion_stream_t stream) {
    return paged_decode_common(d_q, k_pool, v_pool, block_tables, max_blocks_per_seq, ctx_lens,
                               q_pos, batch, n_heads, n_kv_heads, head_dim, block_tokens,
                               num_blocks, kv_dtype, window, global_stride, max_ctx, scale, d_out,
                               d_workspace, workspace_bytes, nullptr, 0, nullptr, 0,
                               (hipStream_t)stream);
}

int nyion_paged_decode_attention_noalloc(const float* d_q, const void* k_pool, const void* v_pool,
                                         const int32_t* block_tables, int max_blocks_per_seq,
                                         const int32_t* ctx_lens, const int32_t* q_pos, int batch,
                                         int n_heads, int n_kv_heads, int head_dim,
                                         int block_tokens, int num_blocks, int kv_dtype, int window,
                                         int global_stride, int max_ctx, float scale, float* d_out,
                                         nyion_stream_t stream) {
    return paged_decode_common(d_q, k_pool, v_pool, block_tables, max_blocks_per_seq, ctx_lens,
                               q_pos, batch, n_heads, n_kv_heads, head_dim, block_tokens,
                               num_blocks, kv_dtype, window, global_stride, max_ctx, scale, d_out,
                               nullptr, 0, nullptr, 0, nullptr, 0, (hipStream_t)stream, true);
}

int nyion_paged_decode_attention_tracked(
    const float* d_q, const void* k_pool, const void* v_pool, const int32_t* block_tables,
    int max_blocks_per_seq, const int32_t* ctx_lens, const int32_t* q_pos, int batch, int n_heads,
    int n_kv_heads, int head_dim, int block_tokens, int num_blocks, int kv_dtype, int window,
    int global_stride, int max_ctx, float scale, float* d_out, void* d_workspace,
    size_t workspace_bytes, float* d_scores, int scores_stride, double* d_importance,
    int importance_stride, nyion_stream_t stream) {
    if (!d_scores) {
        clear_error();
        return set_error(NYION_ERR_INVALID, "tracked decode: null scores buffer");
    }
    return paged_decode_common(d_q, k_pool, v_pool, block_tables, max_blocks_per_seq, ctx_lens,
                               q_pos, batch, n_heads, n_kv_heads, head_dim, block_tokens,
                               num_blocks, kv_dtype, window, global_stride, max_ctx, scale, d_out,
                               d_workspace, workspace_bytes, d_scores, scores_stride, d_importance,
                               importance_stride, (hipStream_t)stream);
}

int nyion_paged_decode_attention_scores(
    const float* d_q, const void* k_pool, const void* v_pool, const int32_t* block_tables,
    int max_blocks_per_seq, const int32_t* ctx_lens, const int32_t* q_pos, int batch, int n_heads,
    int n_kv_heads, int head_dim, int block_tokens, int num_blocks, int kv_dtype, int window,
    int global_stride, int max_ctx, float scale, float* d_out, void* d_workspace,
    size_t workspace_bytes, float* d_scores, int scores_stride, nyion_stream_t stream) {
    if (!d_scores) {
        clear_error();
        return set_error(NYION_ERR_INVALID, "tracked decode: null scores buffer");
    }
    return paged_decode_common(d_q, k_pool, v_pool, block_tables, max_blocks_per_seq, ctx_lens,
                               q_pos, batch, n_heads, n_kv_heads, head_dim, block_tokens,
                               num_blocks, kv_dtype, window, global_stride, max_ctx, scale, d_out,
                               d_workspace, workspace_bytes, d_scores, scores_stride, nullptr, 0,
                               (hipStream_t)stream, false, false);
}

int nyion_paged_decode_attention_tracked_pipelined(
    const float* d_q, const void* k_pool, const void* v_pool, const int32_t* block_tables,
    int max_blocks_per_seq, const int32_t* ctx_lens, const int32_t* q_pos, int batch, int n_heads,
    int n_kv_heads, int head_dim, int block_tokens, int num_blocks, int kv_dtype, int window,
    int global_stride, int max_ctx, float scale, float* d_out, void* d_workspace,
    size_t workspace_bytes, float* d_scores, int scores_stride, const float* d_prev_scores,
    double* d_prev_importance, int importance_stride, nyion_stream_t stream) {
    if (!d_scores) {
        clear_error();
        return set_error(NYION_ERR_INVALID, "tracked decode: null scores buffer");
    }
    return paged_decode_common(d_q, k_pool, v_pool, block_tables, max_blocks_per_seq, ctx_lens,
                               q_pos, batch, n_heads, n_kv_heads, head_dim, block_tokens,
                               num_blocks, kv_dtype, window, global_stride, max_ctx, scale, d_out,
                               d_workspace, workspace_bytes, d_scores, scores_stride,
                               d_prev_importance, importance_stride, (hipStream_t)stream, false,
                               false, d_prev_scores);
}

int nyion_paged_decode_importance(const int32_t* ctx_lens, const int32_t* q_pos, int batch,
                                  int n_heads, int window, int global_stride, int max_ctx,
                                  const float* d_scores, int scores_stride, double* d_importance,
                                  int importance_stride, nyion_stream_t stream) {
    clear_error();
    int rc;
    if ((rc = require_device()) != NYION_OK) return rc;
    if (!ctx_lens || !d_scores || !d_importance)
        return set_error(NYION_ERR_INVALID, "decode importance: null ctx_lens/scores/importance");
    if (batch <= 0 || n_heads <= 0 || max_ctx <= 0)
        return set_error(NYION_ERR_INVALID, "decode importance: batch/heads/max_ctx must be positive");
    if ((long long)scores_stride < (long long)max_ctx + 2 || importance_stride < max_ctx)
        return set_error(NYION_ERR_INVALID,
                         "decode importance: scores_stride %d must be >= max_ctx + 2 and "
                         "importance_stride %d >= max_ctx (%d)",
                         scores_stride, importance_stride, max_ctx);
    if (!aligned(d_scores, 4) || !aligned(d_importance, 8))
        return set_error(NYION_ERR_INVALID, "decode importance: buffer alignment");
    // the attended sets exactly as the decode call with these arguments saw them
    DecodeArgs a{};
    a.n_heads = n_heads;
    a.max_len = window_main_len(max_ctx, window);
    a.mode = window > 0 ? MODE_WINDOW : MODE_FULL;
    a.window = window;
    a.global_stride = global_stride;
    a.ctx_lens = ctx_lens;
    a.q_pos = q_pos;
    a.scores = const_cast<float*>(d_scores);
    a.scores_stride = scores_stride;
    return launch_importance(a, batch, max_ctx, d_importance, importance_stride, (hipStream_t)stream);
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

int nyion_zone_decode_attention(const float* d_q, const void* k_pool, const void* v_pool,
                                int64_t pool_units, const int64_t* page_bases, int max_pages_per_seq,
                                int n_layers, int layer, const int32_t* ctx_lens,
                                const int32_t* q_pos, int batch, int n_heads, int n_kv_heads,
                                int head_dim, int kv_dtype, int window, int global_stride,
                                int max_ctx, float scale, float* d_out, void* d_workspace,
                                size_t workspace_bytes, nyion_stream_t stream) {
    clear_error();
    int rc;
    if ((rc = require_device()) != NYION_OK) return rc;
    if (!d_q || !d_out || !page_bases || !ctx_lens)
        return set_error(NYION_ERR_INVALID, "zone decode: null q/out/page_bases/ctx_lens");
    if (!aligned(d_q, 16) || !aligned(d_out, 16))
        return set_error(NYION_ERR_INVALID, "zone decode: q/out must be 16-byte aligned");
    if (kv_dtype != NYION_KV_F32 && kv_dtype != NYION_KV_Q4_20B && kv_dtype != NYION_KV_F16)
        return set_error(NYION_ERR_INVALID, "zone decode: kv_dtype %d", kv_dtype);
    if ((rc = check_pool_ptrs(k_pool, v_pool, kv_dtype)) != NYION_OK) return rc;
    ZoneMap zone;
    if ((rc = make_zone_map(zone, pool_units, max_pages_per_seq, n_layers, layer, n_kv_heads,
                            kv_dtype, "zone decode")) != NYION_OK)
        return rc;
    if (pool_units < 32 * row_elems(head_dim, kv_dtype))
        return set_error(NYION_ERR_INVALID, "zone decode: pools of %lld units hold less than 32 rows",
                         (long long)pool_units);
    if (max_ctx <= 0 || zone_pos(max_ctx - 1).page >= max_pages_per_seq)
        return set_error(NYION_ERR_INVALID,
                         "zone decode: max_ctx %d needs %d pages per sequence, the table has %d",
                         max_ctx, max_ctx > 0 ? zone_pos(max_ctx - 1).page + 1 : 0, max_pages_per_seq);
    DecodePlan pl;
    if ((rc = plan_common(pl, batch, n_heads, n_kv_heads, head_dim, kv_dtype,
                          window_main_len(max_ctx, window), window > 0 && global_stride > 0,
                          true, scale)) != NYION_OK)
        return rc;
    pl.zone = true;  // the aligned walk over 32-token units of zone pages
    if ((rc = attach_workspace(pl, d_workspace, workspace_bytes)) != NYION_OK) return rc;
    DecodeArgs& a = pl.a;
    a.q = d_q;
    a.k = k_pool;
    a.v = v_pool;
    a.ctx_lens = ctx_lens;
    a.q_pos = q_pos;
    a.out = d_out;
    a.token_stride = (int)row_elems(head_dim, kv_dtype);
    a.page_bases = page_bases;
    a.zone = zone;
    a.bt_log2 = kZoneUnitLog2;
    a.mode = window > 0 ? MODE_WINDOW : MODE_FULL;
    a.window = window;
    a.global_stride = global_stride;
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
    // the node's scores buffer: n_heads*seq_len floats, the least any
    // reference caller provides
    const size_t scores_bytes =
        d_scores && aligned(d_scores, 256) ? (size_t)n_heads * seq_len * sizeof(float) : 0;
    DecodePlan pl;
    if ((rc = node_plan(pl, n_heads, n_kv_heads, seq_len, head_dim, kv_dtype, scores_bytes)) != NYION_OK)
        return rc;
    DecodeArgs& a = pl.a;
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

}  // extern "C"

// Split-K scratch of the project-ABI names, which take no scratch argument
// (the CUDA originals cudaMalloc'ed a scores buffer per call): one device
// buffer per (device, stream), allocated by the first call on that stream
// that needs more than the stream's buffer holds and kept until the process
// ends.  Calls on one stream are ordered by the stream; calls on different
// streams use different buffers.  A buffer that has to grow is replaced
// after its stream's queued work is done.
static float* legacy_scratch(hipStream_t stream, size_t bytes) {
    static std::mutex mu;
    static std::map<std::pair<int, uintptr_t>, std::pair<float*, size_t>> bufs;
    const int dev = current_device();
    if (dev < 0) return nullptr;
    std::lock_guard<std::mutex> g(mu);
    auto& e = bufs[{dev, (uintptr_t)stream}];
    if (e.first && e.second >= bytes) return e.first;
    size_t want = (size_t)1 << 20;
    while (want < bytes) want <<= 1;
    if (e.first) {
        if (hipStreamSynchronize(stream) != hipSuccess || hipFree(e.first) != hipSuccess) {
            (void)hipGetLastError();
            set_error(NYION_ERR_LAUNCH, "attention scratch: releasing the stream's buffer failed");
            e = {nullptr, 0};
            return nullptr;
        }
        e = {nullptr, 0};
    }
    void* p = nullptr;
    if (hipMalloc(&p, want) != hipSuccess) {
        (void)hipGetLastError();
        set_error(NYION_ERR_OOM, "attention scratch: hipMalloc of %zu bytes failed", want);
        return nullptr;
    }
    e = {(float*)p, want};
    return (float*)p;
}

// The node with the stream's scratch standing in for d_scores.
static int legacy_node(const float* d_q, const void* d_k, const void* d_v, float* d_out, int n_heads,
                       int n_kv_heads, int seq_len, int head_dim, int kv_stride, int kv_dtype,
                       hipStream_t stream) {
    clear_error();
    if (require_device() != NYION_OK) return -1;
    float* scratch = legacy_scratch(stream, (size_t)n_heads * seq_len * sizeof(float));
    if (!scratch) return -1;
    const int rc = nyion_attention_node(d_q, d_k, d_v, scratch, d_out, (uint32_t)n_heads,
                                        (uint32_t)n_kv_heads, (uint32_t)seq_len, (uint32_t)head_dim,
                                        (uint32_t)kv_stride, kv_dtype, stream);
    return rc == NYION_OK ? 0 : -1;
}

extern "C" {

int gpu_attention_streamed(const float* d_q, const float* d_k_cache, const float* d_v_cache,
                           float* d_output, int n_heads, int n_kv_heads, int seq_len, int head_dim,
                           int kv_stride, nyion_stream_t stream) {
    if (n_heads <= 0 || n_kv_heads <= 0 || seq_len <= 0 || head_dim <= 0 || kv_stride <= 0) {
        set_error(NYION_ERR_INVALID, "gpu_attention_streamed: non-positive size");
        return -1;
    }
    return legacy_node(d_q, d_k_cache, d_v_cache, d_output, n_heads, n_kv_heads, seq_len, head_dim,
                       kv_stride, NYION_KV_F32, (hipStream_t)stream);
}

int gpu_attention_device(const float* d_q, const float* d_k_cache, const float* d_v_cache,
                         float* d_output, int n_heads, int n_kv_heads, int seq_len, int head_dim,
                         int kv_stride) {
    return gpu_attention_streamed(d_q, d_k_cache, d_v_cache, d_output, n_heads, n_kv_heads, seq_len,
                                  head_dim, kv_stride, nullptr);
}

size_t nyion_attention_node_scratch_bytes(uint32_t n_heads, uint32_t n_kv_heads, uint32_t seq_len,
                                          uint32_t head_dim) {
    DecodePlan pl;
    const size_t avail = (size_t)n_heads * seq_len * sizeof(float);
    const int rc = node_plan(pl, n_heads, n_kv_heads, seq_len, head_dim, NYION_KV_F32, avail);
    clear_error();
    return rc == NYION_OK ? pl.ws_bytes : 0;
}

}  // extern "C"

// The attention node captured on a private stream and instantiated.
static void* graph_create_node(const float* d_q, const void* d_k_cache, const void* d_v_cache,
                               float* d_scores, float* d_output, int n_heads, int n_kv_heads,
                               int seq_len, int head_dim, int kv_stride, int kv_dtype) {
    clear_error();
    if (require_device() != NYION_OK) return nullptr;
    if (n_heads <= 0 || n_kv_heads <= 0 || seq_len <= 0 || head_dim <= 0 || kv_stride <= 0) {
        set_error(NYION_ERR_INVALID, "gpu_graph_create_attention: non-positive size");
        return nullptr;
    }
    hipStream_t s = nullptr;
    if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) {
        set_error(NYION_ERR_LAUNCH, "gpu_graph_create_attention: stream: %s", hipGetErrorString(hipGetLastError()));
        return nullptr;
    }
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    int rc = NYION_OK;
    if (hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal) != hipSuccess) {
        rc = set_error(NYION_ERR_LAUNCH, "gpu_graph_create_attention: begin capture failed");
    } else {
        // the node records its launches (and, with d_scores, the fill kernel
        // that clears its arrival counters) on the capturing stream
        rc = nyion_attention_node(d_q, d_k_cache, d_v_cache, d_scores, d_output, (uint32_t)n_heads,
                                  (uint32_t)n_kv_heads, (uint32_t)seq_len, (uint32_t)head_dim,
                                  (uint32_t)kv_stride, kv_dtype, s);
        const hipError_t e = hipStreamEndCapture(s, &graph);
        if (rc == NYION_OK && e != hipSuccess)
            rc = set_error(NYION_ERR_LAUNCH, "gpu_graph_create_attention: end capture: %s", hipGetErrorString(e));
        if (rc == NYION_OK && hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) != hipSuccess) {
            rc = set_error(NYION_ERR_LAUNCH, "gpu_graph_create_attention: instantiate failed");
            exec = nullptr;
        }
    }
    if (graph) (void)hipGraphDestroy(graph);
    (void)hipStreamDestroy(s);
    return rc == NYION_OK ? (void*)exec : nullptr;
}

extern "C" {

void* gpu_graph_create_attention(const float* d_q, const float* d_k_cache, const float* d_v_cache,
                                 float* d_scores, float* d_output, int n_heads, int n_kv_heads,
                                 int seq_len, int head_dim, int kv_stride) {
    return graph_create_node(d_q, d_k_cache, d_v_cache, d_scores, d_output, n_heads, n_kv_heads,
                             seq_len, head_dim, kv_stride, NYION_KV_F32);
}

void* gpu_graph_create_attention_half(const float* d_q, const uint16_t* d_k_cache,
                                      const uint16_t* d_v_cache, float* d_scores, float* d_output,
                                      int n_heads, int n_kv_heads, int seq_len, int head_dim,
                                      int kv_stride) {
    return graph_create_node(d_q, d_k_cache, d_v_cache, d_scores, d_output, n_heads, n_kv_heads,
                             seq_len, head_dim, kv_stride, NYION_KV_F16);
}

int gpu_attention_streamed_half(const float* d_q, const uint16_t* d_k_cache,
                                const uint16_t* d_v_cache, float* d_output, int n_heads,
                                int n_kv_heads, int seq_len, int head_dim, int kv_stride,
                                nyion_stream_t stream) {
    if (n_heads <= 0 || n_kv_heads <= 0 || seq_len <= 0 || head_dim <= 0 || kv_stride <= 0) {
        set_error(NYION_ERR_INVALID, "gpu_attention_streamed_half: non-positive size");
        return -1;
    }
    return legacy_node(d_q, d_k_cache, d_v_cache, d_output, n_heads, n_kv_heads, seq_len, head_dim,
                       kv_stride, NYION_KV_F16, (hipStream_t)stream);
}

int gpu_graph_replay_attention(void* graph_handle, nyion_stream_t stream) {
    clear_error();
    if (!graph_handle) {
        set_error(NYION_ERR_INVALID, "gpu_graph_replay_attention: null graph");
        return -1;
    }
    const hipError_t e = hipGraphLaunch((hipGraphExec_t)graph_handle, (hipStream_t)stream);
    if (e != hipSuccess) {
        set_error(NYION_ERR_LAUNCH, "gpu_graph_replay_attention: %s", hipGetErrorString(e));
        return -1;
    }
    return 0;
}

void gpu_graph_destroy(void* graph_handle) {
    if (graph_handle) (void)hipGraphExecDestroy((hipGraphExec_t)graph_handle);
}

}  // extern "C"
