// prefill_attention.hip — causal prefill attention on MFMA (gfx950).
//
// The reference prefills by calling ops::attention once per token with
// seq_len = abs_pos + 1 (swamp-engine/src/executor.rs:132-137, ops.rs:170-278):
// row i of a chunk that starts at position p attends to keys [0, p + i], the
// p cached ones first.  Here one kernel computes all rows of a chunk as a
// flash-attention style pass: bf16 q, k, v (and the p history tokens' k, v)
// in, fp32 accumulate, f32 out.
//
// Work decomposition.  A workgroup owns one kv head and eight (four at
// head_dim 64) (q head, 32-row block) pairs that read the same K/V: for GQA
// 4:1 these are the four q heads of the group on 64 rows, so every K/V tile
// staged in LDS feeds eight wavefronts.  Workgroups are numbered so that each XCD
// (workgroup id mod 8) takes a contiguous run of the (kv head, row block)
// list: with 8 kv heads every XCD's L2 holds the K/V of one head.  Within a
// head, row blocks are issued longest-first.
//
// Per 64-key tile:
//   K tile  [64][D] bf16 -> LDS, rows padded by 16 bytes
//   V tile  [64][D] bf16 -> LDS as fp16, transposed to V^T [D][64] (key
//           pairs packed into 32-bit words, rows padded by 16 bytes)
//   S^T[64 keys][32 rows] = K . Q^T      v_mfma_f32_32x32x16_bf16, Q^T from
//                                        registers (loaded once)
//   online softmax per row (rows are lanes; 32 keys per lane per half), the
//   running max moved only when a half's weights against it grow too large
//   O[32 rows][D] += P . V               v_mfma_f32_32x32x16_f16, A = P in
//                                        fp16 converted in registers from the
//                                        S^T accumulators, B = V^T from LDS
// LDS holds two tiles: the next tile is written from registers (its global
// loads were issued a whole tile earlier) while the current one is consumed,
// with one barrier per tile.
//
// fp16 for P and V keeps 11 significant bits (p <= 2^14 after the lazy max),
// so the P.V product stays within the f32 reference's tolerance; V must lie
// within the fp16 range (|v| <= 65504).
#include <math.h>

#include "common.hpp"
#include "kv_write.hpp"

namespace nyion {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

int kv_write_impl(void* k_pool, void* v_pool, const int32_t* block_table, int block_tokens,
                  int num_blocks, int n_kv_heads, int head_dim, int kv_dtype, int start_pos,
                  int n_tokens, const float* k, const float* v, hipStream_t stream);
int kv_write_bf16_impl(void* k_pool, void* v_pool, const int32_t* block_table, int block_tokens,
                       int num_blocks, int n_kv_heads, int head_dim, int kv_dtype, int start_pos,
                       int n_tokens, const uint16_t* k, const uint16_t* v, hipStream_t stream);

struct PrefillArgs {
    const uint16_t* q;  // [N][Hq][D]
    const uint16_t* k;  // [N][Hkv][D]
    const uint16_t* v;
    const uint16_t* kh;  // [n_hist][Hkv][D]: the sequence's tokens before the chunk
    const uint16_t* vh;
    float* out;  // [N][Hq][D]
    int n;
    int n_hist;
    int n_heads;
    int n_kv_heads;
    int group;     // q heads per kv head
    int hw;        // q heads per workgroup (4, 2 or 1: the largest dividing the group)
    int rb_per_wg; // 32-row blocks per workgroup (wavefronts / hw)
    int n_rbg;     // row-block groups
    int n_items;   // kv heads x head subsets x row-block groups
    int causal;
    float scale_log2;
    // the chunk's paged K/V write into f32 or binary16 pools, done by the
    // kernel (kv_write != 0): each workgroup of head subset 0 writes its own
    // tokens' rows for its kv head after its attention work
    WriteArgs kvw;
    int kv_write;
    int kv_f16;
    int v_check;  // no pools: the same workgroups only check their V rows' range
};

constexpr int BN = 64;  // keys per tile

// Threads per workgroup: eight wavefronts at head_dim 128 (two per SIMD, one
// workgroup per CU), so each K/V tile staged in LDS feeds eight
// (q head, 32-row) pairs; four at head_dim 64.
template <int D>
constexpr int prefill_threads() {
    return D == 128 ? 512 : 256;
}
// Largest sum of one lane's 16 softmax weights of a half that is used as
// computed; above it the half's row max is taken and the weights redone.
// Every weight enters the P.V product as binary16, so the limit stays well
// below 65504.
constexpr float kPrefillSumLimit = 16384.0f;

// LDS tiles, padded by 16 bytes per row so that every lane's reads are one
// base address plus compile-time offsets (no per-read address registers):
//   K   [BN][D] bf16, row stride D*2+16 bytes;
//   V^T [D][BN] fp16, row stride BN*2+16 bytes.  Within each 16-key group the
//       keys sit in the order 0-3, 8-11, 4-7, 12-15, which is the order of
//       the PV k-step's B operand (lane half h holds keys 4h..4h+3 and
//       8+4h..8+4h+3), so one 16-byte read fetches it.
template <int D>
struct PrefillLds {
    static constexpr int KROW = D * 2 + 16;   // bytes
    static constexpr int VROW = BN * 2 + 16;  // bytes
    static constexpr int KBYTES = BN * KROW;
    static constexpr int VBYTES = D * VROW;
    static constexpr int BUF = KBYTES + VBYTES;
};

// Position of key w (0..15) of a 16-key group in V^T row order.
__device__ __forceinline__ int vt_pos(int w) {
    return (w & 3) | (((w >> 3) & 1) << 2) | (((w >> 2) & 1) << 3);
}

typedef _Float16 halfx2 __attribute__((ext_vector_type(2)));

// max(v, v of lane ^ 32): v_permlane32_swap exchanges the two 32-lane halves
// without going through LDS (the result pair holds v and its partner in
// either order, depending on the half).
__device__ __forceinline__ float max_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Two f32 -> one word of two fp16 (lo in the low half), round to nearest
// even; one v_cvt_pk_f16_f32.
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, halfx2{(_Float16)lo, (_Float16)hi});
}

// One tile's K (or V) in registers between its global loads and its LDS
// stores (K chunk u: key (tid+NT*u) / (D/8); V unit u: key pair and 8 dims).
// K is staged one tile ahead of V.
template <int D>
struct KStage {
    static constexpr int NT = prefill_threads<D>();
    static constexpr int LOADS = BN * (D / 8) / NT;
    u32x4 k[LOADS];
};
template <int D>
struct VStage {
    static constexpr int NT = prefill_threads<D>();
    static constexpr int UNITS = (BN / 2) * (D / 8) / NT;
    u32x4 v0[UNITS];
    u32x4 v1[UNITS];
};

// Buffer descriptor of a K or V source: n tokens of tok_stride elements
// from `base` (the bytes of one kv head's rows; the host keeps n *
// n_kv_heads * head_dim below 2^30, so every byte offset fits 31 bits).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t source_rsrc(const uint16_t* base, int n,
                                                               int tok_stride) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, n * tok_stride * 2, 0x00020000);
}

// Loads of the tile whose first key is token kt of a source of n tokens
// (kt may be negative for the first history tile).  A tile inside [0, n)
// is read with buffer loads (one per-thread offset, the tile offset in a
// scalar register); only a tile that reaches outside clamps K rows and
// zeroes V rows.
template <int D>
__device__ __forceinline__ void stage_load_k(KStage<D>& st, const uint16_t* kbase, int tok_stride,
                                             int n, int kt, int tid) {
    constexpr int CPR = D / 8;
    constexpr int STEP = KStage<D>::NT / CPR;  // keys between a thread's chunks
    if (kt >= 0 && kt + BN <= n) {
        // buffer loads: the source's descriptor and the tile offset in scalar
        // registers, one per-thread 32-bit offset (no per-lane address math)
        const __amdgpu_buffer_rsrc_t r = source_rsrc(kbase, n, tok_stride);
        const int off = ((tid / CPR) * tok_stride + 8 * (tid % CPR)) * 2;
        const int t0 = kt * tok_stride * 2, step = STEP * tok_stride * 2;
#pragma unroll
        for (int u = 0; u < KStage<D>::LOADS; u++)
            st.k[u] = __builtin_amdgcn_raw_buffer_load_b128(r, off, t0 + u * step, 0);
        return;
    }
#pragma unroll
    for (int u = 0; u < KStage<D>::LOADS; u++) {
        const int t = min(max(kt + tid / CPR + u * STEP, 0), n - 1);  // outside: finite, masked
        st.k[u] = *(const u32x4*)(kbase + (long long)t * tok_stride + 8 * (tid % CPR));
    }
}

template <int D>
__device__ __forceinline__ void stage_load_v(VStage<D>& st, const uint16_t* vbase, int tok_stride,
                                             int n, int kt, int tid) {
    constexpr int STEP = 8 * (VStage<D>::NT / (BN / 2));  // dims between a thread's units
    const int t = kt + 2 * (tid % (BN / 2));
    const int d0 = 8 * (tid / (BN / 2));
    if (kt >= 0 && kt + BN <= n) {
        const __amdgpu_buffer_rsrc_t r = source_rsrc(vbase, n, tok_stride);
        const int off = ((t - kt) * tok_stride + d0) * 2;
        const int t0 = kt * tok_stride * 2, row = tok_stride * 2;
#pragma unroll
        for (int u = 0; u < VStage<D>::UNITS; u++) {
            st.v0[u] = __builtin_amdgcn_raw_buffer_load_b128(r, off + 2 * STEP * u, t0, 0);
            st.v1[u] = __builtin_amdgcn_raw_buffer_load_b128(r, off + 2 * STEP * u, t0 + row, 0);
        }
        return;
    }
#pragma unroll
    for (int u = 0; u < VStage<D>::UNITS; u++) {
        st.v0[u] = t >= 0 && t < n ? *(const u32x4*)(vbase + (long long)t * tok_stride + d0 + STEP * u)
                                   : u32x4{0, 0, 0, 0};
        st.v1[u] = t + 1 >= 0 && t + 1 < n
                       ? *(const u32x4*)(vbase + (long long)(t + 1) * tok_stride + d0 + STEP * u)
                       : u32x4{0, 0, 0, 0};
    }
}

// The tile at key kt (relative to the chunk): keys below 0 come from the
// history, the rest from the chunk.  kt is uniform, so the selects are
// scalar and one copy of the loads serves both sources.
template <int D>
__device__ __forceinline__ void load_k_tile(KStage<D>& st, const PrefillArgs& a,
                                            const uint16_t* kbase, const uint16_t* khbase,
                                            int tok_stride, int kt, int tid) {
    const bool hist = kt < 0;
    stage_load_k<D>(st, hist ? khbase : kbase, tok_stride, hist ? a.n_hist : a.n,
                    hist ? kt + a.n_hist : kt, tid);
}
template <int D>
__device__ __forceinline__ void load_v_tile(VStage<D>& st, const PrefillArgs& a,
                                            const uint16_t* vbase, const uint16_t* vhbase,
                                            int tok_stride, int kt, int tid) {
    const bool hist = kt < 0;
    stage_load_v<D>(st, hist ? vhbase : vbase, tok_stride, hist ? a.n_hist : a.n,
                    hist ? kt + a.n_hist : kt, tid);
}

template <int D>
__device__ __forceinline__ void stage_store_k(const KStage<D>& st, unsigned char* kslot, int tid) {
    using L = PrefillLds<D>;
    constexpr int CPR = D / 8;
#pragma unroll
    for (int u = 0; u < KStage<D>::LOADS; u++) {
        const int id = tid + KStage<D>::NT * u;
        *(u32x4*)(kslot + (id / CPR) * L::KROW + 16 * (id % CPR)) = st.k[u];
    }
}

template <int D>
__device__ __forceinline__ void stage_store_v(const VStage<D>& st, unsigned char* vslot, int tid) {
    using L = PrefillLds<D>;
#pragma unroll
    for (int u = 0; u < VStage<D>::UNITS; u++) {
        const int id = tid + VStage<D>::NT * u;
        const int key = 2 * (id % (BN / 2));
        const int dc = id / (BN / 2);
        const int col = (key & ~15) + vt_pos(key & 15);  // even: keys key, key+1
#pragma unroll
        for (int e = 0; e < 8; e++) {
            // dim 8dc+e: low half from key, high half from key+1
            // bf16 -> f32 is a 16-bit shift (or mask for the high half); bf16
            // values in the fp16 range convert to fp16 exactly
            const uint32_t x0 = st.v0[u][e >> 1], x1 = st.v1[u][e >> 1];
            const float lo = __uint_as_float((e & 1) ? (x0 & 0xffff0000u) : (x0 << 16));
            const float hi = __uint_as_float((e & 1) ? (x1 & 0xffff0000u) : (x1 << 16));
            *(uint32_t*)(vslot + (8 * dc + e) * L::VROW + 2 * col) = pack_f16x2(lo, hi);
        }
    }
}

template <int D>
__global__ __launch_bounds__(prefill_threads<D>(), 512 / prefill_threads<D>()) void prefill_kernel(
    PrefillArgs a) {
    using L = PrefillLds<D>;
    constexpr int DT = D / 32;  // output dim tiles
    constexpr int KS = D / 16;  // k-steps of the S product

    // three K slots, then two V^T slots
    __shared__ __attribute__((aligned(16))) unsigned char lds[3 * L::KBYTES + 2 * L::VBYTES];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 31;   // row (S^T col) / dim within tile (O col)
    const int h = lane >> 5;   // half

    // workgroup -> work item: XCD x = id % 8 takes items [x*per, (x+1)*per)
    const int per = (a.n_items + 7) / 8;
    const int item = ((int)blockIdx.x & 7) * per + ((int)blockIdx.x >> 3);
    if (item >= a.n_items) return;
    const int p = item / a.n_rbg;                         // kv head * subsets + subset
    const int rbg = a.n_rbg - 1 - (item - p * a.n_rbg);  // longest first
    const int subsets = a.group / a.hw;
    const int g = p / subsets;
    const int hs = p - g * subsets;
    const int head = g * a.group + hs * a.hw + (wave % a.hw);
    const int row0 = (rbg * a.rb_per_wg + wave / a.hw) * 32;
    const int wg_row_end = min(a.n, (rbg + 1) * a.rb_per_wg * 32);
    // Keys are numbered relative to the chunk: history token t is key
    // t - n_hist (negative), chunk token t is key t.  History tiles end at
    // key -1, so the chunk's tiles start at key 0 whatever n_hist is, and
    // only the first history tile can be partial.
    const int key_end = a.causal ? wg_row_end : a.n;
    const int n_htiles = (a.n_hist + BN - 1) / BN;
    const int n_tiles = n_htiles + (key_end + BN - 1) / BN;
    const int kt0 = -n_htiles * BN;
    const int key_lo = -a.n_hist;                                  // first key of every row
    const int lim = a.causal ? min(row0 + j, a.n - 1) : a.n - 1;  // last key of this lane's row

    // Q^T operand (B of S^T = K.Q^T): row row0+j, dims 16s + 8h .. +7
    bf16x8 qreg[KS];
    {
        const int r = row0 + j;
        const bool ok = r < a.n;
        const uint16_t* qrow = a.q + ((long long)min(r, a.n - 1) * a.n_heads + head) * D;
#pragma unroll
        for (int s = 0; s < KS; s++) {
            uint4 t = ok ? *(const uint4*)(qrow + 16 * s + 8 * h) : uint4{0, 0, 0, 0};
            qreg[s] = __builtin_bit_cast(bf16x8, t);
        }
    }

    floatx16 o[DT];
#pragma unroll
    for (int t = 0; t < DT; t++) o[t] = floatx16{};
    float mrun = -1e30f;  // finite: exp2(s - mrun) of a masked s is 0, never NaN
    float lrun = 0.f;

    const uint16_t* kbase = a.k + (long long)g * D;
    const uint16_t* vbase = a.v + (long long)g * D;
    const uint16_t* khbase = a.kh + (long long)g * D;
    const uint16_t* vhbase = a.vh + (long long)g * D;
    const int tok_stride = a.n_kv_heads * D;
    unsigned char* const kslot0 = lds;
    unsigned char* const vslot0 = lds + 3 * L::KBYTES;
    KStage<D> kst;
    VStage<D> vst;

    // S^T of 32-key half kb of the tile in K slot `ks` (K rows kb*32 + j,
    // chunk 2s + h)
    auto scores_half = [&](const unsigned char* ks, int kb) {
        const unsigned char* kp = ks + (kb * 32 + j) * L::KROW + 16 * h;
        floatx16 st = floatx16{};
#pragma unroll
        for (int s0_ = 0; s0_ < KS; s0_ += 4) {
            bf16x8 kf[4];
#pragma unroll
            for (int s = 0; s < 4; s++) kf[s] = __builtin_bit_cast(bf16x8, *(const uint4*)(kp + 32 * (s0_ + s)));
#pragma unroll
            for (int s = 0; s < 4; s++) st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[s], qreg[s0_ + s], st, 0, 0, 0);
        }
        return st;
    };

    // Online softmax of half kb of the tile at key kt and O += P.V over its
    // two 16-key k-steps (consume_half).  Lane holds row row0+j, keys
    // kt + 32kb + 8(r/4) + 4h + r%4 in st[r].  The exps come before any
    // branch, so they interleave with the MFMAs issued before them.
    // Causal / range mask of half kb of the tile at key kt: the key of
    // st[r] is kt + 32kb + 4h + c(r), c(r) = 8(r/4) + r%4, compared as the
    // constant c(r) against this lane's bounds.
    auto mask_half = [&](floatx16& st, int kt, int kb) {
        const int hi = lim - kt - 32 * kb - 4 * h;
        const int lo = key_lo - kt - 32 * kb - 4 * h;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int c = 8 * (r >> 2) + (r & 3);
            st[r] = c <= hi && c >= lo ? st[r] : -INFINITY;
        }
    };
    // B operands of the PV product of half kb: V^T row 32dt + j, the 8 keys
    // of k-step t = 2kb + t2.  They are read before the softmax that
    // produces P, so the PV MFMAs do not wait on LDS.
    auto load_vhalf = [&](const unsigned char* vs, int kb, halfx8 (&vb)[2][DT]) {
        const unsigned char* vp = vs + j * L::VROW + 16 * h + 64 * kb;
#pragma unroll
        for (int t2 = 0; t2 < 2; t2++)
#pragma unroll
            for (int dt = 0; dt < DT; dt++)
                vb[t2][dt] = __builtin_bit_cast(halfx8, *(const uint4*)(vp + 32 * dt * L::VROW + 32 * t2));
    };
    auto consume_half = [&](floatx16 st, const halfx8 (&vb)[2][DT]) {
        // p = exp2(s*scale - m), one FMA + one exp per score, converted to
        // fp16 pairs; the row sum adds the f32 values in two chains of plain
        // adds (a v_dot2 sum of the fp16 pairs competes with the MFMAs for
        // issue and measured 1-2 % slower).  A operands of the PV product: k-step
        // t2 of this half holds keys 16t2 + 8(e/4) + 4h + e%4 (e = 0..7).
        halfx8 pa[2];
        float psum = 0.f;
        auto exps = [&]() {
            float sa = 0.f, sb = 0.f;
#pragma unroll
            for (int t2 = 0; t2 < 2; t2++)
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(st[8 * t2 + e], a.scale_log2, -mrun));
                    const float p1 =
                        __builtin_amdgcn_exp2f(__builtin_fmaf(st[8 * t2 + e + 1], a.scale_log2, -mrun));
                    sa += p0;
                    sb += p1;
                    pa[t2][e] = (_Float16)p0;
                    pa[t2][e + 1] = (_Float16)p1;
                }
            psum = sa + sb;
        };
        // The running max m (log2 units, scaled) is not recomputed per half:
        // the exps run against the current m, and only when some lane's sum
        // of p exceeds kPrefillSumLimit (so some p may be past it, up to an
        // fp16 overflow) is the half's row max taken, m raised to it, O and
        // the row sum rescaled and the exps redone.  Every kept p is then at
        // most kPrefillSumLimit.  The first half of every row takes this
        // path (m starts at -1e30, so its p are inf); a NaN sum (NaN inputs)
        // does not, and propagates as in the f32 reference.
        exps();
        if (__any(psum > kPrefillSumLimit)) {
            float mt = -INFINITY;
#pragma unroll
            for (int r = 0; r < 16; r++) mt = fmaxf(mt, st[r]);
            mt = max_xor32(mt) * a.scale_log2;  // scale > 0: max commutes
            const float mnew = fmaxf(mrun, mt);
            const float alpha = __builtin_amdgcn_exp2f(mrun - mnew);
            mrun = mnew;
            lrun *= alpha;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                // O reg r of this lane is row 8(r/4) + 4h + r%4
                const float ar = __shfl(alpha, 8 * (r >> 2) + 4 * h + (r & 3));
#pragma unroll
                for (int t = 0; t < DT; t++) o[t][r] *= ar;
            }
            exps();
        }
        lrun += psum;
#pragma unroll
        for (int t2 = 0; t2 < 2; t2++)
#pragma unroll
            for (int dt = 0; dt < DT; dt++)
                o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(pa[t2], vb[t2][dt], o[dt], 0, 0, 0);
    };
    auto tile_masked = [&](int kt) {
        return (kt + BN > a.n) || (a.causal && kt + BN - 1 > row0) || kt < key_lo;
    };
    auto kslot = [&](int it) { return kslot0 + (it % 3) * L::KBYTES; };

    // Pipeline over 32-key halves: the S MFMAs of the next half are issued
    // before the softmax of the current one, so the matrix and vector pipes
    // have independent work.  At the top of iteration it: K slots hold
    // tiles it and it+1, V slot it&1 holds tile it, s0 = S of tile it's
    // first half, and the staging registers hold K of tile it+2 and V of
    // tile it+1.  The iteration writes the staged K into the slot of tile
    // it-1 and the staged V into the other V slot (both last read one
    // iteration ago), issues the next global loads and synchronises once.
    // Prologue: K and V of tile 0 and K of tile 1 in one round of loads,
    // then K of tile 2 and V of tile 1 requested as soon as the staging
    // registers are in LDS.
    {
        KStage<D> kst1;
        load_k_tile<D>(kst, a, kbase, khbase, tok_stride, kt0, tid);
        load_v_tile<D>(vst, a, vbase, vhbase, tok_stride, kt0, tid);
        if (n_tiles > 1) load_k_tile<D>(kst1, a, kbase, khbase, tok_stride, kt0 + BN, tid);
        stage_store_k<D>(kst, kslot0, tid);
        stage_store_v<D>(vst, vslot0, tid);
        if (n_tiles > 1) stage_store_k<D>(kst1, kslot0 + L::KBYTES, tid);
    }
    if (n_tiles > 2) load_k_tile<D>(kst, a, kbase, khbase, tok_stride, kt0 + 2 * BN, tid);
    if (n_tiles > 1) load_v_tile<D>(vst, a, vbase, vhbase, tok_stride, kt0 + BN, tid);
    __syncthreads();
    floatx16 s0 = scores_half(kslot0, 0);

    auto step = [&](int it, bool masked) {
        const int kt = kt0 + it * BN;
        const unsigned char* vs = vslot0 + (it & 1) * L::VBYTES;
        halfx8 vb[2][DT];
        // Waves w and w + 4 of the workgroup share a SIMD, and at equal
        // priority the older one wins every issue conflict: it reached the
        // barrier ~1100 cycles before its partner on every tile.  The younger
        // wave takes priority for the first half of the step, so the two
        // arrive together (waits ~270 / ~170 cycles; 1-2 % faster).
        if (wave >= 4) __builtin_amdgcn_s_setprio(1);
        load_vhalf(vs, 0, vb);
        if (masked) mask_half(s0, kt, 0);
        floatx16 s1 = scores_half(kslot(it), 1);
        consume_half(s0, vb);
        s0 = scores_half(kslot(it + 1), 0);
        load_vhalf(vs, 1, vb);
        if (wave >= 4) __builtin_amdgcn_s_setprio(0);
        if (masked) mask_half(s1, kt, 1);
        consume_half(s1, vb);
        // a slot past the last tile is written and never read
        stage_store_k<D>(kst, kslot(it + 2), tid);
        stage_store_v<D>(vst, vslot0 + ((it + 1) & 1) * L::VBYTES, tid);
        if (it + 3 < n_tiles) load_k_tile<D>(kst, a, kbase, khbase, tok_stride, kt + 3 * BN, tid);
        if (it + 2 < n_tiles) load_v_tile<D>(vst, a, vbase, vhbase, tok_stride, kt + 2 * BN, tid);
        __syncthreads();
    };
    int it = 0;
    if (n_tiles > 1 && tile_masked(kt0)) step(it++, true);  // partial first history tile
    for (; it + 1 < n_tiles && !tile_masked(kt0 + it * BN); it++) step(it, false);
    for (; it + 1 < n_tiles; it++) step(it, true);
    {
        const int it = n_tiles - 1;
        const int kt = kt0 + it * BN;
        const unsigned char* vs = vslot0 + (it & 1) * L::VBYTES;
        floatx16 s1 = scores_half(kslot(it), 1);
        if (tile_masked(kt)) {
            mask_half(s0, kt, 0);
            mask_half(s1, kt, 1);
        }
        halfx8 vb[2][DT];
        load_vhalf(vs, 0, vb);
        consume_half(s0, vb);
        load_vhalf(vs, 1, vb);
        consume_half(s1, vb);
    }

    // epilogue: divide by the row sums and store
    const float lt = lrun + __shfl_xor(lrun, 32);
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int rr = 8 * (r >> 2) + 4 * h + (r & 3);
        const float lr = __shfl(lt, rr);
        const int rowg = row0 + rr;
        if (rowg < a.n) {
            const float inv = 1.0f / lr;
            float* orow = a.out + ((long long)rowg * a.n_heads + head) * D;
#pragma unroll
            for (int dt = 0; dt < DT; dt++) orow[32 * dt + j] = o[dt][r] * inv;
        }
    }

    // this workgroup's tokens' K/V rows for kv head g into the paged pools
    // (every (token, kv head) by exactly one workgroup), with the V range
    // check the binary16 P.V product needs; without pools, the check alone
    if ((a.kv_write || a.v_check) && hs == 0) {
        constexpr int VEC = D / 4;
        const int r0 = rbg * a.rb_per_wg * 32;
        const int r1 = min(a.n, r0 + a.rb_per_wg * 32);
        float vmax = 0.f;
        for (int i = tid; i < (r1 - r0) * VEC; i += prefill_threads<D>()) {
            const int r = r0 + i / VEC, x = i % VEC;
            if (!a.kv_write)
                vmax = fmaxf(vmax, v_absmax(*(const uint2*)(a.v + ((long long)r * a.n_kv_heads + g) * D + 4 * x)));
            else
                vmax = fmaxf(vmax, a.kv_f16 ? write_kv_vec<true>(a.kvw, r, g, x)
                                            : write_kv_vec<false>(a.kvw, r, g, x));
        }
        report_range(a.kvw.status, vmax >= 65520.f, kRangePrefillV);
    }
}

}  // namespace nyion

using namespace nyion;

static int prefill_impl(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                        const uint16_t* k_hist, const uint16_t* v_hist, int n_hist, int n,
                        int n_heads, int n_kv_heads, int head_dim, int causal, float scale,
                        float* out, void* k_pool, void* v_pool, const int32_t* block_table,
                        int block_tokens, int num_blocks, int kv_dtype, int start_pos,
                        nyion_stream_t stream) {
    clear_error();
    int rc;
    if ((rc = require_device()) != NYION_OK) return rc;
    if (!q || !k || !v || !out) return set_error(NYION_ERR_INVALID, "prefill: null q/k/v/out");
    if (n <= 0 || n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads)
        return set_error(NYION_ERR_INVALID, "prefill: n=%d heads=%d/%d", n, n_heads, n_kv_heads);
    if (head_dim != 64 && head_dim != 128)
        return set_error(NYION_ERR_UNSUPPORTED, "prefill: head_dim %d (supported: 64, 128)", head_dim);
    if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || !aligned(out, 16))
        return set_error(NYION_ERR_INVALID, "prefill: q/k/v/out must be 16-byte aligned");
    if (n_hist < 0) return set_error(NYION_ERR_INVALID, "prefill: n_hist %d", n_hist);
    if (n_hist > 0 && (!k_hist || !v_hist || !aligned(k_hist, 16) || !aligned(v_hist, 16)))
        return set_error(NYION_ERR_INVALID, "prefill: history needs 16-byte aligned k_hist/v_hist");
    // K/V byte offsets are 32-bit (buffer loads): below 2^30 elements per source
    if ((long long)n * n_kv_heads * head_dim >= (1LL << 30) ||
        (long long)n * n_heads * head_dim >= (1LL << 40))
        return set_error(NYION_ERR_UNSUPPORTED, "prefill: chunk of %d tokens too large", n);
    if ((long long)n_hist * n_kv_heads * head_dim >= (1LL << 30) ||
        (long long)n_hist + n + 2 * BN >= (1LL << 31))
        return set_error(NYION_ERR_UNSUPPORTED, "prefill: history of %d tokens too large", n_hist);
    const int group = n_heads / n_kv_heads;
    // q heads per workgroup: 4, 2 or 1, the largest that divides the group
    // (and so also the wavefront count); the remaining wavefronts take more
    // row blocks of the same heads
    int hw = 4;
    while (group % hw) hw /= 2;
    const int waves = (head_dim == 128 ? 512 : 256) / 64;
    PrefillArgs a{};
    a.q = q;
    a.k = k;
    a.v = v;
    // with no history the history pointers are never read; they alias k/v
    a.kh = n_hist > 0 ? k_hist : k;
    a.vh = n_hist > 0 ? v_hist : v;
    a.out = out;
    a.n = n;
    a.n_hist = n_hist;
    a.n_heads = n_heads;
    a.n_kv_heads = n_kv_heads;
    a.group = group;
    a.hw = hw;
    a.rb_per_wg = waves / hw;
    const int rows_per_wg = 32 * a.rb_per_wg;
    a.n_rbg = (n + rows_per_wg - 1) / rows_per_wg;
    const long long items = (long long)n_kv_heads * (group / hw) * a.n_rbg;
    if (items > (1LL << 30)) return set_error(NYION_ERR_UNSUPPORTED, "prefill: %lld work items", items);
    a.n_items = (int)items;
    a.causal = causal ? 1 : 0;
    const float sc = scale > 0.f ? scale : 1.0f / sqrtf((float)head_dim);
    a.scale_log2 = sc * 1.4426950408889634f;
    if (k_pool || v_pool) {
        if (!k_pool || !v_pool || !block_table)
            return set_error(NYION_ERR_INVALID, "prefill: KV write needs k_pool, v_pool and block_table");
        if (kv_dtype == NYION_KV_F32 || kv_dtype == NYION_KV_F16) {
            if ((rc = prefill_write_args(a.kvw, k_pool, v_pool, block_table, block_tokens, num_blocks,
                                         n_kv_heads, head_dim, kv_dtype, start_pos, n, k, v)) !=
                NYION_OK)
                return rc;
            a.kv_write = 1;
            a.kv_f16 = kv_dtype == NYION_KV_F16;
        }
    } else {
        a.v_check = 1;
        a.kvw.status = device_status_word();
    }
    dim3 grid(8 * ((a.n_items + 7) / 8));
    hipStream_t st = (hipStream_t)stream;
    if (head_dim == 128)
        hipLaunchKernelGGL(prefill_kernel<128>, grid, dim3(prefill_threads<128>()), 0, st, a);
    else
        hipLaunchKernelGGL(prefill_kernel<64>, grid, dim3(prefill_threads<64>()), 0, st, a);
    if ((rc = check_launch("prefill")) != NYION_OK) return rc;
    // V enters the P.V product as binary16: values of magnitude >= 65520 are
    // reported through the status word (the chunk's V by the kernel's own
    // tail, with or without its f32 / binary16 pool write, or by the Q4
    // write's check; the history's here)
    if (n_hist > 0 &&
        (rc = v_range_check(v_hist, (long long)n_hist * n_kv_heads * head_dim, st)) != NYION_OK)
        return rc;
    if (!k_pool && !v_pool) return NYION_OK;  // the kernel checked the chunk's V itself
    if (!a.kv_write)  // 4-bit pools: their own quantising write (with the V range check)
        return kv_write_bf16_impl(k_pool, v_pool, block_table, block_tokens, num_blocks, n_kv_heads,
                                  head_dim, kv_dtype, start_pos, n, k, v, st);
    return NYION_OK;
}

extern "C" int nyion_prefill_attention_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                            int n, int n_heads, int n_kv_heads, int head_dim,
                                            int causal, float scale, float* out, void* k_pool,
                                            void* v_pool, const int32_t* block_table,
                                            int block_tokens, int num_blocks, int kv_dtype,
                                            int start_pos, nyion_stream_t stream) {
    return prefill_impl(q, k, v, nullptr, nullptr, 0, n, n_heads, n_kv_heads, head_dim, causal,
                        scale, out, k_pool, v_pool, block_table, block_tokens, num_blocks,
                        kv_dtype, start_pos, stream);
}

extern "C" int nyion_prefill_attention_bf16_ctx(const uint16_t* q, const uint16_t* k,
                                                const uint16_t* v, const uint16_t* k_hist,
                                                const uint16_t* v_hist, int n_hist, int n,
                                                int n_heads, int n_kv_heads, int head_dim,
                                                int causal, float scale, float* out, void* k_pool,
                                                void* v_pool, const int32_t* block_table,
                                                int block_tokens, int num_blocks, int kv_dtype,
                                                int start_pos, nyion_stream_t stream) {
    return prefill_impl(q, k, v, k_hist, v_hist, n_hist, n, n_heads, n_kv_heads, head_dim, causal,
                        scale, out, k_pool, v_pool, block_table, block_tokens, num_blocks,
                        kv_dtype, start_pos, stream);
}

