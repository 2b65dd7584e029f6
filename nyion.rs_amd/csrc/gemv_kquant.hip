// gemv_kquant.hip — k-quant weight GEMV (gfx950): Q4_K and Q6_K blocks, the
// projection step either side of decode attention.
//
// The reference computes out[r] = sum_j W[r][j] x[j] with W in GGUF k-quant
// blocks of 256 weights:
//  * Q4_K (swamp-kernels/src/fused_gemv_q4k.rs:59-99 dispatch, scalar
//    semantics 395-448): a 144-byte block of f16 d, f16 dmin, 12 bytes of
//    6-bit scales/mins (unpack 30-43) and 128 nibble bytes, where byte i of
//    qs pair p holds element 64p+i (low nibble, sub-block 2p) and element
//    64p+32+i (high nibble, sub-block 2p+1).  The weight is
//    (d*scale)*q - (dmin*min).
//  * Q6_K (swamp-kernels/src/fused_gemv_q6k.rs:22-43 dispatch, scalar
//    semantics 248-293): a 210-byte block of ql[128], qh[64], 16 int8 scales
//    and f16 d.  In half h, for l = 0..31, element 128h + l + 32k (k = 0..3)
//    is q = (low nibble of ql[64h + l] for k = 0, of ql[64h + 32 + l] for
//    k = 1, their high nibbles for k = 2, 3) | (bits 2k..2k+1 of
//    qh[32h + l]) << 4, with weight d * scale[8h + l/16 + 2k] * (q - 32).  d
//    goes through the reference's own f16 conversion (fused_gemv_q6k.rs:
//    11-20), which agrees with IEEE binary16 on normal values only.
//
// Decomposition.  Both formats split a block into eight lane chunks of 32
// weights that form two runs of 16 consecutive x values: Q4_K chunk q is the
// 16 nibble bytes 16q..16q+15 (runs at 64(q/2) + 16(q%2) and +32), Q6_K
// chunk q = 4h + j is ql bytes 16q..16q+15 (runs at 128h + 16j and +64, low
// and high nibbles).  A unit of R consecutive rows of one matrix belongs to
// P wavefronts of a workgroup (P = 1, 2, 4 or 8 by row length, so that up to
// 16384 columns every wavefront makes one pass); lane l of wavefront kp takes
// the chunks c = l + 64 (kp + P k) of every row.  The lane loads the 32 x
// values of its chunk position once and reuses them for its R rows, and
// folds the block formula as
//   s_lo*sum(q x) - m_lo*sum(x) + (same for the high run),
// (Q4_K: s = d*scale, m = dmin*min; Q6_K: s = d*scale, m = 32 s), so a
// weight costs one byte convert and one FMA.  Rows are reduced across the
// wavefront, then the P partials are added in a fixed order through LDS
// (deterministic: batched and multi-matrix calls equal the single call).
// Every byte of W is read once per call (HBM bound: 0.5625 B/weight for
// Q4_K, 0.8203 for Q6_K); x (at most 64 KiB) stays in the caches.
//
// Q6_K blocks are 210 bytes, so a block starts 2 bytes past a dword boundary
// in every other position: its fields are read as the dword-aligned words
// that contain them (never a byte outside those words) and realigned with
// v_alignbit.
//
// One launch serves up to four matrices of one format that share x (the
// executor's q/k/v and gate/up projections) and up to four inputs that share
// W (the batched GEMV of fused_gemv_q4k.rs:456-485; larger batches take
// several launches).
#include "common.hpp"

#include <algorithm>
#include <vector>

namespace nyion {

constexpr int kKqBlockElems = 256;
constexpr int kGemvMaxMats = 4;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
// four dwords at a dword-aligned address (Q6_K fields)
typedef uint32_t u32x4w __attribute__((ext_vector_type(4), aligned(4)));

struct GemvArgs {
    const uint8_t* w[kGemvMaxMats];  // [rows][nb * block bytes]
    float* out[kGemvMaxMats];        // [batch][out_stride], rows of matrix m
    int rows[kGemvMaxMats];
    int wave_start[kGemvMaxMats + 1];  // first unit (R rows) of each matrix
    int n_mats;
    const float* x;  // [batch][x_stride]
    long long x_stride;
    long long out_stride;
    int nb;  // blocks per row
};

// What one lane needs of one row for one chunk: the two scales and the two
// mins of its runs and the 32 quantised values as floats.
struct ChunkWeights {
    float s_lo, m_lo, s_hi, m_hi;
    float ql[16], qh[16];
};

// 16 packed bytes -> floats: the masked words go through an empty asm so that
// the compiler does not narrow the byte fields and each value is one
// v_cvt_f32_ubyte{0..3}
__device__ __forceinline__ void bytes_to_floats(const uint32_t (&lo)[4], const uint32_t (&hi)[4],
                                                float (&fl)[16], float (&fh)[16]) {
#pragma unroll
    for (int v = 0; v < 4; v++) {
        uint32_t l = lo[v], h = hi[v];
        asm volatile("" : "+v"(l), "+v"(h));
#pragma unroll
        for (int e = 0; e < 4; e++) {
            fl[4 * v + e] = (float)((l >> (8 * e)) & 0xffu);
            fh[4 * v + e] = (float)((h >> (8 * e)) & 0xffu);
        }
    }
}

// ---------------------------------------------------------------------------
// Q4_K
// ---------------------------------------------------------------------------

// Scale and min of sub-block j (0..7) from the 12 packed bytes in words
// s0 (bytes 0-3), s1 (4-7), s2 (8-11) (unpack_scales_q4k).
__device__ __forceinline__ void q4k_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int j,
                                              uint32_t& sc, uint32_t& mn) {
    if (j < 4) {
        sc = (s0 >> (8 * j)) & 63u;
        mn = (s1 >> (8 * j)) & 63u;
    } else {
        const int k = 8 * (j - 4);
        const uint32_t b8 = (s2 >> k) & 0xffu;
        sc = (b8 & 0xfu) | (((s0 >> k) >> 6 & 3u) << 4);
        mn = (b8 >> 4) | (((s1 >> k) >> 6 & 3u) << 4);
    }
}

struct Q4kFormat {
    static constexpr int kBlockBytes = 144;
    static constexpr int kRunGap = 32;  // x distance from the low run to the high run
    // one buffer copied forward per step: alternating the two takes more
    // registers and costs the four-row kernel a wavefront per SIMD
    // (8B-shaped gate/up 22.5 -> 25.5 us)
    static constexpr bool kAlternateBuffers = false;
    // four rows per unit: 155 registers, three wavefronts per SIMD (two rows
    // ran the 8B-shaped gate/up 22.8 -> 24.1 us)
    static constexpr int kMaxRows = 4;
    static constexpr const char* kName = "gemv q4k";
    // the block's 16-byte header and the chunk's 16 nibble bytes
    struct Raw {
        u32x4 hdr, qs;
    };
    __device__ static int x_offset(int q) { return 64 * (q >> 1) + 16 * (q & 1); }
    __device__ __forceinline__ static void load(const uint8_t* bp, int q, Raw& r) {
        // weights are read once per call: streaming loads
        r.hdr = __builtin_nontemporal_load((const u32x4*)bp);
        r.qs = __builtin_nontemporal_load((const u32x4*)(bp + 16 + 16 * q));
    }
    __device__ __forceinline__ static void unpack(const Raw& r, int q, ChunkWeights& cw) {
        const int pq = q >> 1;
        const float d = f16_bits_to_f32(r.hdr.x);
        const float dmin = f16_bits_to_f32(r.hdr.x >> 16);
        uint32_t sc_lo, mn_lo, sc_hi, mn_hi;
        q4k_scale_min(r.hdr.y, r.hdr.z, r.hdr.w, 2 * pq, sc_lo, mn_lo);
        q4k_scale_min(r.hdr.y, r.hdr.z, r.hdr.w, 2 * pq + 1, sc_hi, mn_hi);
        cw.s_lo = d * (float)sc_lo;
        cw.m_lo = dmin * (float)mn_lo;
        cw.s_hi = d * (float)sc_hi;
        cw.m_hi = dmin * (float)mn_hi;
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int v = 0; v < 4; v++) {
            lo[v] = r.qs[v] & 0x0f0f0f0fu;
            hi[v] = (r.qs[v] >> 4) & 0x0f0f0f0fu;
        }
        bytes_to_floats(lo, hi, cw.ql, cw.qh);
    }
};

// ---------------------------------------------------------------------------
// Q6_K
// ---------------------------------------------------------------------------

// The block scale as the reference converts it (fused_gemv_q6k.rs:11-20):
// IEEE binary16 for exponents 1..30; exponent 0 gives the bits
// sign | (1009 << 23 wrapped to 32 bits) | mant << 13 and exponent 31 the
// normal-formula value.
__device__ __forceinline__ float q6k_scale_to_f32(uint32_t v) {
    const uint32_t sign = (v >> 15 & 1u) << 31;
    const uint32_t e = (v >> 10) & 0x1fu;
    const uint32_t mant = (v & 0x3ffu) << 13;
    const uint32_t ebits = e == 0 ? (1009u << 23) : ((e + 112u) << 23);
    return __uint_as_float(sign | ebits | mant);
}

struct Q6kFormat {
    static constexpr int kBlockBytes = 210;
    static constexpr int kRunGap = 64;
    // the two buffers alternate by step parity, saving the copy of the raw
    // words between steps at the same occupancy (output projection 19.5 ->
    // 18.9 us)
    static constexpr bool kAlternateBuffers = true;
    // two rows per unit: four take 202 registers, two wavefronts per SIMD
    // (the 32000 x 2048 output projection 19.3 -> 18.1 us at two)
    static constexpr int kMaxRows = 2;
    static constexpr const char* kName = "gemv q6k";
    // dword-aligned words covering the chunk's 16 ql bytes and 16 qh bytes
    // (four plus one each), its two scales and the word holding d, and the
    // block's misalignment in bits (0 or 16)
    struct Raw {
        u32x4 ql, qh;
        uint32_t qlx, qhx, dw, shift;
        int sc_lo, sc_hi;
    };
    __device__ static int x_offset(int q) { return 128 * (q >> 2) + 16 * (q & 3); }
    __device__ __forceinline__ static void load(const uint8_t* bp, int q, Raw& r) {
        const int h = q >> 2, j = q & 3;
        const uint32_t mis = (uint32_t)(uintptr_t)bp & 3u;  // 0 or 2: blocks are 2-byte aligned
        const uint8_t* b4 = bp - mis;
        const int ql_off = 16 * q;                      // ql[64h + 16j]
        const int qh_off = 128 + 32 * h + 16 * (j & 1);  // qh[32h + 16(j%2)]
        const int sc_off = 192 + 8 * h + (j & 1) + 2 * (j >> 1);
        const int tail = 12 + 2 * (int)mis;  // the word holding the field's last byte
        // ordinary loads: seven loads touch each block, and with the streaming
        // hint a line could leave L2 before the last of them, which then
        // fetches it again from HBM (the 32000 x 2048 output projection took
        // 28 us streamed, 19 us cached)
        r.ql = *(const u32x4w*)(b4 + ql_off);
        r.qlx = *(const uint32_t*)(b4 + ql_off + tail);
        r.qh = *(const u32x4w*)(b4 + qh_off);
        r.qhx = *(const uint32_t*)(b4 + qh_off + tail);
        r.dw = *(const uint32_t*)(b4 + 208);
        r.sc_lo = *(const int8_t*)(bp + sc_off);
        r.sc_hi = *(const int8_t*)(bp + sc_off + 4);
        r.shift = 8u * mis;
    }
    __device__ __forceinline__ static void unpack(const Raw& r, int q, ChunkWeights& cw) {
        const uint32_t k2 = 2u * (uint32_t)((q & 3) >> 1);  // 2k of the low run (k = 0 or 1)
        const float d = q6k_scale_to_f32((r.dw >> r.shift) & 0xffffu);
        cw.s_lo = d * (float)r.sc_lo;
        cw.s_hi = d * (float)r.sc_hi;
        cw.m_lo = 32.f * cw.s_lo;
        cw.m_hi = 32.f * cw.s_hi;
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const uint32_t l = __builtin_amdgcn_alignbit(v < 3 ? r.ql[v + 1] : r.qlx, r.ql[v], r.shift);
            const uint32_t hb = __builtin_amdgcn_alignbit(v < 3 ? r.qh[v + 1] : r.qhx, r.qh[v], r.shift);
            // q = nibble | (2 high bits) << 4: bits 2k..2k+1 of qh for the low
            // run, 2k+4..2k+5 for the high run, moved to bits 4..5 of each byte
            lo[v] = (l & 0x0f0f0f0fu) | ((hb << (4u - k2)) & 0x30303030u);
            hi[v] = ((l >> 4) & 0x0f0f0f0fu) | ((hb >> k2) & 0x30303030u);
        }
        bytes_to_floats(lo, hi, cw.ql, cw.qh);
    }
};

// ---------------------------------------------------------------------------
// The persistent kernel, shared by both formats
// ---------------------------------------------------------------------------

template <class F, int R>
struct GemvStep {
    typename F::Raw raw[R];
};

template <class F, int R, int B, int P>
__global__ __launch_bounds__(64 * P) void gemv_kquant_kernel(GemvArgs a) {
    __shared__ float part[2][P][R * B];  // per-wavefront partial sums, by unit parity
    const int lane = threadIdx.x & 63;
    const int kp = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));  // share of the row
    const int q = lane & 7;  // chunk within its block (fixed per lane)
    const int xo = F::x_offset(q);  // first x of the low run within the block
    const int n_chunks = a.nb * 8;
    const int npass = (n_chunks + 64 * P - 1) / (64 * P);
    const int U = a.wave_start[a.n_mats];
    const int G = (int)gridDim.x;
    const long long row_bytes = (long long)a.nb * F::kBlockBytes;

    // x runs of every input for chunk c (16 low-run and 16 high-run values)
    // and their sums.  A chunk past the row reads block 0's (in bounds),
    // which its lane never uses: it skips the chunk's arithmetic.  Once per
    // call (one pass per row) the loads go out together; zeroing the values
    // of such a chunk would make each pair of loads wait for the one before.
    // Per pass (longer rows), the zeroing stays: without it the compiler
    // moves those loads ahead and holds up to 43 more registers, a wavefront
    // per SIMD in most instantiations.
    float xl[B][16], xh[B][16], sl[B], sh[B];
    auto load_x = [&](int c, bool zero_past) __attribute__((always_inline)) {
        const bool ok = c < n_chunks;
        const int blk = ok ? c >> 3 : 0;
#pragma unroll
        for (int b = 0; b < B; b++) {
            const float* xp = a.x + b * a.x_stride + blk * kKqBlockElems + xo;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                float4 lo = *(const float4*)(xp + 4 * v);
                float4 hi = *(const float4*)(xp + F::kRunGap + 4 * v);
                if (zero_past && !ok) lo = hi = float4{0.f, 0.f, 0.f, 0.f};
                xl[b][4 * v] = lo.x; xl[b][4 * v + 1] = lo.y; xl[b][4 * v + 2] = lo.z; xl[b][4 * v + 3] = lo.w;
                xh[b][4 * v] = hi.x; xh[b][4 * v + 1] = hi.y; xh[b][4 * v + 2] = hi.z; xh[b][4 * v + 3] = hi.w;
            }
            float s0 = 0.f, s1 = 0.f;
#pragma unroll
            for (int k = 0; k < 16; k++) {
                s0 += xl[b][k];
                s1 += xh[b][k];
            }
            sl[b] = s0;
            sh[b] = s1;
        }
    };
    // weights of step t = (unit blockIdx.x + (t / npass) G, pass t % npass);
    // rows past the matrix and chunks past the row read row r0 / block 0
    auto load_w = [&](int t, GemvStep<F, R>& st) __attribute__((always_inline)) {
        const int u = (int)blockIdx.x + (t / npass) * G;
        const int pass = t % npass;
        int m = 0;
#pragma unroll
        for (int i = 1; i < kGemvMaxMats; i++)
            if (i < a.n_mats && u >= a.wave_start[i]) m = i;
        const int r0 = (u - a.wave_start[m]) * R;
        const int nr = min(R, a.rows[m] - r0);
        const int c = lane + 64 * (kp + P * pass);
        const int blk = c < n_chunks ? c >> 3 : 0;
#pragma unroll
        for (int i = 0; i < R; i++) {
            const uint8_t* bp = a.w[m] + (long long)(r0 + (i < nr ? i : 0)) * row_bytes +
                                (long long)blk * F::kBlockBytes;
            F::load(bp, q, st.raw[i]);
        }
    };

    // steps of this workgroup: its units blockIdx.x, +G, ... times the passes
    const int units_here = (int)blockIdx.x < U ? (U - (int)blockIdx.x + G - 1) / G : 0;
    const int T = units_here * npass;
    // x before the first weights: a wavefront's loads complete in order, so
    // the x sums wait for x alone (the weights requested first made them wait
    // for those too: the TinyLlama step 485 -> 497 us)
    if (npass == 1) load_x(lane + 64 * kp, false);  // the same chunk positions for every row
    GemvStep<F, R> buf[2];  // current and next step's raw weights
    if (T > 0) load_w(0, buf[0]);
    float acc[R][B];
#pragma unroll
    for (int i = 0; i < R; i++)
#pragma unroll
        for (int b = 0; b < B; b++) acc[i][b] = 0.f;

    auto step = [&](int t, const GemvStep<F, R>& cur, GemvStep<F, R>& nxt) __attribute__((always_inline)) {
        if (t + 1 < T) load_w(t + 1, nxt);  // next step's weights in flight
        const int pass = t % npass;
        const int c = lane + 64 * (kp + P * pass);
        if (npass > 1) load_x(c, true);
        if (c < n_chunks) {
#pragma unroll
            for (int i = 0; i < R; i++) {
                ChunkWeights cw;
                F::unpack(cur.raw[i], q, cw);
#pragma unroll
                for (int b = 0; b < B; b++) {
                    float dl = 0.f, dh = 0.f;
#pragma unroll
                    for (int k = 0; k < 16; k++) {
                        dl = __builtin_fmaf(cw.ql[k], xl[b][k], dl);
                        dh = __builtin_fmaf(cw.qh[k], xh[b][k], dh);
                    }
                    acc[i][b] += cw.s_lo * dl - cw.m_lo * sl[b] + (cw.s_hi * dh - cw.m_hi * sh[b]);
                }
            }
        }
        if (pass == npass - 1) {
            // unit done: wavefront sums, then the P partials in order kp = 0..P-1
            const int u = (int)blockIdx.x + (t / npass) * G;
            int m = 0;
#pragma unroll
            for (int i = 1; i < kGemvMaxMats; i++)
                if (i < a.n_mats && u >= a.wave_start[i]) m = i;
            const int r0 = (u - a.wave_start[m]) * R;
            const int nr = min(R, a.rows[m] - r0);
#pragma unroll
            for (int i = 0; i < R; i++)
#pragma unroll
                for (int b = 0; b < B; b++) {
                    acc[i][b] = wave_reduce_dpp<false>(acc[i][b]);
                }
            if (P == 1) {
                if (lane == 0)
#pragma unroll
                    for (int i = 0; i < R; i++)
#pragma unroll
                        for (int b = 0; b < B; b++)
                            if (i < nr) a.out[m][b * a.out_stride + r0 + i] = acc[i][b];
            } else {
                // slots alternate by unit, so one barrier per unit suffices
                const int par = (t / npass) & 1;
                if (lane == 0)
#pragma unroll
                    for (int k = 0; k < R * B; k++) part[par][kp][k] = acc[k / B][k % B];
                __syncthreads();
                if (kp == 0 && lane == 0) {
#pragma unroll
                    for (int i = 0; i < R; i++)
#pragma unroll
                        for (int b = 0; b < B; b++) {
                            float v = part[par][0][i * B + b];
#pragma unroll
                            for (int k = 1; k < P; k++) v += part[par][k][i * B + b];
                            if (i < nr) a.out[m][b * a.out_stride + r0 + i] = v;
                        }
                }
            }
#pragma unroll
            for (int i = 0; i < R; i++)
#pragma unroll
                for (int b = 0; b < B; b++) acc[i][b] = 0.f;
        }
    };
    if constexpr (F::kAlternateBuffers) {
        for (int t = 0; t < T; t += 2) {
            step(t, buf[0], buf[1]);
            if (t + 1 < T) step(t + 1, buf[1], buf[0]);
        }
    } else {
        for (int t = 0; t < T; t++) {
            step(t, buf[0], buf[1]);
            buf[0] = buf[1];
        }
    }
}

// Resident workgroups of one instantiation on the current device (per
// device, computed on first use there).
template <class F, int R, int B, int P>
static int gemv_capacity() {
    static std::atomic<int> cache[kMaxDevices];
    return per_device_value(
        cache,
        [] {
            int per_cu = 0;
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, gemv_kquant_kernel<F, R, B, P>,
                                                             64 * P, 0) != hipSuccess) {
                (void)hipGetLastError();
                return 0;
            }
            return (per_cu > 0 ? per_cu : 1) * device_cu_count();
        },
        1024);
}

template <class F, int R, int B, int P>
static void launch_rbp(const GemvArgs& a, int units, hipStream_t st) {
    const int cap = gemv_capacity<F, R, B, P>();
    const int grid = units < cap ? units : cap;
    hipLaunchKernelGGL((gemv_kquant_kernel<F, R, B, P>), dim3(grid), dim3(64 * P), 0, st, a);
}

// Instantiations whose registers would spill: four rows of four inputs on
// eight wavefronts.
template <class F, int R, int B, int P>
constexpr bool gemv_fits() {
    return !(R == 4 && B == 4 && P == 8);
}

template <class F, int R, int B>
static void launch_p(const GemvArgs& a, int P, int units, hipStream_t st) {
    if (P == 1)
        launch_rbp<F, R, B, 1>(a, units, st);
    else if (P == 2)
        launch_rbp<F, R, B, 2>(a, units, st);
    else if (P == 4)
        launch_rbp<F, R, B, 4>(a, units, st);
    else if constexpr (gemv_fits<F, R, B, 8>())
        launch_rbp<F, R, B, 8>(a, units, st);
}

// Wavefronts per row: enough for one pass of 64 chunks each up to 16384
// columns (longer rows take several passes).  Rows per unit: R in {1, 2, 4}
// doubles while the launch keeps at least 4096 (unit, wavefront) pairs, up
// to the format's kMaxRows (two at four inputs and eight wavefronts per row,
// which would not fit four rows).
template <class F, int B>
static void launch_gemv(GemvArgs& a, int total_rows, hipStream_t st) {
    const int chunks = a.nb * 8;
    const int P = chunks <= 64 ? 1 : chunks <= 128 ? 2 : chunks <= 256 ? 4 : 8;
    const int r_max = std::min(F::kMaxRows, (B == 4 && P == 8) ? 2 : 4);
    int R = 1;
    while (R < r_max && (long long)(total_rows / (2 * R)) * P >= 4096) R *= 2;
    int units = 0;
    for (int m = 0; m < a.n_mats; m++) {
        a.wave_start[m] = units;
        units += (a.rows[m] + R - 1) / R;
    }
    for (int m = a.n_mats; m <= kGemvMaxMats; m++) a.wave_start[m] = units;
    if (R == 4)
        launch_p<F, 4, B>(a, P, units, st);
    else if (R == 2)
        launch_p<F, 2, B>(a, P, units, st);
    else
        launch_p<F, 1, B>(a, P, units, st);
}

// Weight pointers: 16-byte aligned for Q4_K (its blocks are 144 bytes, so
// every block is), 2-byte aligned for Q6_K (blocks hold f16 d).
template <class F>
static bool weights_aligned(const void* p) {
    return aligned(p, F::kBlockBytes % 16 == 0 ? 16 : 2);
}

template <class F>
static int gemv_impl(const uint8_t* const* ws, const float* x, long long x_stride, float* const* outs,
                     long long out_stride, const int32_t* row_counts, int n_mats, int n_cols, int batch,
                     hipStream_t st) {
    clear_error();
    int rc;
    if ((rc = require_device()) != NYION_OK) return rc;
    if (n_mats < 1 || n_mats > kGemvMaxMats)
        return set_error(NYION_ERR_INVALID, "%s: %d matrices (1..%d)", F::kName, n_mats, kGemvMaxMats);
    if (n_cols <= 0 || n_cols % kKqBlockElems)
        return set_error(NYION_ERR_INVALID, "%s: n_cols %d not a positive multiple of 256", F::kName, n_cols);
    if (!x || !aligned(x, 16) || batch < 1 || (batch > 1 && (x_stride < n_cols || x_stride % 4)))
        return set_error(NYION_ERR_INVALID, "%s: x must be 16-byte aligned, rows of >= n_cols "
                                            "floats with a stride that is a multiple of 4", F::kName);
    long long total_rows = 0;
    GemvArgs a{};
    for (int m = 0; m < n_mats; m++) {
        if (!ws[m] || !outs[m] || !weights_aligned<F>(ws[m]) || row_counts[m] <= 0)
            return set_error(NYION_ERR_INVALID, "%s: matrix %d: null/unaligned pointer or %d rows", F::kName,
                             m, row_counts[m]);
        if (batch > 1 && out_stride < row_counts[m])
            return set_error(NYION_ERR_INVALID, "%s: out_stride %lld < rows %d", F::kName, out_stride,
                             row_counts[m]);
        a.w[m] = ws[m];
        a.out[m] = outs[m];
        a.rows[m] = row_counts[m];
        total_rows += row_counts[m];
    }
    if (total_rows > (1LL << 30)) return set_error(NYION_ERR_UNSUPPORTED, "%s: %lld rows", F::kName, total_rows);
    a.n_mats = n_mats;
    a.nb = n_cols / kKqBlockElems;
    a.x_stride = x_stride;
    a.out_stride = out_stride;
    // inputs in launches of 4, 2 and 1 (each launch reads W once)
    for (int b0 = 0; b0 < batch;) {
        const int width = batch - b0 >= 4 ? 4 : (batch - b0 >= 2 ? 2 : 1);
        a.x = x + b0 * x_stride;
        for (int m = 0; m < n_mats; m++) a.out[m] = outs[m] + b0 * out_stride;
        if (width == 4)
            launch_gemv<F, 4>(a, (int)total_rows, st);
        else if (width == 2)
            launch_gemv<F, 2>(a, (int)total_rows, st);
        else
            launch_gemv<F, 1>(a, (int)total_rows, st);
        if ((rc = check_launch(F::kName)) != NYION_OK) return rc;
        b0 += width;
    }
    return NYION_OK;
}

}  // namespace nyion

using namespace nyion;

extern "C" {

int nyion_gemv_q4k(const uint8_t* d_w, const float* d_x, float* d_out, int n_rows, int n_cols,
                   nyion_stream_t stream) {
    const int32_t rows = n_rows;
    return gemv_impl<Q4kFormat>(&d_w, d_x, n_cols, &d_out, n_rows, &rows, 1, n_cols, 1,
                                (hipStream_t)stream);
}

int nyion_gemv_q4k_multi(const uint8_t* const* d_ws, const float* d_x, float* const* d_outs,
                         const int32_t* row_counts, int n_mats, int n_cols, nyion_stream_t stream) {
    if (!d_ws || !d_outs || !row_counts) {
        clear_error();
        return set_error(NYION_ERR_INVALID, "gemv q4k multi: null matrix arrays");
    }
    return gemv_impl<Q4kFormat>(d_ws, d_x, n_cols, d_outs, 0, row_counts, n_mats, n_cols, 1,
                                (hipStream_t)stream);
}

int nyion_gemv_q4k_batched(const uint8_t* d_w, const float* d_x, int64_t x_stride, float* d_out,
                           int64_t out_stride, int n_rows, int n_cols, int batch,
                           nyion_stream_t stream) {
    const int32_t rows = n_rows;
    return gemv_impl<Q4kFormat>(&d_w, d_x, x_stride, &d_out, out_stride, &rows, 1, n_cols, batch,
                                (hipStream_t)stream);
}

int nyion_gemv_q6k(const uint8_t* d_w, const float* d_x, float* d_out, int n_rows, int n_cols,
                   nyion_stream_t stream) {
    const int32_t rows = n_rows;
    return gemv_impl<Q6kFormat>(&d_w, d_x, n_cols, &d_out, n_rows, &rows, 1, n_cols, 1,
                                (hipStream_t)stream);
}

int nyion_gemv_q6k_batched(const uint8_t* d_w, const float* d_x, int64_t x_stride, float* d_out,
                           int64_t out_stride, int n_rows, int n_cols, int batch,
                           nyion_stream_t stream) {
    const int32_t rows = n_rows;
    return gemv_impl<Q6kFormat>(&d_w, d_x, x_stride, &d_out, out_stride, &rows, 1, n_cols, batch,
                                (hipStream_t)stream);
}

int nyion_gemv_specs(const nyion_gemv_spec* specs, int n_specs, nyion_stream_t stream) {
    clear_error();
    if (n_specs < 0 || (n_specs > 0 && !specs))
        return set_error(NYION_ERR_INVALID, "gemv specs: %d specs at %p", n_specs, (const void*)specs);
    for (int i = 0; i < n_specs; i++) {
        const nyion_gemv_spec& g = specs[i];
        if (g.block_bytes != Q4kFormat::kBlockBytes && g.block_bytes != Q6kFormat::kBlockBytes)
            return set_error(NYION_ERR_INVALID, "gemv specs: spec %d: block_bytes %d (144 Q4_K or 210 Q6_K)",
                             i, g.block_bytes);
        if (g.n_rows < 0 || g.n_cols <= 0 || g.n_cols % kKqBlockElems)
            return set_error(NYION_ERR_INVALID, "gemv specs: spec %d: %d x %d", i, g.n_rows, g.n_cols);
        if (g.n_rows > 0 && (!g.w || !g.x || !g.out))
            return set_error(NYION_ERR_INVALID, "gemv specs: spec %d: null pointer", i);
        const bool w_ok = g.block_bytes == Q4kFormat::kBlockBytes ? weights_aligned<Q4kFormat>(g.w)
                                                                 : weights_aligned<Q6kFormat>(g.w);
        if (g.n_rows > 0 && (!w_ok || !aligned(g.x, 16)))
            return set_error(NYION_ERR_INVALID, "gemv specs: spec %d: W or x not aligned (x 16 bytes, "
                                                "Q4_K W 16 bytes, Q6_K W 2 bytes)", i);
    }
    // specs of one format, width and input share a launch (up to four each)
    std::vector<char> done(n_specs, 0);
    for (int i = 0; i < n_specs; i++) {
        if (done[i] || specs[i].n_rows == 0) continue;
        const nyion_gemv_spec& g = specs[i];
        const uint8_t* ws[kGemvMaxMats];
        float* outs[kGemvMaxMats];
        int32_t rows[kGemvMaxMats];
        int n = 0;
        for (int j = i; j < n_specs && n < kGemvMaxMats; j++) {
            const nyion_gemv_spec& h = specs[j];
            if (done[j] || h.n_rows == 0 || h.block_bytes != g.block_bytes || h.n_cols != g.n_cols || h.x != g.x)
                continue;
            ws[n] = h.w;
            outs[n] = h.out;
            rows[n] = h.n_rows;
            n++;
            done[j] = 1;
        }
        const int rc = g.block_bytes == Q4kFormat::kBlockBytes
                           ? gemv_impl<Q4kFormat>(ws, g.x, g.n_cols, outs, 0, rows, n, g.n_cols, 1,
                                                  (hipStream_t)stream)
                           : gemv_impl<Q6kFormat>(ws, g.x, g.n_cols, outs, 0, rows, n, g.n_cols, 1,
                                                  (hipStream_t)stream);
        if (rc != NYION_OK) return rc;
    }
    return NYION_OK;
}

}  // extern "C"
