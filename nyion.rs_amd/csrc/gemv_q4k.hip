// gemv_q4k.hip — Q4_K weight GEMV (gfx950), the projection step either side
// of decode attention.
//
// The reference computes out[r] = sum_j W[r][j] x[j] with W in GGUF Q4_K
// blocks (swamp-kernels/src/fused_gemv_q4k.rs:59-99 dispatch, scalar
// semantics 395-448): per 256 weights a 144-byte block of f16 d, f16 dmin,
// 12 bytes of 6-bit scales/mins (unpack 30-43) and 128 nibble bytes, where
// byte i of qs pair p holds element 64p+i (low nibble, sub-block 2p) and
// element 64p+32+i (high nibble, sub-block 2p+1).  The weight is
// (d*scale)*q - (dmin*min).
//
// Decomposition.  A unit of R consecutive rows of one matrix belongs to P
// wavefronts of a workgroup (P = 1, 2 or 4 by row length, so that up to
// 8192 columns every wavefront makes one pass); lane l of wavefront kp takes
// the 16-byte nibble chunks c = l + 64 (kp + P k) of every row: chunk c is
// block c/8, chunk c%8 of its 128 nibble bytes, i.e. 16 weights of sub-block
// 2p and the 16 at the same offsets in sub-block 2p+1 (p = (c%8)/2).  The
// lane loads the 32 matching x values once per chunk position and reuses
// them for its R rows, and folds the block formula as
//   (d*sc_lo)*sum(q x) - (dmin*m_lo)*sum(x) + (same for the high nibbles),
// so a weight costs one byte convert and one FMA.  Rows are reduced across
// the wavefront, then the P partials are added in a fixed order through LDS
// (deterministic: batched and multi-matrix calls equal the single call).  Every byte of W is read once per call (HBM
// bound: 0.5625 B/weight); x (at most 64 KiB) stays in the caches.
//
// One launch serves up to four matrices that share x (the executor's
// q/k/v and gate/up projections) and up to four inputs that share W (the
// batched GEMV of fused_gemv_q4k.rs:456-485; larger batches take several
// launches).
#include "common.hpp"

namespace nyion {

constexpr int kQ4kBlockElems = 256;
constexpr int kQ4kBlockBytes = 144;
constexpr int kGemvMaxMats = 4;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct GemvQ4kArgs {
    const uint8_t* w[kGemvMaxMats];  // [rows][nb * 144]
    float* out[kGemvMaxMats];        // [batch][out_stride], rows of matrix m
    int rows[kGemvMaxMats];
    int wave_start[kGemvMaxMats + 1];  // first unit (R rows) of each matrix
    int n_mats;
    const float* x;  // [batch][x_stride]
    long long x_stride;
    long long out_stride;
    int nb;  // blocks per row
};

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

// Per-lane work of one (unit, pass) step: the R rows' 16-byte header and
// nibble chunk.
template <int R>
struct GemvStep {
    u32x4 hdr[R];
    u32x4 qs[R];
};

template <int R, int B, int P>
__global__ __launch_bounds__(64 * P) void gemv_q4k_kernel(GemvQ4kArgs a) {
    __shared__ float part[2][P][R * B];  // per-wavefront partial sums, by unit parity
    const int lane = threadIdx.x & 63;
    const int kp = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));  // share of the row
    const int q = lane & 7;  // nibble chunk within its block (fixed per lane)
    const int pq = q >> 1;
    const int xo = 64 * pq + 16 * (q & 1);  // first x of the low run within the block
    const int n_chunks = a.nb * 8;
    const int npass = (n_chunks + 64 * P - 1) / (64 * P);
    const int U = a.wave_start[a.n_mats];
    const int G = (int)gridDim.x;
    const long long row_bytes = (long long)a.nb * kQ4kBlockBytes;

    // x runs of every input for chunk c (16 low-run and 16 high-run values)
    // and their sums; zero for a chunk past the row
    float xl[B][16], xh[B][16], sl[B], sh[B];
    auto load_x = [&](int c) __attribute__((always_inline)) {
        const bool ok = c < n_chunks;
        const int blk = ok ? c >> 3 : 0;
#pragma unroll
        for (int b = 0; b < B; b++) {
            const float* xp = a.x + b * a.x_stride + blk * kQ4kBlockElems + xo;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                float4 lo = *(const float4*)(xp + 4 * v);
                float4 hi = *(const float4*)(xp + 32 + 4 * v);
                if (!ok) lo = hi = float4{0.f, 0.f, 0.f, 0.f};
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
    auto load_w = [&](int t, GemvStep<R>& st) __attribute__((always_inline)) {
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
                                (long long)blk * kQ4kBlockBytes;
            // weights are read once per call: streaming loads
            st.hdr[i] = __builtin_nontemporal_load((const u32x4*)bp);
            st.qs[i] = __builtin_nontemporal_load((const u32x4*)(bp + 16 + 16 * q));
        }
    };

    // steps of this workgroup: its units blockIdx.x, +G, ... times the passes
    const int units_here = (int)blockIdx.x < U ? (U - (int)blockIdx.x + G - 1) / G : 0;
    const int T = units_here * npass;
    if (npass == 1) load_x(lane + 64 * kp);  // the same chunk positions for every row
    GemvStep<R> cur, nxt;
    if (T > 0) load_w(0, cur);
    float acc[R][B];
#pragma unroll
    for (int i = 0; i < R; i++)
#pragma unroll
        for (int b = 0; b < B; b++) acc[i][b] = 0.f;

    for (int t = 0; t < T; t++) {
        if (t + 1 < T) load_w(t + 1, nxt);  // next step's weights in flight
        const int pass = t % npass;
        const int c = lane + 64 * (kp + P * pass);
        if (npass > 1) load_x(c);
        if (c < n_chunks) {
#pragma unroll
            for (int i = 0; i < R; i++) {
                const float d = f16_bits_to_f32(cur.hdr[i].x);
                const float dmin = f16_bits_to_f32(cur.hdr[i].x >> 16);
                uint32_t sc_lo, mn_lo, sc_hi, mn_hi;
                q4k_scale_min(cur.hdr[i].y, cur.hdr[i].z, cur.hdr[i].w, 2 * pq, sc_lo, mn_lo);
                q4k_scale_min(cur.hdr[i].y, cur.hdr[i].z, cur.hdr[i].w, 2 * pq + 1, sc_hi, mn_hi);
                const float sv_lo = d * (float)sc_lo, mv_lo = dmin * (float)mn_lo;
                const float sv_hi = d * (float)sc_hi, mv_hi = dmin * (float)mn_hi;
                // nibbles -> floats once per row: the masked words go through an
                // empty asm so that the compiler does not narrow the byte
                // fields and each value is one v_cvt_f32_ubyte{0..3}
                float ql[16], qh[16];
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    uint32_t lo = cur.qs[i][v] & 0x0f0f0f0fu;
                    uint32_t hi = (cur.qs[i][v] >> 4) & 0x0f0f0f0fu;
                    asm volatile("" : "+v"(lo), "+v"(hi));
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        ql[4 * v + e] = (float)((lo >> (8 * e)) & 0xffu);
                        qh[4 * v + e] = (float)((hi >> (8 * e)) & 0xffu);
                    }
                }
#pragma unroll
                for (int b = 0; b < B; b++) {
                    float dl = 0.f, dh = 0.f;
#pragma unroll
                    for (int k = 0; k < 16; k++) {
                        dl = __builtin_fmaf(ql[k], xl[b][k], dl);
                        dh = __builtin_fmaf(qh[k], xh[b][k], dh);
                    }
                    acc[i][b] += sv_lo * dl - mv_lo * sl[b] + (sv_hi * dh - mv_hi * sh[b]);
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
                    float v = acc[i][b];
#pragma unroll
                    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
                    acc[i][b] = v;
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
        cur = nxt;
    }
}

// Resident workgroups of one instantiation on this device.
template <int R, int B, int P>
static int gemv_capacity() {
    static int cap = 0;
    if (cap == 0) {
        int per_cu = 0, cus = 0, dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, gemv_q4k_kernel<R, B, P>, 64 * P, 0) !=
                hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
            (void)hipGetLastError();
            return 1024;
        }
        cap = (per_cu > 0 ? per_cu : 1) * (cus > 0 ? cus : 1);
    }
    return cap;
}

template <int R, int B, int P>
static void launch_rbp(const GemvQ4kArgs& a, int units, hipStream_t st) {
    const int cap = gemv_capacity<R, B, P>();
    const int grid = units < cap ? units : cap;
    hipLaunchKernelGGL((gemv_q4k_kernel<R, B, P>), dim3(grid), dim3(64 * P), 0, st, a);
}

template <int R, int B>
static void launch_p(const GemvQ4kArgs& a, int P, int units, hipStream_t st) {
    if (P == 1)
        launch_rbp<R, B, 1>(a, units, st);
    else if (P == 2)
        launch_rbp<R, B, 2>(a, units, st);
    else if (P == 4)
        launch_rbp<R, B, 4>(a, units, st);
    else if constexpr (!(R == 4 && B == 4))  // four rows of four inputs do not fit eight wavefronts
        launch_rbp<R, B, 8>(a, units, st);
}

// Wavefronts per row: enough for one pass of 64 chunks each up to 16384
// columns (longer rows take several passes).  Rows per unit: the largest R
// in {1, 2, 4} that still gives every SIMD four wavefronts (two at four
// inputs and eight wavefronts per row, which would not fit four rows).
template <int B>
static void launch_gemv(GemvQ4kArgs& a, int total_rows, hipStream_t st) {
    const int chunks = a.nb * 8;
    const int P = chunks <= 64 ? 1 : chunks <= 128 ? 2 : chunks <= 256 ? 4 : 8;
    const int r_max = (B == 4 && P == 8) ? 2 : 4;
    int R = 1;
    while (R < r_max && (long long)(total_rows / (2 * R)) * P >= 4096) R *= 2;
    int units = 0;
    for (int m = 0; m < a.n_mats; m++) {
        a.wave_start[m] = units;
        units += (a.rows[m] + R - 1) / R;
    }
    for (int m = a.n_mats; m <= kGemvMaxMats; m++) a.wave_start[m] = units;
    if (R == 4)
        launch_p<4, B>(a, P, units, st);
    else if (R == 2)
        launch_p<2, B>(a, P, units, st);
    else
        launch_p<1, B>(a, P, units, st);
}

static int gemv_q4k_impl(const uint8_t* const* ws, const float* x, long long x_stride,
                         float* const* outs, long long out_stride, const int32_t* row_counts,
                         int n_mats, int n_cols, int batch, hipStream_t st) {
    clear_error();
    int rc;
    if ((rc = require_device()) != NYION_OK) return rc;
    if (n_mats < 1 || n_mats > kGemvMaxMats)
        return set_error(NYION_ERR_INVALID, "gemv q4k: %d matrices (1..%d)", n_mats, kGemvMaxMats);
    if (n_cols <= 0 || n_cols % kQ4kBlockElems)
        return set_error(NYION_ERR_INVALID, "gemv q4k: n_cols %d not a positive multiple of 256", n_cols);
    if (!x || !aligned(x, 16) || batch < 1 || (batch > 1 && (x_stride < n_cols || x_stride % 4)))
        return set_error(NYION_ERR_INVALID, "gemv q4k: x must be 16-byte aligned, rows of >= n_cols "
                                            "floats with a stride that is a multiple of 4");
    long long total_rows = 0;
    GemvQ4kArgs a{};
    for (int m = 0; m < n_mats; m++) {
        if (!ws[m] || !outs[m] || !aligned(ws[m], 16) || row_counts[m] <= 0)
            return set_error(NYION_ERR_INVALID, "gemv q4k: matrix %d: null/unaligned pointer or %d rows",
                             m, row_counts[m]);
        if (batch > 1 && out_stride < row_counts[m])
            return set_error(NYION_ERR_INVALID, "gemv q4k: out_stride %lld < rows %d", out_stride,
                             row_counts[m]);
        a.w[m] = ws[m];
        a.out[m] = outs[m];
        a.rows[m] = row_counts[m];
        total_rows += row_counts[m];
    }
    if (total_rows > (1LL << 30)) return set_error(NYION_ERR_UNSUPPORTED, "gemv q4k: %lld rows", total_rows);
    a.n_mats = n_mats;
    a.nb = n_cols / kQ4kBlockElems;
    a.x_stride = x_stride;
    a.out_stride = out_stride;
    // inputs in launches of 4, 2 and 1 (each launch reads W once)
    for (int b0 = 0; b0 < batch;) {
        const int width = batch - b0 >= 4 ? 4 : (batch - b0 >= 2 ? 2 : 1);
        a.x = x + b0 * x_stride;
        for (int m = 0; m < n_mats; m++) a.out[m] = outs[m] + b0 * out_stride;
        if (width == 4)
            launch_gemv<4>(a, (int)total_rows, st);
        else if (width == 2)
            launch_gemv<2>(a, (int)total_rows, st);
        else
            launch_gemv<1>(a, (int)total_rows, st);
        if ((rc = check_launch("gemv q4k")) != NYION_OK) return rc;
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
    return gemv_q4k_impl(&d_w, d_x, n_cols, &d_out, n_rows, &rows, 1, n_cols, 1,
                         (hipStream_t)stream);
}

int nyion_gemv_q4k_multi(const uint8_t* const* d_ws, const float* d_x, float* const* d_outs,
                         const int32_t* row_counts, int n_mats, int n_cols, nyion_stream_t stream) {
    if (!d_ws || !d_outs || !row_counts) {
        clear_error();
        return set_error(NYION_ERR_INVALID, "gemv q4k multi: null matrix arrays");
    }
    return gemv_q4k_impl(d_ws, d_x, n_cols, d_outs, 0, row_counts, n_mats, n_cols, 1,
                         (hipStream_t)stream);
}

int nyion_gemv_q4k_batched(const uint8_t* d_w, const float* d_x, int64_t x_stride, float* d_out,
                           int64_t out_stride, int n_rows, int n_cols, int batch,
                           nyion_stream_t stream) {
    const int32_t rows = n_rows;
    return gemv_q4k_impl(&d_w, d_x, x_stride, &d_out, out_stride, &rows, 1, n_cols, batch,
                         (hipStream_t)stream);
}

}  // extern "C"
