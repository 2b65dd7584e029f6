// sparse_q4.hip — ops::attention_sparse_q4 (swamp-engine/src/ops.rs:597-723)
// over one layer of zone pools of Q4-20B rows.
//
// The function attends attention_sparse's position set (the last `window`
// positions up to valid_end and every global_stride-th earlier one, at most
// 128; ops.rs:612-623) and reads the rows with its own rules, which differ
// from the cache writer's (cache.rs:655-663):
//   * group g of row (t, kv head) is the 20 bytes at (slot * groups + g) * 20
//     of the (layer, kv head) block of t's zone page (ops.rs:639-644);
//   * its 16 nibble bytes give elements 0..15 from their low nibbles and
//     16..31 from their high nibbles (ops.rs:653-656);
//   * element = fma(d, nibble, dmin) (ops.rs:661-662);
//   * q.k is accumulated in 16 FMA lanes over 16-element chunks and the lanes
//     are added in order (ops.rs:664-674), then times 1/sqrt(head_dim);
//   * weights are exp(s - max) times 1/sum, and positions whose weight is
//     below 1e-8 add nothing to the output (ops.rs:678-692).
// Each score is computed in exactly that order, so the scores equal the
// reference's bit for bit; the exponentials and the sums are the device's.
//
// Work: a segment is (sequence, kv head); its position list is cut into
// pieces of 256 positions, one workgroup each (the grid covers the host's
// bound on the list).  Two launches, no cross-workgroup waits:
//   1. scores: one thread per position decodes its K row, scores every q
//      head of the group, stores the scores and the piece's per-head
//      (max, sum of exp) partials;
//   2. weights and V: every piece combines its segment's partials into the
//      head's max and 1/sum (pieces in order), turns its scores into
//      weights (dropping those below 1e-8), decodes its V rows into LDS in
//      16 KiB batches and accumulates sum(w * v) in position order;
//      the segment's last piece to finish (an arrival counter) adds the
//      pieces' partial outputs in piece order (one piece: written directly).
// Bytes per attended (token, kv head): K and V rows, 2 * 20 * head_dim / 32.
#include <math.h>

#include "common.hpp"

namespace nyion {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kSq4Threads = 256;    // positions per piece
constexpr int kSq4MaxGroup = 32;    // q heads per kv head
constexpr int kSq4MaxGlobals = 128;  // ops.rs:615

struct Sq4Args {
    const float* q;            // [B][Hq][D]
    const uint8_t* k;          // zone pools (bytes)
    const uint8_t* v;
    const int64_t* page_bases;  // [B][n_pages]
    const int32_t* ctx_lens;    // [B]
    const int32_t* q_pos;       // [B] or nullptr (ctx - 1)
    float* out;                 // [B][Hq][D]
    float* scores;              // [seg][group][pieces * 256]
    float2* ml;                 // [seg][pieces][group] (max, sum of exp)
    float* part;                // [seg][pieces][group][D]
    int* counters;              // [seg] arrivals, zero between calls
    ZoneMap zone;
    int n_heads, n_kv_heads, group, pieces, window, global_stride;
    float scale;
};

// The position list of sequence b: count, start of the window part, count of
// globals.
struct Sq4List {
    int n, ws, n_glob;
};

__device__ __forceinline__ Sq4List sq4_list(const Sq4Args& a, int b) {
    Sq4List l{0, 0, 0};
    const int len = a.ctx_lens[b];
    if (len <= 0) return l;
    const int qp = a.q_pos ? a.q_pos[b] : len - 1;
    const int ve = qp < len - 1 ? qp : len - 1;
    if (ve < 0) return l;
    l.ws = ve > a.window ? ve - a.window + 1 : 0;
    if (a.global_stride > 0) {
        const int gc = l.ws / a.global_stride;
        l.n_glob = gc < kSq4MaxGlobals ? gc : kSq4MaxGlobals;
    }
    l.n = l.n_glob + (ve - l.ws + 1);
    return l;
}

__device__ __forceinline__ int sq4_pos(const Sq4Args& a, const Sq4List& l, int i) {
    return i < l.n_glob ? a.global_stride * i : l.ws + (i - l.n_glob);
}

// Byte offset of row (t, kv head h) of sequence b, or -1 when its page is
// absent or outside the pool.
__device__ __forceinline__ long long sq4_row(const Sq4Args& a, int b, int t, int h, int row_bytes) {
    ZoneMap z = a.zone;
    z.page_base = a.page_bases + (long long)b * a.zone.n_pages;
    return zone_row_offset(z, t, h, row_bytes);
}

// Elements 16*half .. 16*half + 15 of one group in the A5 order: the low
// (half 0) or high (half 1) nibbles of its 16 bytes, fma(d, nibble, dmin).
__device__ __forceinline__ void sq4_half(const uint32_t* w5, int half, float* out) {
    const float d = f16_bits_to_f32(w5[0]);
    const float dmin = f16_bits_to_f32(w5[0] >> 16);
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const uint32_t byte = (w5[1 + j / 4] >> (8 * (j % 4))) & 0xffu;
        const uint32_t nib = half ? byte >> 4 : byte & 0xfu;
        out[j] = __builtin_fmaf(d, (float)nib, dmin);
    }
}

typedef const __attribute__((address_space(4))) float* sq4_cfloat_ptr;

template <int D>
__global__ __launch_bounds__(kSq4Threads) void sq4_scores_kernel(Sq4Args a) {
    constexpr int G = D / 32;           // groups per row
    constexpr int W = G * 5;            // 4-byte words per row
    extern __shared__ float4 sm4[];  // 16-byte aligned: float4 accesses
    float* sm = (float*)sm4;
    float* sc_s = sm;                   // [group][256]
    const int seg = blockIdx.y, piece = blockIdx.x;
    const int b = seg / a.n_kv_heads, h = seg % a.n_kv_heads;
    const int tid = threadIdx.x;
    const Sq4List l = sq4_list(a, b);
    const int i = piece * kSq4Threads + tid;
    long long off = -1;
    if (i < l.n) off = sq4_row(a, b, sq4_pos(a, l, i), h, W * 4);
    // q of the group is the same for every lane: it is read through the
    // constant address space into scalar registers, each FMA taking its q
    // operand from there.  Its 64-byte lines are requested together here
    // (32 at a time), so the per-head loads below hit the scalar cache.
    const sq4_cfloat_ptr qb =
        (sq4_cfloat_ptr)(a.q + ((long long)b * a.n_heads + (long long)h * a.group) * D);
    for (int x0 = 0; x0 < a.group * D; x0 += 32 * 16) {
        float t = 0.0f;
#pragma unroll
        for (int x = 0; x < 32; x++) t += x0 + 16 * x < a.group * D ? qb[x0 + 16 * x] : 0.0f;
        asm volatile("" ::"s"(t));
    }
    // the row's words (plain loads: the lanes' 40- or 80-byte rows share cache
    // lines, which the later words of the row hit in L1)
    uint32_t w[W];
#pragma unroll
    for (int x = 0; x < W; x++) w[x] = 0;
    if (off >= 0) {
        const uint32_t* rw = (const uint32_t*)(a.k + off);
#pragma unroll
        for (int x = 0; x < W; x++) w[x] = rw[x];
    }
    float kf[D];
#pragma unroll
    for (int g = 0; g < G; g++) {
        sq4_half(w + 5 * g, 0, kf + 32 * g);
        sq4_half(w + 5 * g, 1, kf + 32 * g + 16);
    }
    float* srow = a.scores + (long long)seg * a.group * ((long long)a.pieces * kSq4Threads) + i;
    for (int r = 0; r < a.group; r++) {
        float acc[16];
#pragma unroll
        for (int x = 0; x < 16; x++) acc[x] = 0.0f;
#pragma unroll
        for (int c = 0; c < D; c += 16)
#pragma unroll
            for (int x = 0; x < 16; x++) acc[x] = __builtin_fmaf(kf[c + x], qb[r * D + c + x], acc[x]);
        float dot = 0.0f;
#pragma unroll
        for (int x = 0; x < 16; x++) dot = dot + acc[x];
        const float s = off >= 0 ? dot * a.scale : -INFINITY;
        sc_s[r * kSq4Threads + tid] = s;
        if (i < l.n) srow[(long long)r * a.pieces * kSq4Threads] = s;
    }
    __syncthreads();
    // per head: the piece's max and sum of exp(s - max), one wavefront per head
    const int wave = tid >> 6, lane = tid & 63;
    for (int r = wave; r < a.group; r += kSq4Threads / 64) {
        float v[4];
#pragma unroll
        for (int x = 0; x < 4; x++) v[x] = sc_s[r * kSq4Threads + lane + 64 * x];
        const float m = wave_reduce_dpp<true>(fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])));
        float e = 0.0f;
        if (m != -INFINITY) {
#pragma unroll
            for (int x = 0; x < 4; x++) e += v[x] == -INFINITY ? 0.0f : expf(v[x] - m);
        }
        e = wave_reduce_dpp<false>(e);
        if (lane == 0) a.ml[((long long)seg * a.pieces + piece) * a.group + r] = float2{m, e};
    }
}

// LDS rows of decoded V per batch: 32 KiB of f32 (two batches of 128 rows at
// head_dim 64, four of 64 at head_dim 128), rows padded by 4 floats, so that
// three workgroups fit a CU's LDS.
template <int D> constexpr int sq4_vrows() { return 8192 / D; }
template <int D> constexpr int sq4_vstride() { return D + 4; }
constexpr int kSq4Hb = 8;  // heads per thread in the weighted sum

template <int D>
__global__ __launch_bounds__(kSq4Threads) void sq4_values_kernel(Sq4Args a) {
    constexpr int G = D / 32;
    constexpr int W = G * 5;
    constexpr int VR = sq4_vrows<D>(), VS = sq4_vstride<D>();
    constexpr int Q = D / 4;  // 4-dim quads per row
    const int WP = (a.group + kSq4Hb - 1) / kSq4Hb * kSq4Hb;  // weights per row, padded
    extern __shared__ float4 sm4[];  // 16-byte aligned: float4 accesses
    float* sm = (float*)sm4;
    float* w_s = sm;                    // [256][WP] weights (0: skipped or padding)
    float* v_s = w_s + kSq4Threads * WP;  // [VR][VS] decoded V rows; then split sums
    float* mi_s = v_s + VR * VS;        // [group][2] (max, 1/sum)
    const int seg = blockIdx.y, piece = blockIdx.x;
    const int b = seg / a.n_kv_heads, h = seg % a.n_kv_heads;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const Sq4List l = sq4_list(a, b);
    const int first = piece * kSq4Threads;
    const int n_here = l.n - first < kSq4Threads ? l.n - first : kSq4Threads;
    // pieces holding positions (a context past max_ctx is cut at the grid)
    const int used = min((l.n + kSq4Threads - 1) / kSq4Threads, a.pieces);
    // this thread's V row (position first + tid), in flight during the merge
    long long off = -1;
    if (tid < n_here) off = sq4_row(a, b, sq4_pos(a, l, first + tid), h, W * 4);
    uint32_t vw[W];
#pragma unroll
    for (int x = 0; x < W; x++) vw[x] = 0;
    if (off >= 0) {
        const uint32_t* rw = (const uint32_t*)(a.v + off);
#pragma unroll
        for (int x = 0; x < W; x++) vw[x] = rw[x];
    }
    // every head's score of this position, requested with the V row and
    // ahead of the pieces' (max, sum) below, none of which it depends on
    float sv[kSq4MaxGroup];
    {
        const float* src = a.scores + (long long)seg * a.group * ((long long)a.pieces * kSq4Threads) +
                           first + tid;
#pragma unroll
        for (int r = 0; r < kSq4MaxGroup; r++)
            sv[r] = r < a.group && tid < n_here ? src[(long long)r * a.pieces * kSq4Threads] : -INFINITY;
    }
    // the head's max and 1/sum over the pieces, in piece order
    for (int r = wave; r < a.group; r += kSq4Threads / 64) {
        const float2* mlr = a.ml + (long long)seg * a.pieces * a.group + r;
        const float2 mine = lane < used ? mlr[(long long)lane * a.group] : float2{-INFINITY, 0.0f};
        float m = mine.x;
        for (int p = lane + 64; p < used; p += 64) m = fmaxf(m, mlr[(long long)p * a.group].x);
        m = wave_reduce_dpp<true>(m);
        float sum = 0.0f;
        if (m != -INFINITY) {
            float e = mine.x == -INFINITY ? 0.0f : mine.y * expf(mine.x - m);
            sum = wave_reduce_dpp<false>(e);
            for (int p0 = 64; p0 < used; p0 += 64) {  // more than 64 pieces
                e = 0.0f;
                if (p0 + lane < used) {
                    const float2 x = mlr[(long long)(p0 + lane) * a.group];
                    e = x.x == -INFINITY ? 0.0f : x.y * expf(x.x - m);
                }
                sum += wave_reduce_dpp<false>(e);
            }
        }
        if (lane == 0) {
            mi_s[2 * r] = m;
            mi_s[2 * r + 1] = 1.0f / sum;
        }
    }
    __syncthreads();
    {
        // every head's weight of this position
#pragma unroll
        for (int r = 0; r < kSq4MaxGroup; r++) {
            if (r < WP) {
                float w = 0.0f;
                if (r < a.group && sv[r] != -INFINITY) {
                    w = expf(sv[r] - mi_s[2 * r]) * mi_s[2 * r + 1];
                    if (w < 1e-8f) w = 0.0f;  // ops.rs:692
                }
                w_s[tid * WP + r] = w;
            }
        }
    }
    // weighted sum: a thread owns one 4-dim quad of kSq4Hb heads (block hb)
    // over one of `splits` consecutive ranges of each batch's rows
    const int nhb = WP / kSq4Hb;
    const int quad = tid % Q, rest = tid / Q;
    const int hb = rest % nhb, split = rest / nhb;
    const int splits = (kSq4Threads / Q) / nhb;
    const bool active = split < splits;
    float acc[kSq4Hb][4];
#pragma unroll
    for (int k = 0; k < kSq4Hb; k++)
#pragma unroll
        for (int x = 0; x < 4; x++) acc[k][x] = 0.0f;
    for (int b0 = 0; b0 < n_here; b0 += VR) {
        __syncthreads();  // weights written / the previous batch consumed
        if (tid >= b0 && tid < b0 + VR) {
            float* dst = v_s + (tid - b0) * VS;
#pragma unroll
            for (int g = 0; g < G; g++) {
                float vals[16];
                sq4_half(vw + 5 * g, 0, vals);
#pragma unroll
                for (int x = 0; x < 4; x++)
                    *(float4*)(dst + 32 * g + 4 * x) =
                        float4{vals[4 * x], vals[4 * x + 1], vals[4 * x + 2], vals[4 * x + 3]};
                sq4_half(vw + 5 * g, 1, vals);
#pragma unroll
                for (int x = 0; x < 4; x++)
                    *(float4*)(dst + 32 * g + 16 + 4 * x) =
                        float4{vals[4 * x], vals[4 * x + 1], vals[4 * x + 2], vals[4 * x + 3]};
            }
        }
        __syncthreads();
        const int rows = n_here - b0 < VR ? n_here - b0 : VR;
        const int chunk = (rows + splits - 1) / splits;
        const int p_lo = split * chunk, p_hi = min(rows, p_lo + chunk);
        if (active) {
            const float* vq = v_s + 4 * quad;
            const float* wq = w_s + (b0 * WP) + kSq4Hb * hb;
            for (int p = p_lo; p < p_hi; p++) {
                const float4 v = *(const float4*)(vq + p * VS);
                const float4 w0 = *(const float4*)(wq + p * WP);
                const float4 w1 = *(const float4*)(wq + p * WP + 4);
                const float w[kSq4Hb] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
                for (int k = 0; k < kSq4Hb; k++) {
                    // a skipped weight leaves the sum as it is (no 0 * v)
                    const bool on = w[k] != 0.0f;
                    acc[k][0] = on ? __builtin_fmaf(v.x, w[k], acc[k][0]) : acc[k][0];
                    acc[k][1] = on ? __builtin_fmaf(v.y, w[k], acc[k][1]) : acc[k][1];
                    acc[k][2] = on ? __builtin_fmaf(v.z, w[k], acc[k][2]) : acc[k][2];
                    acc[k][3] = on ? __builtin_fmaf(v.w, w[k], acc[k][3]) : acc[k][3];
                }
            }
        }
    }
    // the splits' sums, added in split order
    __syncthreads();  // v_s is free
    float* red = v_s;  // [splits][WP][D]
    if (active) {
#pragma unroll
        for (int k = 0; k < kSq4Hb; k++)
            *(float4*)(red + ((long long)split * WP + kSq4Hb * hb + k) * D + 4 * quad) =
                float4{acc[k][0], acc[k][1], acc[k][2], acc[k][3]};
    }
    __syncthreads();
    const bool direct = a.pieces == 1;
    float* out_b = a.out + ((long long)b * a.n_heads + (long long)h * a.group) * D;
    float* part_s = a.part + (long long)seg * a.pieces * a.group * D;
    const __amdgpu_buffer_rsrc_t rpart =
        partial_rsrc(part_s, direct ? 0u : (uint32_t)(a.pieces * a.group * D * 4));
    for (int o4 = tid; o4 < a.group * Q; o4 += kSq4Threads) {
        const int r = o4 / Q, qd = o4 % Q;
        float4 t = float4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 4
        for (int sp = 0; sp < splits; sp++) {
            const float4 x = *(const float4*)(red + ((long long)sp * WP + r) * D + 4 * qd);
            t.x += x.x;
            t.y += x.y;
            t.z += x.z;
            t.w += x.w;
        }
        if (direct) {
            *(float4*)(out_b + r * D + 4 * qd) = t;
        } else if (piece < used) {  // pieces past the list hold nothing to add
            const u32x4_t d = {__float_as_uint(t.x), __float_as_uint(t.y), __float_as_uint(t.z),
                               __float_as_uint(t.w)};
            __builtin_amdgcn_raw_buffer_store_b128(d, rpart, ((piece * a.group + r) * D + 4 * qd) * 4, 0,
                                                   kSc1);
        }
    }
    if (direct) return;
    // publish: every wavefront's write-through stores complete, then the
    // piece's arrival is counted; the segment's last piece to arrive adds
    // the pieces' partial outputs in piece order and resets the counter
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    __shared__ int last;
    if (tid == 0)
        last = __hip_atomic_fetch_add(a.counters + seg, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               a.pieces - 1;
    __syncthreads();
    if (!last) return;
    for (int o4 = tid; o4 < a.group * Q; o4 += kSq4Threads) {
        const int r = o4 / Q, qd = o4 % Q;
        const uint32_t off0 = (r * D + 4 * qd) * 4, step = a.group * D * 4;
        float4 t = float4{0.0f, 0.0f, 0.0f, 0.0f};
        int p = 0;
        for (; p + 8 <= used; p += 8) {  // eight loads in flight, added in piece order
            u32x4_t x[8];
#pragma unroll
            for (int k = 0; k < 8; k++)
                x[k] = __builtin_amdgcn_raw_buffer_load_b128(rpart, off0 + (p + k) * step, 0, kSc1);
#pragma unroll
            for (int k = 0; k < 8; k++) {
                t.x += __uint_as_float(x[k][0]);
                t.y += __uint_as_float(x[k][1]);
                t.z += __uint_as_float(x[k][2]);
                t.w += __uint_as_float(x[k][3]);
            }
        }
        for (; p < used; p++) {
            const u32x4_t x = __builtin_amdgcn_raw_buffer_load_b128(rpart, off0 + p * step, 0, kSc1);
            t.x += __uint_as_float(x[0]);
            t.y += __uint_as_float(x[1]);
            t.z += __uint_as_float(x[2]);
            t.w += __uint_as_float(x[3]);
        }
        *(float4*)(out_b + r * D + 4 * qd) = t;
    }
    if (tid == 0) __hip_atomic_store(a.counters + seg, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

static long long sq4_bound(int window, int max_ctx) {
    const long long w = (long long)(window > 0 ? window : 0) + kSq4MaxGlobals;
    return max_ctx < w ? max_ctx : w;
}

struct Sq4Sizes {
    int pieces;
    size_t scores, ml, part, counters;
    size_t total() const { return scores + ml + part + counters; }
};

static Sq4Sizes sq4_sizes(int batch, int n_heads, int n_kv_heads, int head_dim, int window,
                          int max_ctx) {
    Sq4Sizes z;
    z.pieces = (int)((sq4_bound(window, max_ctx) + kSq4Threads - 1) / kSq4Threads);
    const size_t rows = (size_t)batch * n_heads;  // (sequence, q head)
    z.scores = rows * z.pieces * kSq4Threads * sizeof(float);
    z.ml = rows * z.pieces * sizeof(float2);
    z.part = z.pieces > 1 ? rows * z.pieces * head_dim * sizeof(float) : 0;
    z.counters = z.pieces > 1 ? (size_t)batch * n_kv_heads * sizeof(int) : 0;
    auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
    z.scores = up(z.scores);
    z.ml = up(z.ml);
    z.part = up(z.part);
    z.counters = up(z.counters);
    return z;
}

template <int D>
static int sq4_launch(Sq4Args& a, int batch, hipStream_t st) {
    const dim3 grid(a.pieces, batch * a.n_kv_heads);
    const int wp = (a.group + kSq4Hb - 1) / kSq4Hb * kSq4Hb;
    const size_t lds1 = (size_t)a.group * kSq4Threads * sizeof(float);
    const size_t lds2 = ((size_t)kSq4Threads * wp + sq4_vrows<D>() * sq4_vstride<D>() + 2 * a.group) *
                        sizeof(float);
    hipLaunchKernelGGL(sq4_scores_kernel<D>, grid, dim3(kSq4Threads), lds1, st, a);
    int rc = check_launch("attention_sparse_q4 scores");
    if (rc != NYION_OK) return rc;
    hipLaunchKernelGGL(sq4_values_kernel<D>, grid, dim3(kSq4Threads), lds2, st, a);
    return check_launch("attention_sparse_q4 values");
}

}  // namespace nyion

using namespace nyion;

extern "C" {

size_t nyion_attention_sparse_q4_workspace_size(int batch, int n_heads, int n_kv_heads, int head_dim,
                                                int window, int max_ctx) {
    if (batch <= 0 || n_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0 || max_ctx <= 0) return 0;
    return sq4_sizes(batch, n_heads, n_kv_heads, head_dim, window, max_ctx).total();
}

int nyion_attention_sparse_q4(const float* d_q, const void* k_pool, const void* v_pool,
                              int64_t pool_bytes, const int64_t* page_bases, int max_pages_per_seq,
                              int n_layers, int layer, const int32_t* ctx_lens, const int32_t* q_pos,
                              int batch, int n_heads, int n_kv_heads, int head_dim, int window,
                              int global_stride, int max_ctx, float* d_out, void* d_workspace,
                              size_t workspace_bytes, nyion_stream_t stream) {
    clear_error();
    int rc;
    if ((rc = require_device()) != NYION_OK) return rc;
    if (!d_q || !d_out || !k_pool || !v_pool || !page_bases || !ctx_lens)
        return set_error(NYION_ERR_INVALID, "attention_sparse_q4: null argument");
    if (!aligned(k_pool, 4) || !aligned(v_pool, 4))
        return set_error(NYION_ERR_INVALID, "attention_sparse_q4: pools must be 4-byte aligned");
    if (batch <= 0 || n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads)
        return set_error(NYION_ERR_INVALID, "attention_sparse_q4: batch %d, heads %d/%d", batch,
                         n_heads, n_kv_heads);
    if (head_dim != 64 && head_dim != 128)
        return set_error(NYION_ERR_UNSUPPORTED, "attention_sparse_q4: head_dim %d (64 or 128)",
                         head_dim);
    const int group = n_heads / n_kv_heads;
    if (group > kSq4MaxGroup)
        return set_error(NYION_ERR_UNSUPPORTED, "attention_sparse_q4: %d q heads per kv head (max %d)",
                         group, kSq4MaxGroup);
    if (window < 0) return set_error(NYION_ERR_INVALID, "attention_sparse_q4: window %d", window);
    if ((long long)batch * n_kv_heads > 65535)
        return set_error(NYION_ERR_UNSUPPORTED, "attention_sparse_q4: batch * n_kv_heads %lld",
                         (long long)batch * n_kv_heads);
    ZoneMap zone;
    if ((rc = make_zone_map(zone, pool_bytes, max_pages_per_seq, n_layers, layer, n_kv_heads,
                            NYION_KV_Q4_20B, "attention_sparse_q4")) != NYION_OK)
        return rc;
    if (max_ctx <= 0 || zone_pos(max_ctx - 1).page >= max_pages_per_seq)
        return set_error(NYION_ERR_INVALID,
                         "attention_sparse_q4: max_ctx %d needs %d pages per sequence, the table has %d",
                         max_ctx, max_ctx > 0 ? zone_pos(max_ctx - 1).page + 1 : 0, max_pages_per_seq);
    const Sq4Sizes z = sq4_sizes(batch, n_heads, n_kv_heads, head_dim, window, max_ctx);
    if ((long long)z.pieces * group * head_dim * 4 >= (1LL << 31))
        return set_error(NYION_ERR_UNSUPPORTED, "attention_sparse_q4: window %d too long", window);
    if (!d_workspace || workspace_bytes < z.total())
        return set_error(NYION_ERR_WORKSPACE,
                         "attention_sparse_q4: workspace of %zu bytes, %zu needed", workspace_bytes,
                         z.total());
    if (!aligned(d_workspace, 256) || !aligned(d_q, 16) || !aligned(d_out, 16))
        return set_error(NYION_ERR_INVALID,
                         "attention_sparse_q4: q/out must be 16-byte and the workspace 256-byte aligned");
    Sq4Args a{};
    a.q = d_q;
    a.k = (const uint8_t*)k_pool;
    a.v = (const uint8_t*)v_pool;
    a.page_bases = page_bases;
    a.ctx_lens = ctx_lens;
    a.q_pos = q_pos;
    a.out = d_out;
    a.scores = (float*)d_workspace;
    a.ml = (float2*)((char*)d_workspace + z.scores);
    a.part = z.part ? (float*)((char*)d_workspace + z.scores + z.ml) : nullptr;
    a.counters = z.counters ? (int*)((char*)d_workspace + z.scores + z.ml + z.part) : nullptr;
    a.zone = zone;
    a.n_heads = n_heads;
    a.n_kv_heads = n_kv_heads;
    a.group = group;
    a.pieces = z.pieces;
    a.window = window;
    a.global_stride = global_stride;
    a.scale = 1.0f / sqrtf((float)head_dim);  // ops.rs:610
    hipStream_t st = (hipStream_t)stream;
    return head_dim == 64 ? sq4_launch<64>(a, batch, st) : sq4_launch<128>(a, batch, st);
}

}  // extern "C"
