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
// bound on the list).  Three launches, no cross-workgroup waits:
//   1. scores: one thread per position decodes its K row, scores every q
//      head of the group, stores the scores and the piece's per-head
//      (max, sum of exp) partials;
//   2. weights and V: every piece combines its segment's partials into the
//      head's max and 1/sum (pieces in order), turns its scores into
//      weights (dropping those below 1e-8), decodes its V rows into LDS in
//      16 KiB batches and accumulates sum(w * v) in position order;
//   3. merge: the output is the sum of the pieces' partial outputs in piece
//      order (skipped when one piece covers every sequence).
// Bytes per attended (token, kv head): K and V rows, 2 * 20 * head_dim / 32.
#include <math.h>

#include "common.hpp"

namespace nyion {

constexpr int kSq4Threads = 256;    // positions per piece
// V rows decoded into LDS per batch: 16 KiB of f32, one 16-element unit per thread
template <int D> constexpr int sq4_vrows() { return 4096 / D; }
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

template <int D>
__global__ __launch_bounds__(kSq4Threads) void sq4_scores_kernel(Sq4Args a) {
    constexpr int G = D / 32;           // groups per row
    constexpr int W = G * 5;            // 4-byte words per row
    extern __shared__ float sm[];
    float* q_s = sm;                     // [group][D]
    float* sc_s = sm + a.group * D;      // [group][256]
    const int seg = blockIdx.y, piece = blockIdx.x;
    const int b = seg / a.n_kv_heads, h = seg % a.n_kv_heads;
    const int tid = threadIdx.x;
    const Sq4List l = sq4_list(a, b);
    const float* qb = a.q + ((long long)b * a.n_heads + (long long)h * a.group) * D;
    for (int i = tid; i < a.group * D; i += kSq4Threads) q_s[i] = qb[i];
    const int i = piece * kSq4Threads + tid;
    long long off = -1;
    if (i < l.n) off = sq4_row(a, b, sq4_pos(a, l, i), h, W * 4);
    float kf[D];
    if (off >= 0) {
        const uint32_t* rw = (const uint32_t*)(a.k + off);
        uint32_t w[W];
#pragma unroll
        for (int x = 0; x < W; x++) w[x] = __builtin_nontemporal_load(rw + x);
#pragma unroll
        for (int g = 0; g < G; g++) {
            sq4_half(w + 5 * g, 0, kf + 32 * g);
            sq4_half(w + 5 * g, 1, kf + 32 * g + 16);
        }
    }
    __syncthreads();
    for (int r = 0; r < a.group; r++) {
        float s = -INFINITY;
        if (off >= 0) {
            const float* qr = q_s + r * D;
            float acc[16];
#pragma unroll
            for (int x = 0; x < 16; x++) acc[x] = 0.0f;
#pragma unroll
            for (int c = 0; c < D; c += 16)
#pragma unroll
                for (int x = 0; x < 16; x++) acc[x] = __builtin_fmaf(kf[c + x], qr[c + x], acc[x]);
            float dot = 0.0f;
#pragma unroll
            for (int x = 0; x < 16; x++) dot = dot + acc[x];
            s = dot * a.scale;
        }
        sc_s[r * kSq4Threads + tid] = s;
        if (i < l.n)
            a.scores[((long long)seg * a.group + r) * ((long long)a.pieces * kSq4Threads) + i] = s;
    }
    __syncthreads();
    // per head: the piece's max and sum of exp(s - max), one wavefront per head
    const int wave = tid >> 6, lane = tid & 63;
    for (int r = wave; r < a.group; r += kSq4Threads / 64) {
        float v[4];
#pragma unroll
        for (int x = 0; x < 4; x++) v[x] = sc_s[r * kSq4Threads + lane + 64 * x];
        float m = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
        float e = 0.0f;
        if (m != -INFINITY) {
#pragma unroll
            for (int x = 0; x < 4; x++) e += v[x] == -INFINITY ? 0.0f : expf(v[x] - m);
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) e += __shfl_xor(e, o);
        if (lane == 0) a.ml[((long long)seg * a.pieces + piece) * a.group + r] = float2{m, e};
    }
}

template <int D>
__global__ __launch_bounds__(kSq4Threads) void sq4_values_kernel(Sq4Args a) {
    constexpr int G = D / 32;
    constexpr int W = G * 5;
    constexpr int kMaxOut = kSq4MaxGroup * D / kSq4Threads;
    extern __shared__ float sm[];
    float* w_s = sm;                             // [group][256] weights (0: skipped)
    constexpr int VR = sq4_vrows<D>();
    float* v_s = sm + a.group * kSq4Threads;     // [VR][D] decoded V rows
    float* mi_s = v_s + VR * D;                  // [group][2] (max, 1/sum)
    const int seg = blockIdx.y, piece = blockIdx.x;
    const int b = seg / a.n_kv_heads, h = seg % a.n_kv_heads;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const Sq4List l = sq4_list(a, b);
    const int first = piece * kSq4Threads;
    const int n_here = l.n - first < kSq4Threads ? l.n - first : kSq4Threads;
    // pieces holding positions (a context past max_ctx is cut at the grid)
    const int used = min((l.n + kSq4Threads - 1) / kSq4Threads, a.pieces);
    // the head's max and 1/sum over the pieces, in piece order
    for (int r = wave; r < a.group; r += kSq4Threads / 64) {
        const float2* mlr = a.ml + (long long)seg * a.pieces * a.group + r;
        float m = -INFINITY;
        for (int p = lane; p < used; p += 64) m = fmaxf(m, mlr[(long long)p * a.group].x);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
        float sum = 0.0f;
        if (m != -INFINITY) {
            for (int p0 = 0; p0 < used; p0 += 64) {
                float e = 0.0f;
                if (p0 + lane < used) {
                    const float2 x = mlr[(long long)(p0 + lane) * a.group];
                    e = x.x == -INFINITY ? 0.0f : x.y * expf(x.x - m);
                }
#pragma unroll
                for (int o = 32; o > 0; o >>= 1) e += __shfl_xor(e, o);
                sum += e;
            }
        }
        if (lane == 0) {
            mi_s[2 * r] = m;
            mi_s[2 * r + 1] = 1.0f / sum;
        }
    }
    __syncthreads();
    for (int r = 0; r < a.group; r++) {
        float w = 0.0f;
        if (tid < n_here) {
            const float s = a.scores[((long long)seg * a.group + r) * ((long long)a.pieces * kSq4Threads) +
                                     first + tid];
            if (s != -INFINITY) {
                w = expf(s - mi_s[2 * r]) * mi_s[2 * r + 1];
                if (w < 1e-8f) w = 0.0f;  // ops.rs:692
            }
        }
        w_s[r * kSq4Threads + tid] = w;
    }
    const int n_out = a.group * D;
    float acc[kMaxOut];
#pragma unroll
    for (int x = 0; x < kMaxOut; x++) acc[x] = 0.0f;
    for (int r0 = 0; r0 < n_here; r0 += VR) {
        __syncthreads();  // weights written / the previous batch consumed
        // decode rows r0 .. r0 + VR - 1 of the piece: 16-element units, D/16 per row
        for (int u = tid; u < VR * (D / 16); u += kSq4Threads) {
            const int p = u / (D / 16), gu = u % (D / 16);
            float vals[16];
            long long off = -1;
            if (r0 + p < n_here) off = sq4_row(a, b, sq4_pos(a, l, first + r0 + p), h, W * 4);
            if (off >= 0) {
                const uint32_t* gw = (const uint32_t*)(a.v + off) + 5 * (gu >> 1);
                uint32_t w5[5];
#pragma unroll
                for (int x = 0; x < 5; x++) w5[x] = __builtin_nontemporal_load(gw + x);
                sq4_half(w5, gu & 1, vals);
            } else {
#pragma unroll
                for (int x = 0; x < 16; x++) vals[x] = 0.0f;
            }
            float4* dst = (float4*)(v_s + p * D + 16 * gu);
#pragma unroll
            for (int x = 0; x < 4; x++)
                dst[x] = float4{vals[4 * x], vals[4 * x + 1], vals[4 * x + 2], vals[4 * x + 3]};
        }
        __syncthreads();
        const int rows = n_here - r0 < VR ? n_here - r0 : VR;
#pragma unroll
        for (int x = 0; x < kMaxOut; x++) {
            const int o = tid + kSq4Threads * x;
            if (o < n_out) {
                const int r = o / D, d = o % D;
                const float* wr = w_s + r * kSq4Threads + r0;
                for (int p = 0; p < rows; p++) {
                    const float w = wr[p];
                    if (w != 0.0f) acc[x] = __builtin_fmaf(v_s[p * D + d], w, acc[x]);
                }
            }
        }
    }
    // pieces past the list write zeros, so the merge reads defined values
    const bool direct = a.pieces == 1;
#pragma unroll
    for (int x = 0; x < kMaxOut; x++) {
        const int o = tid + kSq4Threads * x;
        if (o < n_out) {
            const int r = o / D, d = o % D;
            if (direct)
                a.out[((long long)b * a.n_heads + (long long)h * a.group + r) * D + d] = acc[x];
            else
                a.part[(((long long)seg * a.pieces + piece) * a.group + r) * D + d] = acc[x];
        }
    }
}

template <int D>
__global__ __launch_bounds__(kSq4Threads) void sq4_merge_kernel(Sq4Args a) {
    const int seg = blockIdx.y;
    const int b = seg / a.n_kv_heads, h = seg % a.n_kv_heads;
    const int o = blockIdx.x * kSq4Threads + threadIdx.x;
    if (o >= a.group * D) return;
    const Sq4List l = sq4_list(a, b);
    const int used = min((l.n + kSq4Threads - 1) / kSq4Threads, a.pieces);
    float s = 0.0f;
    for (int p = 0; p < used; p++) s += a.part[((long long)seg * a.pieces + p) * a.group * D + o];
    a.out[((long long)b * a.n_heads + (long long)h * a.group) * D + o] = s;
}

static long long sq4_bound(int window, int max_ctx) {
    const long long w = (long long)(window > 0 ? window : 0) + kSq4MaxGlobals;
    return max_ctx < w ? max_ctx : w;
}

struct Sq4Sizes {
    int pieces;
    size_t scores, ml, part;
};

static Sq4Sizes sq4_sizes(int batch, int n_heads, int head_dim, int window, int max_ctx) {
    Sq4Sizes z;
    z.pieces = (int)((sq4_bound(window, max_ctx) + kSq4Threads - 1) / kSq4Threads);
    const size_t rows = (size_t)batch * n_heads;  // (sequence, q head)
    z.scores = rows * z.pieces * kSq4Threads * sizeof(float);
    z.ml = rows * z.pieces * sizeof(float2);
    z.part = z.pieces > 1 ? rows * z.pieces * head_dim * sizeof(float) : 0;
    auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
    z.scores = up(z.scores);
    z.ml = up(z.ml);
    z.part = up(z.part);
    return z;
}

template <int D>
static int sq4_launch(Sq4Args& a, int batch, hipStream_t st) {
    const dim3 grid(a.pieces, batch * a.n_kv_heads);
    const size_t lds1 = (size_t)a.group * (D + kSq4Threads) * sizeof(float);
    const size_t lds2 = ((size_t)a.group * (kSq4Threads + 2) + sq4_vrows<D>() * D) * sizeof(float);
    hipLaunchKernelGGL(sq4_scores_kernel<D>, grid, dim3(kSq4Threads), lds1, st, a);
    int rc = check_launch("attention_sparse_q4 scores");
    if (rc != NYION_OK) return rc;
    hipLaunchKernelGGL(sq4_values_kernel<D>, grid, dim3(kSq4Threads), lds2, st, a);
    if ((rc = check_launch("attention_sparse_q4 values")) != NYION_OK) return rc;
    if (a.pieces > 1) {
        const dim3 g3((a.group * D + kSq4Threads - 1) / kSq4Threads, batch * a.n_kv_heads);
        hipLaunchKernelGGL(sq4_merge_kernel<D>, g3, dim3(kSq4Threads), 0, st, a);
        rc = check_launch("attention_sparse_q4 merge");
    }
    return rc;
}

}  // namespace nyion

using namespace nyion;

extern "C" {

size_t nyion_attention_sparse_q4_workspace_size(int batch, int n_heads, int head_dim, int window,
                                                int max_ctx) {
    if (batch <= 0 || n_heads <= 0 || head_dim <= 0 || max_ctx <= 0) return 0;
    const Sq4Sizes z = sq4_sizes(batch, n_heads, head_dim, window, max_ctx);
    return z.scores + z.ml + z.part;
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
    const Sq4Sizes z = sq4_sizes(batch, n_heads, head_dim, window, max_ctx);
    if (!d_workspace || workspace_bytes < z.scores + z.ml + z.part)
        return set_error(NYION_ERR_WORKSPACE,
                         "attention_sparse_q4: workspace of %zu bytes, %zu needed", workspace_bytes,
                         z.scores + z.ml + z.part);
    if (!aligned(d_workspace, 256) || !aligned(d_q, 4) || !aligned(d_out, 4))
        return set_error(NYION_ERR_INVALID, "attention_sparse_q4: workspace must be 256-byte aligned");
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
