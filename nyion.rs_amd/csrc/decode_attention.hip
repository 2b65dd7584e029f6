// decode_attention.hip — batched paged GQA decode attention for gfx950.
//
// One query token per sequence (the executor's decode step,
// swamp-engine/src/executor.rs:739-763).  Semantics follow ops::attention
// (swamp-engine/src/ops.rs:170-278) and ops::attention_sparse (ops.rs:85-168);
// see the header for the position sets.
//
// Work decomposition.  A wavefront owns one (sequence, kv head, group of up
// to 16 q heads, split-K partition).  Four independent wavefronts share a
// 256-thread workgroup; they never synchronise and use no LDS.  The 8 q heads
// of a GQA group are processed together so each K/V byte is read from HBM
// exactly once.
//
// Per 16-token tile the wavefront issues two MFMA chains on
// v_mfma_f32_16x16x4_f32 (fp32 in, fp32 accumulate):
//   S[16 tok][16 heads] = K_tile[16][D] . Q^T[D][16]       (D/4 MFMAs)
//   O[16 heads][D]     += P[16 heads][16 tok] . V_tile      (D/4 MFMAs)
// The MFMA output layout of S (lane = head + 16*token_quad, reg = token in
// quad) is exactly the A-operand layout P needs for the second product, so
// probabilities never leave registers.  K and V rows are streamed with
// 128-bit loads straight from the paged pool: for K, lanes (token i, quad k)
// read 64 contiguous bytes per instruction of each row; for V, 16 lanes read
// one whole row per instruction.  Q4-20B rows are dequantised in registers.
//
// Online softmax runs in the log2 domain on the S registers: tile max over
// the 4 registers and the 4 token quads (lane xor 16, 32), rescale, exp2.
// Partitions that do not cover the whole sequence write (m, l, acc) partials
// to the workspace; decode_merge_kernel combines them (log-sum-exp).
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
    const int32_t* tables;  // [B][table_stride] or nullptr (contiguous)
    const int32_t* ctx_lens;   // [B] or nullptr (uniform_len)
    const int32_t* q_pos;      // [B] or nullptr (len - 1)
    const int32_t* positions;  // MODE_LIST: [B][pos_stride]
    const int32_t* n_pos;      // MODE_LIST: [B]
    float* out;                // [B][Hq][D]
    float* ws_acc;             // [(b*Hq + head)*max_parts + p][D]
    float2* ws_ml;             // [(b*Hq + head)*max_parts + p] = (m log2, l)
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
    int part_tokens;  // multiple of 16
    int max_parts;
    int max_len;       // host bound on attended positions per sequence
    float scale_log2;  // scale * log2(e)
};

struct SeqExtent {
    int L;       // number of attended positions
    int ws;      // window start (MODE_WINDOW)
    int n_glob;  // strided globals before the window (MODE_WINDOW)
};

// Attended position set of sequence b (ops.rs:97-113 for the window form,
// ops.rs:183 for valid_end).
// L is clamped to the host bound the grid and workspace were sized for.
__device__ __forceinline__ SeqExtent seq_extent(const DecodeArgs& a, int b) {
    SeqExtent e{0, 0, 0};
    if (a.mode == MODE_LIST) {
        e.L = min(max(a.n_pos[b], 0), a.max_len);
        return e;
    }
    const int len = a.ctx_lens ? a.ctx_lens[b] : a.uniform_len;
    if (len <= 0) return e;
    const int qp = a.q_pos ? a.q_pos[b] : len - 1;
    if (qp < 0) return e;
    const int ve = min(qp, len - 1);
    if (a.mode == MODE_FULL) {
        e.L = min(ve + 1, a.max_len);
        return e;
    }
    const int ws = ve > a.window ? ve - a.window + 1 : 0;
    const int ng = a.global_stride > 0 ? min(ws / a.global_stride, 128) : 0;
    e.ws = ws;
    e.n_glob = ng;
    e.L = min(ng + (ve - ws + 1), a.max_len);
    return e;
}

__device__ __forceinline__ int virt_to_pos(const DecodeArgs& a, const SeqExtent& e, int b, int v) {
    if (a.mode == MODE_FULL) return v;
    if (a.mode == MODE_WINDOW) return v < e.n_glob ? v * a.global_stride : e.ws + (v - e.n_glob);
    return a.positions[(long long)b * a.pos_stride + v];
}

// ---------------------------------------------------------------- loaders
// K operand of lane (row i, quad kq): NC = D/4 values, one per QK MFMA.
//   f32: call c = 4x+y holds dim 16x + 4kq + y  (per x, the 4 quads of a row
//        read 64 contiguous bytes)
//   Q4 : call c holds dim kq*D/4 + c            (contiguous nibbles)
// The Q operand uses the same map (qk_dim).
template <int D, int KVT>
__device__ __forceinline__ int qk_dim(int c, int kq) {
    if constexpr (KVT == NYION_KV_F32)
        return 16 * (c >> 2) + 4 * kq + (c & 3);
    else
        return kq * (D / 4) + c;
}

template <int D, int KVT>
__device__ __forceinline__ void load_k(const void* base, long long off, int kq, float* kv) {
    constexpr int NC = D / 4;
    if (off < 0) {
#pragma unroll
        for (int c = 0; c < NC; c++) kv[c] = 0.f;
        return;
    }
    if constexpr (KVT == NYION_KV_F32) {
        const float* row = (const float*)base + off;
#pragma unroll
        for (int x = 0; x < D / 16; x++) {
            const float4 t = *(const float4*)(row + 16 * x + 4 * kq);
            kv[4 * x + 0] = t.x;
            kv[4 * x + 1] = t.y;
            kv[4 * x + 2] = t.z;
            kv[4 * x + 3] = t.w;
        }
    } else {
        const uint8_t* row = (const uint8_t*)base + off;
        const int e0 = kq * (D / 4);  // first element of this lane
        const int g = e0 >> 5;
        const uint32_t hdr = *(const uint32_t*)(row + kQ4GroupBytes * g);
        const float d = f16_bits_to_f32(hdr), dmin = f16_bits_to_f32(hdr >> 16);
        const uint32_t* nib = (const uint32_t*)(row + kQ4GroupBytes * g + 4 + ((e0 & 31) >> 1));
#pragma unroll
        for (int w = 0; w < D / 32; w++) q4_dequant8(nib[w], d, dmin, kv + 8 * w);
    }
}

// V operand of lane (col j, quad kq) for one row: DPL = D/16 consecutive dims
// starting at DPL*j.
template <int D, int KVT>
__device__ __forceinline__ void load_v(const void* base, long long off, int j, float* vv) {
    constexpr int DPL = D / 16;
    if (off < 0) {
#pragma unroll
        for (int t = 0; t < DPL; t++) vv[t] = 0.f;
        return;
    }
    if constexpr (KVT == NYION_KV_F32) {
        const float* row = (const float*)base + off + DPL * j;
#pragma unroll
        for (int x = 0; x < DPL / 4; x++) {
            const float4 t = *(const float4*)(row + 4 * x);
            vv[4 * x + 0] = t.x;
            vv[4 * x + 1] = t.y;
            vv[4 * x + 2] = t.z;
            vv[4 * x + 3] = t.w;
        }
    } else {
        const uint8_t* row = (const uint8_t*)base + off;
        const int e0 = DPL * j;
        const int g = e0 >> 5;
        const uint32_t hdr = *(const uint32_t*)(row + kQ4GroupBytes * g);
        const float d = f16_bits_to_f32(hdr), dmin = f16_bits_to_f32(hdr >> 16);
        const uint8_t* nb = row + kQ4GroupBytes * g + 4 + ((e0 & 31) >> 1);
        if constexpr (DPL == 8)
            q4_dequant8(*(const uint32_t*)nb, d, dmin, vv);
        else
            q4_dequant4((uint32_t)(*(const uint16_t*)nb), d, dmin, vv);
    }
}

// ---------------------------------------------------------------- kernel

template <int D, int KVT>
__global__ __launch_bounds__(256) void decode_kernel(DecodeArgs a) {
    constexpr int NC = D / 4;    // QK MFMAs per tile
    constexpr int DPL = D / 16;  // PV output tiles (dims per lane per row)

    const int lane = threadIdx.x & 63;
    const int p = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (p >= a.max_parts) return;
    const int kvh = blockIdx.y / a.n_hg;
    const int hg = blockIdx.y - kvh * a.n_hg;
    const int b = blockIdx.z;

    const SeqExtent e = seq_extent(a, b);
    const int j = lane & 15;
    const int kq = lane >> 4;
    const int g_local = min(16, a.group - hg * 16);
    const int head0 = kvh * a.group + hg * 16;
    if (e.L <= 0) {  // nothing to attend to (ctx_len <= 0 or q_pos < 0): zeros
        if (p == 0)
            for (int i = lane; i < g_local * D; i += 64)
                a.out[((long long)b * a.n_heads + head0) * D + i] = 0.f;
        return;
    }
    const int part_begin = p * a.part_tokens;
    if (part_begin >= e.L) return;  // wave-uniform
    const int part_end = min(e.L, part_begin + a.part_tokens);
    const int nparts = (e.L + a.part_tokens - 1) / a.part_tokens;

    RowMap m;
    m.table = a.tables ? a.tables + (long long)b * a.table_stride : nullptr;
    m.block_stride = a.block_stride;
    m.head_stride = a.head_stride;
    m.token_stride = a.token_stride;
    m.bt_log2 = a.bt_log2;
    m.num_blocks = a.num_blocks;
    m.table_len = a.table_stride;

    // Q operand (B of the QK product): head j, dims by qk_dim.  Heads past the
    // group are zero, so their S columns are 0 and never stored.
    float qv[NC];
    {
        const float* qrow = a.q + ((long long)b * a.n_heads + head0 + min(j, g_local - 1)) * D;
        const bool ok = j < g_local;
#pragma unroll
        for (int c = 0; c < NC; c++) qv[c] = ok ? qrow[qk_dim<D, KVT>(c, kq)] : 0.f;
    }

    floatx4 acc[DPL];
#pragma unroll
    for (int t = 0; t < DPL; t++) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
    float mrun = -INFINITY;  // running max (log2 domain), uniform over kq
    float lrun = 0.f;        // this lane's share of the denominator

    for (int t0 = part_begin; t0 < part_end; t0 += 16) {
        // K row of this lane: virtual token t0 + j.
        float kv[NC];
        {
            const int v = t0 + j;
            long long off = -1;
            if (v < part_end) {
                const int pos = virt_to_pos(a, e, b, v);
                if (pos >= 0) off = row_offset(m, pos, kvh);
            }
            load_k<D, KVT>(a.k, off, kq, kv);
        }
        // V rows of this lane: virtual tokens t0 + 4*kq + r.
        float vv[4][DPL];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int v = t0 + 4 * kq + r;
            long long off = -1;
            if (v < part_end) {
                const int pos = virt_to_pos(a, e, b, v);
                if (pos >= 0) off = row_offset(m, pos, kvh);
            }
            load_v<D, KVT>(a.v, off, j, vv[r]);
        }

        // S = K . Q^T   (lane: head j, tokens 4*kq + r in reg r)
        floatx4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NC; c++) s = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[c], qv[c], s, 0, 0, 0);

        float sv[4];
#pragma unroll
        for (int r = 0; r < 4; r++)
            sv[r] = (t0 + 4 * kq + r < part_end) ? s[r] * a.scale_log2 : -1e30f;
        float mt = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
        mt = fmaxf(mt, __shfl_xor(mt, 16));
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        const float mnew = fmaxf(mrun, mt);
        const float alpha = __builtin_amdgcn_exp2f(mrun - mnew);
        float pr[4];
#pragma unroll
        for (int r = 0; r < 4; r++) pr[r] = __builtin_amdgcn_exp2f(sv[r] - mnew);
        lrun = __builtin_fmaf(lrun, alpha, (pr[0] + pr[1]) + (pr[2] + pr[3]));
        mrun = mnew;

        // Rescale O: reg r' of this lane holds head 4*kq + r'.
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float ar = __shfl(alpha, 4 * kq + r);
#pragma unroll
            for (int t = 0; t < DPL; t++) acc[t][r] *= ar;
        }

        // O += P . V  (A = P straight from the S registers)
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int t = 0; t < DPL; t++)
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(pr[r], vv[r][t], acc[t], 0, 0, 0);
    }

    // Denominator per head column: sum the four token quads.
    float lt = lrun + __shfl_xor(lrun, 16);
    lt += __shfl_xor(lt, 32);

#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int hh = 4 * kq + r;  // head (within the 16-group) of acc[.][r]
        const float lh = __shfl(lt, hh);
        const float mh = __shfl(mrun, hh);
        if (hh < g_local) {
            const long long head = head0 + hh;
            if (nparts == 1) {
                const float inv = 1.0f / lh;
                float* o = a.out + ((long long)b * a.n_heads + head) * D + DPL * j;
#pragma unroll
                for (int x = 0; x < DPL / 4; x++)
                    *(float4*)(o + 4 * x) = float4{acc[4 * x + 0][r] * inv, acc[4 * x + 1][r] * inv,
                                                   acc[4 * x + 2][r] * inv, acc[4 * x + 3][r] * inv};
            } else {
                const long long slot = ((long long)b * a.n_heads + head) * a.max_parts + p;
                float* o = a.ws_acc + slot * D + DPL * j;
#pragma unroll
                for (int x = 0; x < DPL / 4; x++)
                    *(float4*)(o + 4 * x) =
                        float4{acc[4 * x + 0][r], acc[4 * x + 1][r], acc[4 * x + 2][r], acc[4 * x + 3][r]};
                if (j == 0) a.ws_ml[slot] = float2{mh, lh};
            }
        }
    }
}

// Log-sum-exp merge of the split-K partials of one (sequence, q head).
// 64 threads, thread = dims tid, tid+64.
template <int D>
__global__ __launch_bounds__(64) void decode_merge_kernel(DecodeArgs a) {
    const int head = blockIdx.x;
    const int b = blockIdx.y;
    const int tid = threadIdx.x;
    const SeqExtent e = seq_extent(a, b);
    float* o = a.out + ((long long)b * a.n_heads + head) * D;
    if (e.L <= 0) return;  // zeros written by decode_kernel
    const int nparts = (e.L + a.part_tokens - 1) / a.part_tokens;
    if (nparts <= 1) return;  // written by decode_kernel
    const long long base = ((long long)b * a.n_heads + head) * a.max_parts;
    float mx = -INFINITY;
    for (int p = 0; p < nparts; p++) mx = fmaxf(mx, a.ws_ml[base + p].x);
    float lsum = 0.f;
    float accd[D / 64];
#pragma unroll
    for (int x = 0; x < D / 64; x++) accd[x] = 0.f;
    for (int p = 0; p < nparts; p++) {
        const float2 ml = a.ws_ml[base + p];
        const float w = __builtin_amdgcn_exp2f(ml.x - mx);
        lsum = __builtin_fmaf(ml.y, w, lsum);
        const float* src = a.ws_acc + (base + p) * D;
#pragma unroll
        for (int x = 0; x < D / 64; x++) accd[x] = __builtin_fmaf(w, src[tid + 64 * x], accd[x]);
    }
    const float inv = 1.0f / lsum;
#pragma unroll
    for (int x = 0; x < D / 64; x++) o[tid + 64 * x] = accd[x] * inv;
}

// ---------------------------------------------------------------- host side

static int g_part_override = 0;

static int pick_partition(int batch, int units_per_seq, int max_len) {
    if (g_part_override > 0) return g_part_override;
    // Enough wavefronts to keep 256 CUs busy through the tail (about 32 per
    // CU over the whole grid), but partitions as long as possible so the
    // partial write-back stays small next to the K/V bytes streamed.
    const long long token_units = (long long)batch * units_per_seq * (long long)max_len;
    const long long target = 8192;
    long long want = token_units / target;
    int p = 32;
    while (p < want && p < 4096) p <<= 1;
    return p;
}

struct DecodePlan {
    DecodeArgs a;
    dim3 grid;
    size_t ws_bytes;
    int head_dim;
    int kvt;
};

static size_t ws_bytes_for(int batch, int n_heads, int head_dim, int max_parts) {
    if (max_parts <= 1) return 0;
    const size_t slots = (size_t)batch * n_heads * max_parts;
    return slots * head_dim * sizeof(float) + slots * sizeof(float2) + 256;
}

static int plan_common(DecodePlan& pl, int batch, int n_heads, int n_kv_heads, int head_dim,
                       int kvt, int max_len, float scale) {
    if (batch <= 0 || n_heads <= 0 || n_kv_heads <= 0)
        return set_error(NYION_ERR_INVALID, "decode: batch/heads must be positive");
    if (n_heads % n_kv_heads)
        return set_error(NYION_ERR_INVALID, "decode: n_heads %d not a multiple of n_kv_heads %d",
                         n_heads, n_kv_heads);
    if (head_dim != 64 && head_dim != 128)
        return set_error(NYION_ERR_UNSUPPORTED, "decode: head_dim %d (supported: 64, 128)", head_dim);
    if (kvt != NYION_KV_F32 && kvt != NYION_KV_Q4_20B)
        return set_error(NYION_ERR_INVALID, "decode: kv_dtype %d", kvt);
    if (max_len <= 0) return set_error(NYION_ERR_INVALID, "decode: max_ctx must be positive");
    if (batch > 65535) return set_error(NYION_ERR_UNSUPPORTED, "decode: batch %d > 65535", batch);
    DecodeArgs& a = pl.a;
    a = DecodeArgs{};
    a.n_heads = n_heads;
    a.n_kv_heads = n_kv_heads;
    a.group = n_heads / n_kv_heads;
    a.n_hg = (a.group + 15) / 16;
    const float sc = scale > 0.f ? scale : 1.0f / sqrtf((float)head_dim);
    a.scale_log2 = sc * 1.4426950408889634f;
    a.part_tokens = pick_partition(batch, n_kv_heads * a.n_hg, max_len);
    a.max_parts = (max_len + a.part_tokens - 1) / a.part_tokens;
    a.max_len = max_len;
    pl.head_dim = head_dim;
    pl.kvt = kvt;
    pl.grid = dim3((a.max_parts + 3) / 4, n_kv_heads * a.n_hg, batch);
    pl.ws_bytes = ws_bytes_for(batch, n_heads, head_dim, a.max_parts);
    return NYION_OK;
}

static int attach_workspace(DecodePlan& pl, void* ws, size_t ws_bytes, int batch) {
    if (pl.ws_bytes == 0) return NYION_OK;
    if (!ws || ws_bytes < pl.ws_bytes)
        return set_error(NYION_ERR_WORKSPACE, "decode: workspace %zu bytes < required %zu", ws_bytes,
                         pl.ws_bytes);
    if (!aligned(ws, 16)) return set_error(NYION_ERR_INVALID, "decode: workspace not 16-byte aligned");
    const size_t slots = (size_t)batch * pl.a.n_heads * pl.a.max_parts;
    pl.a.ws_acc = (float*)ws;
    size_t acc_bytes = (slots * pl.head_dim * sizeof(float) + 255) & ~(size_t)255;
    pl.a.ws_ml = (float2*)((char*)ws + acc_bytes);
    return NYION_OK;
}

static int launch_plan(const DecodePlan& pl, int batch, hipStream_t stream) {
    const int D = pl.head_dim;
#define NYION_DECODE_LAUNCH(DD, KK)                                                        \
    hipLaunchKernelGGL((decode_kernel<DD, KK>), pl.grid, dim3(256), 0, stream, pl.a);      \
    if (pl.a.max_parts > 1)                                                                \
        hipLaunchKernelGGL((decode_merge_kernel<DD>), dim3(pl.a.n_heads, batch), dim3(64), 0, \
                           stream, pl.a);
    if (D == 64 && pl.kvt == NYION_KV_F32) {
        NYION_DECODE_LAUNCH(64, NYION_KV_F32)
    } else if (D == 64) {
        NYION_DECODE_LAUNCH(64, NYION_KV_Q4_20B)
    } else if (pl.kvt == NYION_KV_F32) {
        NYION_DECODE_LAUNCH(128, NYION_KV_F32)
    } else {
        NYION_DECODE_LAUNCH(128, NYION_KV_Q4_20B)
    }
#undef NYION_DECODE_LAUNCH
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

}  // namespace nyion

using namespace nyion;

extern "C" {

int nyion_set_decode_partition_tokens(int tokens) {
    if (tokens != 0 && (tokens < 16 || tokens > 4096 || !is_pow2(tokens)))
        return set_error(NYION_ERR_INVALID, "partition tokens %d: power of two in [16, 4096] or 0",
                         tokens);
    g_part_override = tokens;
    return NYION_OK;
}

int nyion_get_decode_partition_tokens(int batch, int n_kv_heads, int head_dim, int max_len) {
    (void)head_dim;
    return pick_partition(batch, n_kv_heads, max_len);
}

static int window_max_len(int max_ctx, int window, int global_stride) {
    if (window <= 0) return max_ctx;
    long long L = (long long)window + 1 + (global_stride > 0 ? 128 : 0);
    if (L > (long long)max_ctx + 128) L = (long long)max_ctx + 128;
    return (int)L;
}

size_t nyion_paged_decode_workspace_size(int batch, int n_heads, int n_kv_heads, int head_dim,
                                         int max_ctx, int window, int global_stride) {
    DecodePlan pl;
    if (plan_common(pl, batch, n_heads, n_kv_heads, head_dim, NYION_KV_F32,
                    window_max_len(max_ctx, window, global_stride), 0.f) != NYION_OK)
        return 0;
    return pl.ws_bytes;
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
    if ((long long)max_ctx > (long long)max_blocks_per_seq * block_tokens)
        return set_error(NYION_ERR_INVALID,
                         "paged decode: max_ctx %d exceeds max_blocks_per_seq*block_tokens", max_ctx);
    DecodePlan pl;
    if ((rc = plan_common(pl, batch, n_heads, n_kv_heads, head_dim, kv_dtype,
                          window_max_len(max_ctx, window, global_stride), scale)) != NYION_OK)
        return rc;
    if ((rc = attach_workspace(pl, d_workspace, workspace_bytes, batch)) != NYION_OK) return rc;
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
    return launch_plan(pl, batch, (hipStream_t)stream);
}

size_t nyion_paged_decode_positions_workspace_size(int batch, int n_heads, int n_kv_heads,
                                                   int head_dim, int max_positions) {
    DecodePlan pl;
    if (plan_common(pl, batch, n_heads, n_kv_heads, head_dim, NYION_KV_F32, max_positions, 0.f) !=
        NYION_OK)
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
    if ((rc = plan_common(pl, batch, n_heads, n_kv_heads, head_dim, kv_dtype, max_positions,
                          scale)) != NYION_OK)
        return rc;
    if ((rc = attach_workspace(pl, d_workspace, workspace_bytes, batch)) != NYION_OK) return rc;
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
    return launch_plan(pl, batch, (hipStream_t)stream);
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
                          (int)seq_len, 0.f)) != NYION_OK)
        return rc;
    // The node's scores buffer (n_heads*kv_stride floats) is the split-K
    // workspace; without it run one partition per head group.
    DecodeArgs& a = pl.a;
    const size_t scores_bytes = d_scores ? (size_t)n_heads * kv_stride * sizeof(float) : 0;
    if (pl.ws_bytes > scores_bytes) {
        int p = a.part_tokens;
        while (p < (1 << 30) && ws_bytes_for(1, (int)n_heads, (int)head_dim,
                                             (int)((seq_len + p - 1) / p)) > scores_bytes)
            p <<= 1;
        a.part_tokens = p;
        a.max_parts = (int)((seq_len + p - 1) / p);
        pl.grid = dim3((a.max_parts + 3) / 4, a.n_kv_heads * a.n_hg, 1);
        pl.ws_bytes = ws_bytes_for(1, (int)n_heads, (int)head_dim, a.max_parts);
    }
    if ((rc = attach_workspace(pl, d_scores, scores_bytes, 1)) != NYION_OK) return rc;
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
    return launch_plan(pl, 1, (hipStream_t)stream);
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
