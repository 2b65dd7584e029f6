// kv_cache.hip — paged KV writes (f32 copy or on-device Q4-20B quantise),
// and the debug gather / dequantise / quantise kernels.
//
// Q4-20B quantisation restates PagedKVCache::save / save_at
// (swamp-engine/src/cache.rs:637-663, 771-806) byte for byte:
//   d = max|x|/7 (0 when max|x| <= 1e-10), dmin = min x, in f32;
//   stored as IEEE f16 (round to nearest even) at bytes [0,2), [2,4);
//   q = clamp(round_half_away((x - dmin)/d), 0, 15) with the f32 d, dmin;
//   element i -> byte 4 + i/2, low nibble when i is even.
// The library is compiled with -ffp-contract=off, so (x - dmin)/d and the
// dequantiser's d*nib + dmin keep their separate roundings; division is the
// correctly rounded IEEE divide.
#include <float.h>
#include <math.h>

#include <vector>

#include "common.hpp"
#include "kv_write.hpp"

namespace nyion {

__device__ __forceinline__ uint32_t f32_to_f16_bits(float x) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x);
}

// Quantise one group of `len` (<= 32) elements into 5 words (20 bytes).
__device__ __forceinline__ void q4_quantize_group(const float* x, int len, uint32_t w[5]) {
    float mx = 0.0f, mn = FLT_MAX;
    for (int i = 0; i < len; i++) {
        mx = fmaxf(mx, fabsf(x[i]));
        mn = fminf(mn, x[i]);
    }
    const float d = (mx > 1e-10f) ? mx / 7.0f : 0.0f;
    const float dmin = mn;
    w[0] = f32_to_f16_bits(d) | (f32_to_f16_bits(dmin) << 16);
    w[1] = w[2] = w[3] = w[4] = 0u;
    if (d > 1e-10f) {
        for (int i = 0; i < len; i++) {
            float r = roundf((x[i] - dmin) / d);
            r = fmaxf(r, 0.0f);
            r = fminf(r, 15.0f);
            w[1 + (i >> 3)] |= ((uint32_t)r) << (4 * (i & 7));
        }
    }
}

// Eight lanes quantise one 32-element group together (lanes 8j .. 8j+7 of a
// wavefront, every lane active): lane k holds elements 4k .. 4k+3.  The
// group's max |x| and min x are taken across the eight lanes with DPP (the
// operations are exact, so the order does not matter), d and dmin are the
// same f32 values q4_quantize_group computes, and each lane rounds its own
// four elements.  Returns, in lanes k = 0..4 of the eight, word k of the
// group's 20 bytes (the header, then the nibble words).
template <int CTRL>
__device__ __forceinline__ float q4_dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(x), __float_as_int(x), CTRL, 0xf,
                                                      0xf, false));
}

__device__ __forceinline__ uint32_t q4_quantize_group8(float4 x) {
    // from 0 and FLT_MAX as the reference's fold (a NaN element is passed over)
    float mx = fmaxf(fmaxf(fmaxf(0.0f, fabsf(x.x)), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w)));
    float mn = fminf(fminf(fminf(FLT_MAX, x.x), x.y), fminf(x.z, x.w));
    mx = fmaxf(mx, q4_dpp<0xb1>(mx));   // quad_perm [1,0,3,2]
    mn = fminf(mn, q4_dpp<0xb1>(mn));
    mx = fmaxf(mx, q4_dpp<0x4e>(mx));   // quad_perm [2,3,0,1]
    mn = fminf(mn, q4_dpp<0x4e>(mn));
    mx = fmaxf(mx, q4_dpp<0x141>(mx));  // row_half_mirror: the eight lanes
    mn = fminf(mn, q4_dpp<0x141>(mn));
    const float d = (mx > 1e-10f) ? mx / 7.0f : 0.0f;
    const float dmin = mn;
    uint32_t bits = 0;  // this lane's four nibbles: bytes 2k and 2k+1 of the nibble area
    if (d > 1e-10f) {
        const float e[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float r = roundf((e[i] - dmin) / d);
            r = fminf(fmaxf(r, 0.0f), 15.0f);
            bits |= ((uint32_t)r) << (4 * i);
        }
    }
    // nibble word j (1..4) = lanes 2j-2 (low half) and 2j-1 (high half)
    const uint32_t other =
        (uint32_t)__builtin_amdgcn_update_dpp((int)bits, (int)bits, 0xb1, 0xf, 0xf, false);
    const uint32_t pair = bits | (other << 16);  // valid in even lanes
    const int k = threadIdx.x & 7;
    const int base = threadIdx.x & ~7;
    // lane k (1..4) takes the pair word of lane 2k-2 of its group
    const uint32_t nib = (uint32_t)__shfl((int)pair, base + 2 * (k > 0 ? k - 1 : 0));
    const uint32_t hdr = f32_to_f16_bits(d) | (f32_to_f16_bits(dmin) << 16);
    return k == 0 ? hdr : nib;
}

// ------------------------------------------------------------- kernels

// One thread per (row, head, 4 values): f32 rows, or binary16 rows (F16).
// With a bf16 source the kernel also records, in the range-status word,
// whether some V value reaches 65520 in magnitude: the prefill computed
// P.V with V in binary16, which cannot hold it (checked here, where V is
// read anyway, instead of in the prefill's inner loop).
template <bool F16>
__global__ void kv_write_flat_kernel(WriteArgs a) {
    const int vec = a.head_dim / 4;
    const long long n = (long long)a.rows * a.n_kv_heads * vec;
    float vmax = 0.f;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n;
         i += (long long)gridDim.x * blockDim.x) {
        const int x = (int)(i % vec);
        const int h = (int)((i / vec) % a.n_kv_heads);
        const int r = (int)(i / ((long long)vec * a.n_kv_heads));
        vmax = fmaxf(vmax, write_kv_vec<F16>(a, r, h, x));
    }
    if (a.k16) report_range(a.status, vmax >= 65520.f, kRangePrefillV);
}

// The same V range check on its own, for a prefill without a KV write:
// v [n] bf16 (n a multiple of 4, 8-byte aligned).
__global__ void v_range_kernel(const uint16_t* v, long long n, unsigned* status) {
    float vmax = 0.f;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; 4 * i < n;
         i += (long long)gridDim.x * blockDim.x)
        vmax = fmaxf(vmax, v_absmax(*(const uint2*)(v + 4 * i)));
    report_range(status, vmax >= 65520.f, kRangePrefillV);
}

int v_range_check(const uint16_t* v, long long n, hipStream_t stream) {
    unsigned* st = device_status_word();
    if (!st) return NYION_OK;
    long long g = (n / 4 + 255) / 256;
    if (g > 2048) g = 2048;
    if (g < 1) g = 1;
    hipLaunchKernelGGL(v_range_kernel, dim3((unsigned)g), dim3(256), 0, stream, v, n, st);
    return check_launch("prefill V range check");
}

// Eight lanes per (row, head, group), 4 elements a lane (head_dim a multiple
// of 32): the f32 or bf16 rows are read contiguously across the wavefront.
// The grid-stride loop runs whole wavefronts (the DPP exchange needs every
// lane), items past the end store nothing.
__global__ __launch_bounds__(256) void kv_write_q4x8_kernel(WriteArgs a) {
    const int groups = a.head_dim / 32;
    const long long n = (long long)a.rows * a.n_kv_heads * groups * 8;
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i0 = (long long)blockIdx.x * blockDim.x; i0 < n; i0 += stride) {
        const long long i = i0 + threadIdx.x;
        const bool ok = i < n;
        const long long item = ok ? i >> 3 : 0;
        const int k = (int)(i & 7);
        const int g = (int)(item % groups);
        const int h = (int)((item / groups) % a.n_kv_heads);
        const int r = (int)(item / ((long long)groups * a.n_kv_heads));
        const long long src = ((long long)r * a.n_kv_heads + h) * a.head_dim + 32 * g + 4 * k;
        float4 kx, vx;
        if (a.k16) {
            kx = bf16x4_to_f32(*(const uint2*)(a.k16 + src));
            vx = bf16x4_to_f32(*(const uint2*)(a.v16 + src));
        } else {
            kx = *(const float4*)(a.k + src);
            vx = *(const float4*)(a.v + src);
        }
        const uint32_t wk = q4_quantize_group8(kx);
        const uint32_t wv = q4_quantize_group8(vx);
        const long long off = ok ? write_row_offset(a, r, h) : -1;
        if (off >= 0 && k < 5) {
            *(uint32_t*)((uint8_t*)a.k_pool + off + kQ4GroupBytes * g + 4 * k) = wk;
            *(uint32_t*)((uint8_t*)a.v_pool + off + kQ4GroupBytes * g + 4 * k) = wv;
        }
    }
}

// One thread per (row, head, group): quantise K and V groups (any head_dim).
__global__ void kv_write_q4_kernel(WriteArgs a) {
    const int groups = (a.head_dim + 31) / 32;
    const long long n = (long long)a.rows * a.n_kv_heads * groups;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n;
         i += (long long)gridDim.x * blockDim.x) {
        const int g = (int)(i % groups);
        const int h = (int)((i / groups) % a.n_kv_heads);
        const int r = (int)(i / ((long long)groups * a.n_kv_heads));
        const long long off = write_row_offset(a, r, h);
        if (off < 0) continue;
        const long long src = ((long long)r * a.n_kv_heads + h) * a.head_dim + 32 * g;
        const int len = min(32, a.head_dim - 32 * g);
        float kb[32], vb[32];
        const float* ks = a.k + (a.k16 ? 0 : src);
        const float* vs = a.v + (a.k16 ? 0 : src);
        if (a.k16) {
            for (int e = 0; e < len; e++) {
                kb[e] = __uint_as_float((uint32_t)a.k16[src + e] << 16);
                vb[e] = __uint_as_float((uint32_t)a.v16[src + e] << 16);
            }
            ks = kb;
            vs = vb;
        }
        uint32_t w[5];
        q4_quantize_group(ks, len, w);
        uint32_t* dk = (uint32_t*)((uint8_t*)a.k_pool + off + kQ4GroupBytes * g);
#pragma unroll
        for (int t = 0; t < 5; t++) dk[t] = w[t];
        q4_quantize_group(vs, len, w);
        uint32_t* dv = (uint32_t*)((uint8_t*)a.v_pool + off + kQ4GroupBytes * g);
#pragma unroll
        for (int t = 0; t < 5; t++) dv[t] = w[t];
    }
}

// ------------------------------------------------------------- RoPE

// apply_rotation_pair (swamp-engine/src/ops.rs:67-79): x*cos - y*sin,
// x*sin + y*cos, each product rounded before the add (no contraction).
__device__ __forceinline__ float2 rope_pair(float x, float y, float2 cs) {
    return float2{x * cs.x - y * cs.y, x * cs.y + y * cs.x};
}

struct RopeArgs {
    float* q;              // [B][Hq][D], rotated in place
    const float* k;        // [B][Hkv][D] (before RoPE)
    const float2* lut;     // [max_ctx][D/2] (cos, sin)
    int max_ctx;
    int n_heads;
    WriteArgs w;           // k: unused (rotated on the fly), v: source of V rows
};

// One launch for the decode-step QKV epilogue.  Items [0, nq): one q pair
// (b, head, k) each; items [nq, nq + nkv): one K/V unit each -- a pair (f32
// pools) or a 32-element group (Q4-20B pools) of (b, kv head).
template <int KVT>
__global__ __launch_bounds__(256) void rope_kv_append_kernel(RopeArgs a, long long nq, long long nkv) {
    const int D = a.w.head_dim;
    const int half = D / 2;
    for (long long i = blockIdx.x * 256LL + threadIdx.x; i < nq + nkv; i += (long long)gridDim.x * 256) {
        if (i < nq) {
            const int k = (int)(i % half);
            const long long row = i / half;  // b * Hq + head
            const int b = (int)(row / a.n_heads);
            const int pos = a.w.positions[b];
            if (pos < 0) continue;
            const float2 cs = a.lut[(long long)min(pos, a.max_ctx - 1) * half + k];
            float* qp = a.q + row * D + 2 * k;
            const float2 r = rope_pair(qp[0], qp[1], cs);
            qp[0] = r.x;
            qp[1] = r.y;
            continue;
        }
        const long long j = i - nq;
        const int units = KVT == NYION_KV_Q4_20B ? (D + 31) / 32 : half;
        const int u = (int)(j % units);
        const int h = (int)((j / units) % a.w.n_kv_heads);
        const int b = (int)(j / ((long long)units * a.w.n_kv_heads));
        const int pos = a.w.positions[b];
        const long long off = write_row_offset(a.w, b, h);
        if (pos < 0 || off < 0) continue;
        const float2* cs = a.lut + (long long)min(pos, a.max_ctx - 1) * half;
        const long long src = ((long long)b * a.w.n_kv_heads + h) * D;
        if constexpr (KVT == NYION_KV_F32) {
            const float2 r = rope_pair(a.k[src + 2 * u], a.k[src + 2 * u + 1], cs[u]);
            *(float2*)((float*)a.w.k_pool + off + 2 * u) = r;
            *(float2*)((float*)a.w.v_pool + off + 2 * u) = *(const float2*)(a.w.v + src + 2 * u);
        } else if constexpr (KVT == NYION_KV_F16) {
            const float2 r = rope_pair(a.k[src + 2 * u], a.k[src + 2 * u + 1], cs[u]);
            *(uint32_t*)((uint16_t*)a.w.k_pool + off + 2 * u) = f16x2_bits(r.x, r.y);
            const float2 vv = *(const float2*)(a.w.v + src + 2 * u);
            *(uint32_t*)((uint16_t*)a.w.v_pool + off + 2 * u) = f16x2_bits(vv.x, vv.y);
        } else {
            const int len = min(32, D - 32 * u);
            float kb[32];
            for (int e = 0; e < len; e += 2) {
                const float2 r = rope_pair(a.k[src + 32 * u + e], a.k[src + 32 * u + e + 1],
                                           cs[16 * u + e / 2]);
                kb[e] = r.x;
                kb[e + 1] = r.y;
            }
            uint32_t w[5];
            q4_quantize_group(kb, len, w);
            uint32_t* dk = (uint32_t*)((uint8_t*)a.w.k_pool + off + kQ4GroupBytes * u);
#pragma unroll
            for (int t = 0; t < 5; t++) dk[t] = w[t];
            q4_quantize_group(a.w.v + src + 32 * u, len, w);
            uint32_t* dv = (uint32_t*)((uint8_t*)a.w.v_pool + off + kQ4GroupBytes * u);
#pragma unroll
            for (int t = 0; t < 5; t++) dv[t] = w[t];
        }
    }
}

struct GatherArgs {
    const void* pool;
    const int32_t* table;
    float* out;         // [Hkv][n_tokens][D] f32, or
    uint16_t* out_bf16; // [n_tokens][Hkv][D] bf16 (the prefill kernel's history layout)
    long long block_stride;
    long long head_stride;
    int token_stride;
    int bt_log2;
    int num_blocks;
    int n_kv_heads;
    int head_dim;
    int n_tokens;
    int kvt;
    ZoneMap zone;  // zone geometry when zone.page_base is set (table unused)
};

// f32 -> bf16 bits, round to nearest even; NaN -> the quiet NaN 0x7fc0 with
// the sign kept.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    const uint32_t x = __float_as_uint(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return ((x >> 16) & 0x8000u) | 0x7fc0u;
    return (x + 0x7fffu + ((x >> 16) & 1u)) >> 16;
}

// One thread per (head, token, 8 dims), through the decode kernels' RowMap
// and q4_dequant8.
template <bool BF16>
__global__ void kv_gather_kernel(GatherArgs a) {
    const int vec = a.head_dim / 8;
    const long long n = (long long)a.n_kv_heads * a.n_tokens * vec;
    RowMap m;
    m.table = a.table;
    m.block_stride = a.block_stride;
    m.head_stride = a.head_stride;
    m.token_stride = a.token_stride;
    m.bt_log2 = a.bt_log2;
    m.num_blocks = a.num_blocks;
    m.table_len = (a.n_tokens + (1 << a.bt_log2) - 1) >> a.bt_log2;
    m.zone = a.zone;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n;
         i += (long long)gridDim.x * blockDim.x) {
        const int x = (int)(i % vec);
        const int t = (int)((i / vec) % a.n_tokens);
        const int h = (int)(i / ((long long)vec * a.n_tokens));
        const long long off = row_offset(m, t, h);
        float vals[8];
        if (off < 0) {
            for (int e = 0; e < 8; e++) vals[e] = __builtin_nanf("");
        } else if (a.kvt == NYION_KV_F32) {
            const float* src = (const float*)a.pool + off + 8 * x;
            for (int e = 0; e < 8; e++) vals[e] = src[e];
        } else if (a.kvt == NYION_KV_F16) {
            const uint4 w = *(const uint4*)((const uint16_t*)a.pool + off + 8 * x);
            const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
            for (int e = 0; e < 4; e++) {
                const halfx2_t hv = __builtin_bit_cast(halfx2_t, ws[e]);
                vals[2 * e] = (float)hv[0];
                vals[2 * e + 1] = (float)hv[1];
            }
        } else {
            const uint8_t* row = (const uint8_t*)a.pool + off;
            const int e0 = 8 * x;
            const int g = e0 >> 5;
            const uint32_t hdr = *(const uint32_t*)(row + kQ4GroupBytes * g);
            const uint32_t w = *(const uint32_t*)(row + kQ4GroupBytes * g + 4 + ((e0 & 31) >> 1));
            q4_dequant8(w, f16_bits_to_f32(hdr), f16_bits_to_f32(hdr >> 16), vals);
        }
        if (BF16) {
            uint4 w;
            w.x = f32_to_bf16_bits(vals[0]) | (f32_to_bf16_bits(vals[1]) << 16);
            w.y = f32_to_bf16_bits(vals[2]) | (f32_to_bf16_bits(vals[3]) << 16);
            w.z = f32_to_bf16_bits(vals[4]) | (f32_to_bf16_bits(vals[5]) << 16);
            w.w = f32_to_bf16_bits(vals[6]) | (f32_to_bf16_bits(vals[7]) << 16);
            *(uint4*)(a.out_bf16 + ((long long)t * a.n_kv_heads + h) * a.head_dim + 8 * x) = w;
        } else {
            float* dst = a.out + ((long long)h * a.n_tokens + t) * a.head_dim + 8 * x;
            for (int e = 0; e < 8; e++) dst[e] = vals[e];
        }
    }
}

// Row-wise Q4-20B dequantise: one thread per (row, 8 elements).
__global__ void q4_dequant_kernel(const uint8_t* in, long long n_rows, int head_dim, float* out) {
    const int vec = head_dim / 8;
    const int rb = q4_row_bytes(head_dim);
    const long long n = n_rows * vec;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n;
         i += (long long)gridDim.x * blockDim.x) {
        const long long r = i / vec;
        const int e0 = 8 * (int)(i % vec);
        const uint8_t* row = in + r * rb;
        const int g = e0 >> 5;
        const uint32_t hdr = *(const uint32_t*)(row + kQ4GroupBytes * g);
        const uint32_t w = *(const uint32_t*)(row + kQ4GroupBytes * g + 4 + ((e0 & 31) >> 1));
        float vals[8];
        q4_dequant8(w, f16_bits_to_f32(hdr), f16_bits_to_f32(hdr >> 16), vals);
        float* dst = out + r * head_dim + e0;
        for (int e = 0; e < 8; e++) dst[e] = vals[e];
    }
}

// Row-wise Q4-20B quantise, eight lanes per group (head_dim a multiple of
// 32, in 16-byte aligned): whole wavefronts per grid-stride step.
__global__ __launch_bounds__(256) void q4_quantize_x8_kernel(const float* in, long long n_rows,
                                                             int head_dim, uint8_t* out) {
    const int groups = head_dim / 32;
    const int rb = q4_row_bytes(head_dim);
    const long long n = n_rows * groups * 8;
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i0 = (long long)blockIdx.x * blockDim.x; i0 < n; i0 += stride) {
        const long long i = i0 + threadIdx.x;
        const bool ok = i < n;
        const long long item = ok ? i >> 3 : 0;  // (row, group), in order
        const float4 x = *(const float4*)(in + item * 32 + 4 * (i & 7));
        const uint32_t w = q4_quantize_group8(x);
        const long long r = item / groups;
        const int g = (int)(item % groups);
        if (ok && (i & 7) < 5) *(uint32_t*)(out + r * rb + kQ4GroupBytes * g + 4 * (i & 7)) = w;
    }
}

// Row-wise Q4-20B quantise: one thread per (row, group) (any head_dim).
__global__ void q4_quantize_kernel(const float* in, long long n_rows, int head_dim, uint8_t* out) {
    const int groups = (head_dim + 31) / 32;
    const int rb = q4_row_bytes(head_dim);
    const long long n = n_rows * groups;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n;
         i += (long long)gridDim.x * blockDim.x) {
        const long long r = i / groups;
        const int g = (int)(i % groups);
        uint32_t w[5];
        q4_quantize_group(in + r * head_dim + 32 * g, min(32, head_dim - 32 * g), w);
        uint32_t* dst = (uint32_t*)(out + r * rb + kQ4GroupBytes * g);
        for (int t = 0; t < 5; t++) dst[t] = w[t];
    }
}

static int grid_for(long long n, int block) {
    long long g = (n + block - 1) / block;
    if (g > 65536) g = 65536;
    if (g < 1) g = 1;
    return (int)g;
}

// Pools, row format and heads (either geometry).
static int fill_write_rows(WriteArgs& a, void* k_pool, void* v_pool, int n_kv_heads, int head_dim,
                           int kv_dtype) {
    if (!k_pool || !v_pool) return set_error(NYION_ERR_INVALID, "kv write: null pool");
    if (n_kv_heads <= 0) return set_error(NYION_ERR_INVALID, "kv write: n_kv_heads");
    if (kv_dtype == NYION_KV_F32) {
        if (head_dim <= 0 || head_dim % 4)
            return set_error(NYION_ERR_UNSUPPORTED, "kv write f32: head_dim %d not a multiple of 4",
                             head_dim);
        if (!aligned(k_pool, 16) || !aligned(v_pool, 16))
            return set_error(NYION_ERR_INVALID, "kv write f32: pools must be 16-byte aligned");
    } else if (kv_dtype == NYION_KV_F16) {
        if (head_dim <= 0 || head_dim % 4)
            return set_error(NYION_ERR_UNSUPPORTED, "kv write f16: head_dim %d not a multiple of 4",
                             head_dim);
        if (!aligned(k_pool, 8) || !aligned(v_pool, 8))
            return set_error(NYION_ERR_INVALID, "kv write f16: pools must be 8-byte aligned");
    } else if (kv_dtype == NYION_KV_Q4_20B) {
        if (head_dim <= 0) return set_error(NYION_ERR_INVALID, "kv write q4: head_dim");
        if (!aligned(k_pool, 4) || !aligned(v_pool, 4))
            return set_error(NYION_ERR_INVALID, "kv write q4: pools must be 4-byte aligned");
    } else {
        return set_error(NYION_ERR_INVALID, "kv write: kv_dtype %d", kv_dtype);
    }
    const long long row = kv_dtype == NYION_KV_Q4_20B ? q4_row_bytes(head_dim) : head_dim;
    a.k_pool = k_pool;
    a.v_pool = v_pool;
    a.n_kv_heads = n_kv_heads;
    a.head_dim = head_dim;
    a.token_stride = (int)row;
    return NYION_OK;
}

// The above plus the block-table geometry.
static int fill_write_args(WriteArgs& a, void* k_pool, void* v_pool, int block_tokens,
                           int num_blocks, int n_kv_heads, int head_dim, int kv_dtype) {
    int rc;
    if ((rc = fill_write_rows(a, k_pool, v_pool, n_kv_heads, head_dim, kv_dtype)) != NYION_OK)
        return rc;
    if (!is_pow2(block_tokens) || block_tokens > (1 << 20))
        return set_error(NYION_ERR_INVALID, "kv write: block_tokens %d not a power of two",
                         block_tokens);
    if (num_blocks <= 0) return set_error(NYION_ERR_INVALID, "kv write: num_blocks");
    a.bt_log2 = ilog2(block_tokens);
    a.num_blocks = num_blocks;
    a.head_stride = (long long)block_tokens * a.token_stride;
    a.block_stride = (long long)n_kv_heads * block_tokens * a.token_stride;
    return NYION_OK;
}

static int launch_write(const WriteArgs& a, int kv_dtype, hipStream_t stream) {
    if (kv_dtype == NYION_KV_F32 || kv_dtype == NYION_KV_F16) {
        const long long n = (long long)a.rows * a.n_kv_heads * (a.head_dim / 4);
        if (kv_dtype == NYION_KV_F16)
            hipLaunchKernelGGL(kv_write_flat_kernel<true>, dim3(grid_for(n, 256)), dim3(256), 0, stream, a);
        else
            hipLaunchKernelGGL(kv_write_flat_kernel<false>, dim3(grid_for(n, 256)), dim3(256), 0, stream, a);
    } else if (a.head_dim % 32 == 0 && (a.k16 ? aligned(a.k16, 8) && aligned(a.v16, 8)
                                                : aligned(a.k, 16) && aligned(a.v, 16))) {
        const long long n = (long long)a.rows * a.n_kv_heads * (a.head_dim / 32) * 8;
        hipLaunchKernelGGL(kv_write_q4x8_kernel, dim3(grid_for(n, 256)), dim3(256), 0, stream, a);
    } else {
        const long long n = (long long)a.rows * a.n_kv_heads * ((a.head_dim + 31) / 32);
        hipLaunchKernelGGL(kv_write_q4_kernel, dim3(grid_for(n, 256)), dim3(256), 0, stream, a);
    }
    return check_launch("kv write");
}

// Used by the prefill entry point (prefill_attention.hip).
int kv_write_impl(void* k_pool, void* v_pool, const int32_t* block_table, int block_tokens,
                  int num_blocks, int n_kv_heads, int head_dim, int kv_dtype, int start_pos,
                  int n_tokens, const float* k, const float* v, hipStream_t stream) {
    int rc;
    WriteArgs a{};
    if ((rc = fill_write_args(a, k_pool, v_pool, block_tokens, num_blocks, n_kv_heads, head_dim,
                              kv_dtype)) != NYION_OK)
        return rc;
    if (!block_table || !k || !v) return set_error(NYION_ERR_INVALID, "kv write: null argument");
    if (start_pos < 0 || n_tokens <= 0)
        return set_error(NYION_ERR_INVALID, "kv write: start_pos %d, n_tokens %d", start_pos, n_tokens);
    if (kv_dtype != NYION_KV_Q4_20B && (!aligned(k, 16) || !aligned(v, 16)))
        return set_error(NYION_ERR_INVALID, "kv write: k/v must be 16-byte aligned");
    a.tables = block_table;
    a.positions = nullptr;
    a.k = k;
    a.v = v;
    a.table_stride = (int)(((long long)start_pos + n_tokens + block_tokens - 1) / block_tokens);
    a.start_pos = start_pos;
    a.rows = n_tokens;
    a.per_seq = 0;
    return launch_write(a, kv_dtype, stream);
}

int prefill_write_args(WriteArgs& a, void* k_pool, void* v_pool, const int32_t* block_table,
                       int block_tokens, int num_blocks, int n_kv_heads, int head_dim, int kv_dtype,
                       int start_pos, int n_tokens, const uint16_t* k, const uint16_t* v) {
    int rc;
    a = WriteArgs{};
    if ((rc = fill_write_args(a, k_pool, v_pool, block_tokens, num_blocks, n_kv_heads, head_dim,
                              kv_dtype)) != NYION_OK)
        return rc;
    if (!block_table || !k || !v) return set_error(NYION_ERR_INVALID, "kv write: null argument");
    if (start_pos < 0 || n_tokens <= 0)
        return set_error(NYION_ERR_INVALID, "kv write: start_pos %d, n_tokens %d", start_pos, n_tokens);
    if (kv_dtype != NYION_KV_Q4_20B && (!aligned(k, 8) || !aligned(v, 8)))
        return set_error(NYION_ERR_INVALID, "kv write: bf16 k/v must be 8-byte aligned");
    a.tables = block_table;
    a.positions = nullptr;
    a.k16 = k;
    a.v16 = v;
    a.table_stride = (int)(((long long)start_pos + n_tokens + block_tokens - 1) / block_tokens);
    a.start_pos = start_pos;
    a.rows = n_tokens;
    a.per_seq = 0;
    // the V range check of the prefill rides on the f32 / binary16 write
    if (kv_dtype != NYION_KV_Q4_20B) a.status = device_status_word();
    return NYION_OK;
}

int kv_write_bf16_impl(void* k_pool, void* v_pool, const int32_t* block_table, int block_tokens,
                       int num_blocks, int n_kv_heads, int head_dim, int kv_dtype, int start_pos,
                       int n_tokens, const uint16_t* k, const uint16_t* v, hipStream_t stream) {
    int rc;
    WriteArgs a;
    if ((rc = prefill_write_args(a, k_pool, v_pool, block_table, block_tokens, num_blocks,
                                 n_kv_heads, head_dim, kv_dtype, start_pos, n_tokens, k, v)) !=
        NYION_OK)
        return rc;
    // a Q4 write has no V range check of its own: the check runs first
    if (kv_dtype == NYION_KV_Q4_20B &&
        (rc = v_range_check(v, (long long)n_tokens * n_kv_heads * head_dim, stream)) != NYION_OK)
        return rc;
    return launch_write(a, kv_dtype, stream);
}

}  // namespace nyion

using namespace nyion;

extern "C" {

int nyion_kv_write(void* k_pool, void* v_pool, const int32_t* block_table, int block_tokens,
                   int num_blocks, int n_kv_heads, int head_dim, int kv_dtype, int start_pos,
                   int n_tokens, const float* k, const float* v, nyion_stream_t stream) {
    clear_error();
    int rc;
    if ((rc = require_device()) != NYION_OK) return rc;
    return kv_write_impl(k_pool, v_pool, block_table, block_tokens, num_blocks, n_kv_heads,
                         head_dim, kv_dtype, start_pos, n_tokens, k, v, (hipStream_t)stream);
}

int nyion_kv_append_batch(void* k_pool, void* v_pool, const int32_t* block_tables,
                          int max_blocks_per_seq, const int32_t* positions, int batch,
                          int block_tokens, int num_blocks, int n_kv_heads, int head_dim,
                          int kv_dtype, const float* k, const float* v, nyion_stream_t stream) {
    clear_error();
    int rc;
    if ((rc = require_device()) != NYION_OK) return rc;
    WriteArgs a{};
    if ((rc = fill_write_args(a, k_pool, v_pool, block_tokens, num_blocks, n_kv_heads, head_dim,
                              kv_dtype)) != NYION_OK)
        return rc;
    if (!block_tables || !positions || !k || !v || batch <= 0 || max_blocks_per_seq <= 0)
        return set_error(NYION_ERR_INVALID, "kv append: null argument or non-positive size");
    if (kv_dtype != NYION_KV_Q4_20B && (!aligned(k, 16) || !aligned(v, 16)))
        return set_error(NYION_ERR_INVALID, "kv append: k/v must be 16-byte aligned");
    a.tables = block_tables;
    a.positions = positions;
    a.k = k;
    a.v = v;
    a.table_stride = max_blocks_per_seq;
    a.rows = batch;
    a.per_seq = 1;
    return launch_write(a, kv_dtype, (hipStream_t)stream);
}

static int kv_gather_impl(const void* pool, const int32_t* block_table, int block_tokens,
                          int num_blocks, int n_kv_heads, int head_dim, int kv_dtype,
                          int n_tokens, float* out, uint16_t* out_bf16, nyion_stream_t stream) {
    clear_error();
    int rc;
    if ((rc = require_device()) != NYION_OK) return rc;
    if (!pool || !block_table || !(out || out_bf16) || n_tokens <= 0 || n_kv_heads <= 0 ||
        num_blocks <= 0)
        return set_error(NYION_ERR_INVALID, "kv gather: null argument or non-positive size");
    if (out_bf16 && !aligned(out_bf16, 16))
        return set_error(NYION_ERR_INVALID, "kv gather: bf16 output must be 16-byte aligned");
    if (head_dim <= 0 || head_dim % 8)
        return set_error(NYION_ERR_UNSUPPORTED, "kv gather: head_dim %d not a multiple of 8",
                         head_dim);
    if (!is_pow2(block_tokens)) return set_error(NYION_ERR_INVALID, "kv gather: block_tokens");
    if (kv_dtype != NYION_KV_F32 && kv_dtype != NYION_KV_Q4_20B && kv_dtype != NYION_KV_F16)
        return set_error(NYION_ERR_INVALID, "kv gather: kv_dtype");
    if (kv_dtype == NYION_KV_F16 && !aligned(pool, 16))
        return set_error(NYION_ERR_INVALID, "kv gather: f16 pool must be 16-byte aligned");
    const long long row = kv_dtype == NYION_KV_Q4_20B ? q4_row_bytes(head_dim) : head_dim;
    GatherArgs a{};
    a.pool = pool;
    a.table = block_table;
    a.out = out;
    a.out_bf16 = out_bf16;
    a.token_stride = (int)row;
    a.head_stride = (long long)block_tokens * row;
    a.block_stride = (long long)n_kv_heads * block_tokens * row;
    a.bt_log2 = ilog2(block_tokens);
    a.num_blocks = num_blocks;
    a.n_kv_heads = n_kv_heads;
    a.head_dim = head_dim;
    a.n_tokens = n_tokens;
    a.kvt = kv_dtype;
    const long long n = (long long)n_kv_heads * n_tokens * (head_dim / 8);
    if (out_bf16)
        hipLaunchKernelGGL(kv_gather_kernel<true>, dim3(grid_for(n, 256)), dim3(256), 0,
                           (hipStream_t)stream, a);
    else
        hipLaunchKernelGGL(kv_gather_kernel<false>, dim3(grid_for(n, 256)), dim3(256), 0,
                           (hipStream_t)stream, a);
    return check_launch("kv gather");
}

int nyion_kv_gather(const void* pool, const int32_t* block_table, int block_tokens,
                    int num_blocks, int n_kv_heads, int head_dim, int kv_dtype, int n_tokens,
                    float* out, nyion_stream_t stream) {
    return kv_gather_impl(pool, block_table, block_tokens, num_blocks, n_kv_heads, head_dim,
                          kv_dtype, n_tokens, out, nullptr, stream);
}

int nyion_kv_gather_bf16(const void* pool, const int32_t* block_table, int block_tokens,
                         int num_blocks, int n_kv_heads, int head_dim, int kv_dtype, int n_tokens,
                         uint16_t* out, nyion_stream_t stream) {
    return kv_gather_impl(pool, block_table, block_tokens, num_blocks, n_kv_heads, head_dim,
                          kv_dtype, n_tokens, nullptr, out, stream);
}

int64_t nyion_zone_page_id(int64_t pos) {
    if (pos < 0) return -1;
    if (pos <= INT32_MAX) return zone_pos((int)pos).page;
    return 1120 + ((pos - kZoneStart2) >> 10);
}

int nyion_zone_page_tokens(int64_t pos) {
    if (pos < 0) return -1;
    return pos <= INT32_MAX ? 1 << zone_pos((int)pos).page_log2 : 1024;
}

int nyion_zone_kv_write(void* k_pool, void* v_pool, int64_t pool_units, const int64_t* page_base,
                        int n_pages, int n_layers, int layer, int n_kv_heads, int head_dim,
                        int kv_dtype, int start_pos, int n_tokens, const float* k, const float* v,
                        nyion_stream_t stream) {
    clear_error();
    int rc;
    if ((rc = require_device()) != NYION_OK) return rc;
    WriteArgs a{};
    if ((rc = fill_write_rows(a, k_pool, v_pool, n_kv_heads, head_dim, kv_dtype)) != NYION_OK)
        return rc;
    if ((rc = make_zone_map(a.zone, pool_units, n_pages, n_layers, layer, n_kv_heads, kv_dtype,
                            "zone kv write")) != NYION_OK)
        return rc;
    if (!page_base || !k || !v) return set_error(NYION_ERR_INVALID, "zone kv write: null argument");
    if (start_pos < 0 || n_tokens <= 0 || (long long)start_pos + n_tokens > (1LL << 31) - 1)
        return set_error(NYION_ERR_INVALID, "zone kv write: start_pos %d, n_tokens %d", start_pos,
                         n_tokens);
    if (kv_dtype != NYION_KV_Q4_20B && (!aligned(k, 16) || !aligned(v, 16)))
        return set_error(NYION_ERR_INVALID, "zone kv write: k/v must be 16-byte aligned");
    if (zone_pos(start_pos + n_tokens - 1).page >= n_pages)
        return set_error(NYION_ERR_INVALID,
                         "zone kv write: position %d is on page %d, the table has %d pages",
                         start_pos + n_tokens - 1, zone_pos(start_pos + n_tokens - 1).page, n_pages);
    a.page_bases = page_base;
    a.k = k;
    a.v = v;
    a.start_pos = start_pos;
    a.rows = n_tokens;
    a.per_seq = 0;
    return launch_write(a, kv_dtype, (hipStream_t)stream);
}

int nyion_zone_kv_gather(const void* pool, int64_t pool_units, const int64_t* page_base,
                         int n_pages, int n_layers, int layer, int n_kv_heads, int head_dim,
                         int kv_dtype, int n_tokens, float* out, nyion_stream_t stream) {
    clear_error();
    int rc;
    if ((rc = require_device()) != NYION_OK) return rc;
    if (!pool || !page_base || !out || n_tokens <= 0)
        return set_error(NYION_ERR_INVALID, "zone kv gather: null argument or non-positive size");
    if (head_dim <= 0 || head_dim % 8)
        return set_error(NYION_ERR_UNSUPPORTED, "zone kv gather: head_dim %d not a multiple of 8",
                         head_dim);
    if (kv_dtype != NYION_KV_F32 && kv_dtype != NYION_KV_Q4_20B && kv_dtype != NYION_KV_F16)
        return set_error(NYION_ERR_INVALID, "zone kv gather: kv_dtype");
    if ((kv_dtype == NYION_KV_F32 || kv_dtype == NYION_KV_F16) && !aligned(pool, 16))
        return set_error(NYION_ERR_INVALID, "zone kv gather: f32/f16 pool must be 16-byte aligned");
    if (kv_dtype == NYION_KV_Q4_20B && !aligned(pool, 4))
        return set_error(NYION_ERR_INVALID, "zone kv gather: Q4-20B pool must be 4-byte aligned");
    GatherArgs a{};
    if ((rc = make_zone_map(a.zone, pool_units, n_pages, n_layers, layer, n_kv_heads, kv_dtype,
                            "zone kv gather")) != NYION_OK)
        return rc;
    a.zone.page_base = page_base;
    a.pool = pool;
    a.out = out;
    a.token_stride = (int)(kv_dtype == NYION_KV_Q4_20B ? q4_row_bytes(head_dim) : head_dim);
    a.n_kv_heads = n_kv_heads;
    a.head_dim = head_dim;
    a.n_tokens = n_tokens;
    a.kvt = kv_dtype;
    const long long n = (long long)n_kv_heads * n_tokens * (head_dim / 8);
    hipLaunchKernelGGL(kv_gather_kernel<false>, dim3(grid_for(n, 256)), dim3(256), 0,
                       (hipStream_t)stream, a);
    return check_launch("zone kv gather");
}

int nyion_q4_dequant(const uint8_t* in, int64_t n_rows, int head_dim, float* out,
                     nyion_stream_t stream) {
    clear_error();
    int rc;
    if ((rc = require_device()) != NYION_OK) return rc;
    if (!in || !out || n_rows <= 0) return set_error(NYION_ERR_INVALID, "q4 dequant: arguments");
    if (head_dim <= 0 || head_dim % 32)
        return set_error(NYION_ERR_UNSUPPORTED, "q4 dequant: head_dim %d not a multiple of 32",
                         head_dim);
    if (!aligned(in, 4)) return set_error(NYION_ERR_INVALID, "q4 dequant: input not 4-byte aligned");
    const long long n = (long long)n_rows * (head_dim / 8);
    hipLaunchKernelGGL(q4_dequant_kernel, dim3(grid_for(n, 256)), dim3(256), 0, (hipStream_t)stream,
                       in, (long long)n_rows, head_dim, out);
    return check_launch("q4 dequant");
}

int nyion_rope_lut_init(float* d_lut, int head_dim, int max_ctx, nyion_stream_t stream) {
    clear_error();
    int rc;
    if ((rc = require_device()) != NYION_OK) return rc;
    if (!d_lut || head_dim <= 0 || head_dim % 2 || max_ctx <= 0)
        return set_error(NYION_ERR_INVALID, "rope lut: head_dim %d max_ctx %d", head_dim, max_ctx);
    const int half = head_dim / 2;
    // init_rope_lut (ops.rs:20-37) on the host with the C library's
    // powf/cosf/sinf, as the reference computes it, then one copy
    std::vector<float> lut((size_t)max_ctx * half * 2);
    for (int m = 0; m < max_ctx; m++)
        for (int k = 0; k < half; k++) {
            const float freq = 1.0f / powf(10000.0f, (float)(2 * k) / (float)head_dim);
            const float angle = (float)m * freq;
            lut[((size_t)m * half + k) * 2] = cosf(angle);
            lut[((size_t)m * half + k) * 2 + 1] = sinf(angle);
        }
    NYION_CHECK_HIP(hipMemcpyAsync(d_lut, lut.data(), lut.size() * sizeof(float),
                                   hipMemcpyHostToDevice, (hipStream_t)stream));
    NYION_CHECK_HIP(hipStreamSynchronize((hipStream_t)stream));
    return NYION_OK;
}

int nyion_rope_kv_append(float* d_q, const float* d_k, const float* d_v, const float* d_lut,
                         int max_ctx, const int32_t* positions, int batch, int n_heads,
                         int n_kv_heads, int head_dim, void* k_pool, void* v_pool,
                         const int32_t* block_tables, int max_blocks_per_seq, int block_tokens,
                         int num_blocks, int kv_dtype, nyion_stream_t stream) {
    clear_error();
    int rc;
    if ((rc = require_device()) != NYION_OK) return rc;
    RopeArgs a{};
    if ((rc = fill_write_args(a.w, k_pool, v_pool, block_tokens, num_blocks, n_kv_heads, head_dim,
                              kv_dtype)) != NYION_OK)
        return rc;
    if (!d_q || !d_k || !d_v || !d_lut || !positions || !block_tables || batch <= 0 ||
        n_heads <= 0 || max_blocks_per_seq <= 0 || max_ctx <= 0 || head_dim % 2)
        return set_error(NYION_ERR_INVALID, "rope kv append: null argument or bad size");
    if (!aligned(d_q, 8) || !aligned(d_k, 8) || !aligned(d_v, 8) || !aligned(d_lut, 8))
        return set_error(NYION_ERR_INVALID, "rope kv append: buffers must be 8-byte aligned");
    a.q = d_q;
    a.k = d_k;
    a.lut = (const float2*)d_lut;
    a.max_ctx = max_ctx;
    a.n_heads = n_heads;
    a.w.tables = block_tables;
    a.w.positions = positions;
    a.w.v = d_v;
    a.w.table_stride = max_blocks_per_seq;
    a.w.rows = batch;
    a.w.per_seq = 1;
    const long long nq = (long long)batch * n_heads * (head_dim / 2);
    const long long units = kv_dtype == NYION_KV_Q4_20B ? (head_dim + 31) / 32 : head_dim / 2;
    const long long nkv = (long long)batch * n_kv_heads * units;
    const dim3 grid(grid_for(nq + nkv, 256));
    if (kv_dtype == NYION_KV_F32)
        hipLaunchKernelGGL(rope_kv_append_kernel<NYION_KV_F32>, grid, dim3(256), 0,
                           (hipStream_t)stream, a, nq, nkv);
    else if (kv_dtype == NYION_KV_F16)
        hipLaunchKernelGGL(rope_kv_append_kernel<NYION_KV_F16>, grid, dim3(256), 0,
                           (hipStream_t)stream, a, nq, nkv);
    else
        hipLaunchKernelGGL(rope_kv_append_kernel<NYION_KV_Q4_20B>, grid, dim3(256), 0,
                           (hipStream_t)stream, a, nq, nkv);
    return check_launch("rope kv append");
}

int nyion_q4_quantize(const float* in, int64_t n_rows, int head_dim, uint8_t* out,
                      nyion_stream_t stream) {
    clear_error();
    int rc;
    if ((rc = require_device()) != NYION_OK) return rc;
    if (!in || !out || n_rows <= 0 || head_dim <= 0)
        return set_error(NYION_ERR_INVALID, "q4 quantize: arguments");
    if (!aligned(out, 4)) return set_error(NYION_ERR_INVALID, "q4 quantize: output not 4-byte aligned");
    if (head_dim % 32 == 0 && aligned(in, 16)) {
        const long long n = (long long)n_rows * (head_dim / 32) * 8;
        hipLaunchKernelGGL(q4_quantize_x8_kernel, dim3(grid_for(n, 256)), dim3(256), 0,
                           (hipStream_t)stream, in, (long long)n_rows, head_dim, out);
    } else {
        const long long n = (long long)n_rows * ((head_dim + 31) / 32);
        hipLaunchKernelGGL(q4_quantize_kernel, dim3(grid_for(n, 256)), dim3(256), 0,
                           (hipStream_t)stream, in, (long long)n_rows, head_dim, out);
    }
    return check_launch("q4 quantize");
}

}  // extern "C"
