// prefill_attention.hip — causal prefill attention on MFMA (gfx950).
//
// The reference prefills by calling ops::attention once per token with
// seq_len = abs_pos + 1 (swamp-engine/src/executor.rs:132-137, ops.rs:170-278):
// row i attends to keys [0, i].  Here one kernel computes all rows of a chunk
// as a flash-attention style pass: bf16 q, k, v in, fp32 accumulate, f32 out.
//
// Work decomposition.  A 256-thread workgroup owns one kv head and four
// (q head, 32-row block) pairs that read the same K/V: for GQA 4:1 these are
// the four q heads of the group on the same 32 rows, so every K/V tile staged
// in LDS feeds four wavefronts.  Row blocks are issued longest-first.
//
// Per 64-key tile:
//   K tile  [64][D] bf16 -> LDS, 16-byte chunks XOR-swizzled by key row
//   V tile  [64][D] bf16 -> LDS transposed to V^T [D][64] (key pairs packed
//           into 32-bit words, 8-byte chunks XOR-swizzled by dim row)
//   S^T[64 keys][32 rows] = K . Q^T      v_mfma_f32_32x32x16_bf16, Q^T from
//                                        registers (loaded once)
//   online softmax per row (rows are lanes; 32 keys per lane per half)
//   O[32 rows][D] += P . V               A = P converted in registers from
//                                        the S^T accumulators (no shuffles),
//                                        as bf16 hi + lo (two MFMAs), B = V^T
//                                        from LDS
// The next tile's global loads are issued before the current tile's MFMAs.
#include <math.h>

#include "common.hpp"

namespace nyion {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

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
    float* out;  // [N][Hq][D]
    int n;
    int n_heads;
    int n_kv_heads;
    int group;     // q heads per kv head
    int hw;        // q heads per workgroup (min(group, 4))
    int rb_per_wg; // 32-row blocks per workgroup (4 / hw)
    int n_rbg;     // row-block groups
    int causal;
    float scale_log2;
};

constexpr int BN = 64;  // keys per tile

template <int D>
struct PrefillSmem {
    // K tile: [BN][D] bf16, chunk c of key i at (c ^ (i % (D/8)))
    uint4 k[BN * D / 8];
    // V^T tile: [D][BN] bf16 as words; 8-byte chunk q of dim row r at q ^ ((r>>1)&15)
    uint32_t vt[D * BN / 2];
};

template <int D>
__device__ __forceinline__ int k_chunk_index(int key, int c) {
    return key * (D / 8) + (c ^ (key % (D / 8)));
}

// Word index of keys (4*qc + 2*half .. +1) in V^T row r.
__device__ __forceinline__ int vt_word(int r, int qc, int half) {
    return r * (BN / 2) + ((qc ^ ((r >> 1) & 15)) << 1) + half;
}

template <int D>
__global__ __launch_bounds__(256, 2) void prefill_kernel(PrefillArgs a) {
    constexpr int CPR = D / 8;              // 16-byte chunks per row
    constexpr int KLOADS = BN * CPR / 256;  // K chunks per thread per tile
    constexpr int VUNITS = (BN / 2) * (D / 8) / 256;  // (key pair, 8 dims) units per thread
    constexpr int DT = D / 32;              // output dim tiles
    constexpr int KS = D / 16;              // k-steps of the S product

    __shared__ PrefillSmem<D> sm;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int j = lane & 31;   // row (S^T col) / dim within tile (O col)
    const int h = lane >> 5;   // half

    // workgroup -> (kv head, head subset, row-block group)
    const int subsets = a.group / a.hw;
    const int rbg = a.n_rbg - 1 - (int)blockIdx.x;  // longest first
    const int g = blockIdx.y / subsets;
    const int hs = blockIdx.y - g * subsets;
    const int head = g * a.group + hs * a.hw + (wave % a.hw);
    const int row0 = (rbg * a.rb_per_wg + wave / a.hw) * 32;
    const int wg_row_end = min(a.n, (rbg + 1) * a.rb_per_wg * 32);
    const int key_end = a.causal ? wg_row_end : a.n;
    const int n_tiles = (key_end + BN - 1) / BN;

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
    float mrun = -INFINITY;
    float lrun = 0.f;

    // global -> register staging of one tile
    uint4 kst[KLOADS];
    uint4 vst[VUNITS][2];
    auto load_tile = [&](int kt) {
#pragma unroll
        for (int u = 0; u < KLOADS; u++) {
            const int id = tid + 256 * u;
            const int key = id / CPR, c = id % CPR;
            const int t = kt + key;
            kst[u] = t < a.n ? *(const uint4*)(a.k + ((long long)t * a.n_kv_heads + g) * D + 8 * c)
                             : uint4{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < VUNITS; u++) {
            const int id = tid + 256 * u;
            const int kp = id % (BN / 2), dc = id / (BN / 2);
            const int t = kt + 2 * kp;
            vst[u][0] = t < a.n ? *(const uint4*)(a.v + ((long long)t * a.n_kv_heads + g) * D + 8 * dc)
                                : uint4{0, 0, 0, 0};
            vst[u][1] = t + 1 < a.n
                            ? *(const uint4*)(a.v + ((long long)(t + 1) * a.n_kv_heads + g) * D + 8 * dc)
                            : uint4{0, 0, 0, 0};
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int u = 0; u < KLOADS; u++) {
            const int id = tid + 256 * u;
            const int key = id / CPR, c = id % CPR;
            sm.k[k_chunk_index<D>(key, c)] = kst[u];
        }
#pragma unroll
        for (int u = 0; u < VUNITS; u++) {
            const int id = tid + 256 * u;
            const int kp = id % (BN / 2), dc = id / (BN / 2);
            const uint32_t* a0 = (const uint32_t*)&vst[u][0];
            const uint32_t* a1 = (const uint32_t*)&vst[u][1];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                // dims 8dc+e: low half from key 2kp, high half from key 2kp+1
                const uint32_t lo = (e & 1) ? (a0[e >> 1] >> 16) : (a0[e >> 1] & 0xffffu);
                const uint32_t hi = (e & 1) ? (a1[e >> 1] >> 16) : (a1[e >> 1] & 0xffffu);
                const int r = 8 * dc + e;
                const int key = 2 * kp;
                sm.vt[vt_word(r, key >> 2, (key >> 1) & 1)] = lo | (hi << 16);
            }
        }
    };

    if (n_tiles > 0) load_tile(0);
    for (int it = 0; it < n_tiles; it++) {
        const int kt = it * BN;
        __syncthreads();
        store_tile();
        __syncthreads();
        if (it + 1 < n_tiles) load_tile(kt + BN);

        // S^T for the two 32-key halves of the tile
        floatx16 st[2];
#pragma unroll
        for (int kb = 0; kb < 2; kb++) {
            st[kb] = floatx16{};
            const int key = kb * 32 + j;
#pragma unroll
            for (int s = 0; s < KS; s++) {
                const bf16x8 kf = __builtin_bit_cast(bf16x8, sm.k[k_chunk_index<D>(key, 2 * s + h)]);
                st[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qreg[s], st[kb], 0, 0, 0);
            }
        }

        // scale + mask; lane holds row row0+j, keys kt + 32kb + 8(r/4) + 4h + r%4
        const int row = row0 + j;
        const bool need_mask = (kt + BN > a.n) || (a.causal && kt + BN - 1 > row0);
        float mt = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 2; kb++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                float s = st[kb][r] * a.scale_log2;
                if (need_mask) {
                    const int key = kt + 32 * kb + 8 * (r >> 2) + 4 * h + (r & 3);
                    if (key >= a.n || (a.causal && key > row)) s = -INFINITY;
                }
                st[kb][r] = s;
                mt = fmaxf(mt, s);
            }
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        // rows past the end (row >= n) see only -inf in the causal mask when
        // row0+j exceeds every key; keep their max finite
        const float mnew = fmaxf(fmaxf(mrun, mt), -1e30f);
        const float alpha = __builtin_amdgcn_exp2f(mrun - mnew);
        mrun = mnew;
        float psum = 0.f;
        // A operands of the PV product, k-step t = 2kb + half.  P is split
        // into bf16 hi + lo parts (p - hi is exact in f32), so the PV product
        // carries ~16 significant bits of p instead of 8.
        bf16x8 pa[4], pl[4];
#pragma unroll
        for (int kb = 0; kb < 2; kb++)
#pragma unroll
            for (int t2 = 0; t2 < 2; t2++) {
                bf16x8 pk, pr;
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const float p = __builtin_amdgcn_exp2f(st[kb][8 * t2 + e] - mnew);
                    psum += p;
                    const __bf16 hi = (__bf16)p;
                    pk[e] = hi;
                    pr[e] = (__bf16)(p - (float)hi);
                }
                pa[2 * kb + t2] = pk;
                pl[2 * kb + t2] = pr;
            }
        lrun = __builtin_fmaf(lrun, alpha, psum);

        // rescale O rows whose max moved (O reg r of this lane is row 8(r/4)+4h+r%4)
        if (__any(alpha != 1.0f)) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const float ar = __shfl(alpha, 8 * (r >> 2) + 4 * h + (r & 3));
#pragma unroll
                for (int t = 0; t < DT; t++) o[t][r] *= ar;
            }
        }

        // O += P . V
#pragma unroll
        for (int t = 0; t < 4; t++) {
#pragma unroll
            for (int dt = 0; dt < DT; dt++) {
                const int r = 32 * dt + j;  // V^T row (dim)
                const uint2 w0 = *(const uint2*)&sm.vt[vt_word(r, 4 * t + h, 0)];
                const uint2 w1 = *(const uint2*)&sm.vt[vt_word(r, 4 * t + 2 + h, 0)];
                const uint4 w = uint4{w0.x, w0.y, w1.x, w1.y};
                const bf16x8 vb = __builtin_bit_cast(bf16x8, w);
                o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pa[t], vb, o[dt], 0, 0, 0);
                o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pl[t], vb, o[dt], 0, 0, 0);
            }
        }
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
}

}  // namespace nyion

using namespace nyion;

extern "C" int nyion_prefill_attention_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                            int n, int n_heads, int n_kv_heads, int head_dim,
                                            int causal, float scale, float* out, void* k_pool,
                                            void* v_pool, const int32_t* block_table,
                                            int block_tokens, int num_blocks, int kv_dtype,
                                            int start_pos, nyion_stream_t stream) {
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
    const int group = n_heads / n_kv_heads;
    const int hw = group < 4 ? group : 4;
    if (4 % hw || group % hw)
        return set_error(NYION_ERR_UNSUPPORTED, "prefill: GQA group %d (need 1, 2 or a multiple of 4)",
                         group);
    PrefillArgs a{};
    a.q = q;
    a.k = k;
    a.v = v;
    a.out = out;
    a.n = n;
    a.n_heads = n_heads;
    a.n_kv_heads = n_kv_heads;
    a.group = group;
    a.hw = hw;
    a.rb_per_wg = 4 / hw;
    const int rows_per_wg = 32 * a.rb_per_wg;
    a.n_rbg = (n + rows_per_wg - 1) / rows_per_wg;
    a.causal = causal ? 1 : 0;
    const float sc = scale > 0.f ? scale : 1.0f / sqrtf((float)head_dim);
    a.scale_log2 = sc * 1.4426950408889634f;
    if ((long long)n_kv_heads * (group / hw) > 65535)
        return set_error(NYION_ERR_UNSUPPORTED, "prefill: too many heads");
    dim3 grid(a.n_rbg, n_kv_heads * (group / hw));
    hipStream_t st = (hipStream_t)stream;
    if (head_dim == 128)
        hipLaunchKernelGGL(prefill_kernel<128>, grid, dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL(prefill_kernel<64>, grid, dim3(256), 0, st, a);
    if ((rc = check_launch("prefill")) != NYION_OK) return rc;
    if (k_pool || v_pool) {
        if (!k_pool || !v_pool || !block_table)
            return set_error(NYION_ERR_INVALID, "prefill: KV write needs k_pool, v_pool and block_table");
        return kv_write_bf16_impl(k_pool, v_pool, block_table, block_tokens, num_blocks, n_kv_heads,
                                  head_dim, kv_dtype, start_pos, n, k, v, st);
    }
    return NYION_OK;
}
