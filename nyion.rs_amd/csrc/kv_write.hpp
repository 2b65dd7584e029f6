// kv_write.hpp — the paged KV write's arguments and per-row device code,
// shared by the write kernels (kv_cache.hip) and the prefill kernel, which
// writes its chunk's K/V rows itself (prefill_attention.hip).
#pragma once

#include "common.hpp"

namespace nyion {

struct WriteArgs {
    void* k_pool;
    void* v_pool;
    const int32_t* tables;  // [batch][table_stride]
    const int32_t* positions;  // per-sequence position (append) or nullptr
    const float* k;  // [rows][Hkv][D] f32, or nullptr when the bf16 source is used
    const float* v;
    const uint16_t* k16;  // [rows][Hkv][D] bf16 bits (prefill path)
    const uint16_t* v16;
    int table_stride;
    int start_pos;  // used when positions == nullptr
    int rows;       // tokens (single sequence) or sequences (append)
    int per_seq;    // 1: row r is sequence r at positions[r]; 0: row r is token start_pos+r of seq 0
    int n_kv_heads;
    int head_dim;
    int bt_log2;
    int num_blocks;
    long long block_stride;  // row units
    long long head_stride;
    int token_stride;
    unsigned* status;  // bf16 source: the device's range-status word (V beyond binary16)
    // zone geometry: sequence s's page offsets at page_bases + s * zone.n_pages
    // (tables unused); nullptr: block tables
    const int64_t* page_bases;
    ZoneMap zone;
};

// bf16 -> f32 is exact (the bf16 bits are the high half of the f32).
__device__ __forceinline__ float4 bf16x4_to_f32(uint2 w) {
    return float4{__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u),
                  __uint_as_float(w.y << 16), __uint_as_float(w.y & 0xffff0000u)};
}

__device__ __forceinline__ long long write_row_offset(const WriteArgs& a, int r, int h) {
    const int seq = a.per_seq ? r : 0;
    const int pos = a.per_seq ? a.positions[r] : a.start_pos + r;
    if (pos < 0) return -1;
    RowMap m;
    m.table = a.tables + (long long)seq * a.table_stride;
    m.block_stride = a.block_stride;
    m.head_stride = a.head_stride;
    m.token_stride = a.token_stride;
    m.bt_log2 = a.bt_log2;
    m.num_blocks = a.num_blocks;
    m.table_len = a.table_stride;
    m.zone = a.zone;
    m.zone.page_base = a.page_bases ? a.page_bases + (long long)seq * a.zone.n_pages : nullptr;
    return row_offset(m, pos, h);
}

typedef _Float16 halfx2_t __attribute__((ext_vector_type(2)));

// Two f32 -> one word of two binary16 (round to nearest even), lo first.
__device__ __forceinline__ uint32_t f16x2_bits(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, halfx2_t{(_Float16)lo, (_Float16)hi});
}

// Largest |v| of four bf16 values (the bits of two words).
__device__ __forceinline__ float v_absmax(uint2 w) {
    const float a = __uint_as_float(w.x << 16), b = __uint_as_float(w.x & 0xffff0000u);
    const float c = __uint_as_float(w.y << 16), d = __uint_as_float(w.y & 0xffff0000u);
    return fmaxf(fmaxf(fabsf(a), fabsf(b)), fmaxf(fabsf(c), fabsf(d)));
}

// One (row r, kv head h, four values x) of a f32 or binary16 (F16) pool
// write from f32 or bf16 rows; returns the largest |v| of the four bf16 V
// values (0 for an f32 source) for the prefill's V range check.
template <bool F16>
__device__ __forceinline__ float write_kv_vec(const WriteArgs& a, int r, int h, int x) {
    const long long src = ((long long)r * a.n_kv_heads + h) * a.head_dim + 4 * x;
    float4 kk, vv;
    float vmax = 0.f;
    if (a.k16) {
        const uint2 vw = *(const uint2*)(a.v16 + src);
        vmax = v_absmax(vw);
        kk = bf16x4_to_f32(*(const uint2*)(a.k16 + src));
        vv = bf16x4_to_f32(vw);
    } else {
        kk = *(const float4*)(a.k + src);
        vv = *(const float4*)(a.v + src);
    }
    const long long off = write_row_offset(a, r, h);
    if (off < 0) return vmax;
    if (F16) {
        *(uint2*)((uint16_t*)a.k_pool + off + 4 * x) = uint2{f16x2_bits(kk.x, kk.y), f16x2_bits(kk.z, kk.w)};
        *(uint2*)((uint16_t*)a.v_pool + off + 4 * x) = uint2{f16x2_bits(vv.x, vv.y), f16x2_bits(vv.z, vv.w)};
    } else {
        *(float4*)((float*)a.k_pool + off + 4 * x) = kk;
        *(float4*)((float*)a.v_pool + off + 4 * x) = vv;
    }
    return vmax;
}

// Host: the write arguments of a prefill chunk's bf16 K/V rows into f32 or
// binary16 pools, validated (kv_cache.hip).
int prefill_write_args(WriteArgs& a, void* k_pool, void* v_pool, const int32_t* block_table,
                       int block_tokens, int num_blocks, int n_kv_heads, int head_dim, int kv_dtype,
                       int start_pos, int n_tokens, const uint16_t* k, const uint16_t* v);

}  // namespace nyion
