// common.hpp — shared host/device helpers of libnyion_hip.so (gfx950 only).
//
// The Q4-20B unpack and the paged row addressing here are used by the decode
// kernels, the KV-write kernels and the debug gather/dequant kernels alike,
// so the debug entry points validate exactly the code the hot path runs.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <string>

#include "../../include/nyion_hip.h"
#include "host_status.hpp"

namespace nyion {

// ------------------------------------------------------------ errors

#define NYION_CHECK_HIP(expr)                                                                \
    do {                                                                                     \
        hipError_t e_ = (expr);                                                              \
        if (e_ != hipSuccess)                                                                \
            return ::nyion::set_error(NYION_ERR_LAUNCH, "%s: %s (%s:%d)", #expr,             \
                                      hipGetErrorString(e_), __FILE__, __LINE__);            \
    } while (0)

// Launch-error check after a <<<>>> launch.
int check_launch(const char* what);

// True when the current device is a gfx950 (cached per device).
int require_device();

// ------------------------------------------------------------ per device

constexpr int kMaxDevices = 64;

// The current HIP device, or -1 (no device, or an id beyond kMaxDevices).
int current_device();

// A value computed once per device by `make` (an int > 0; `fallback` when
// there is no device or `make` fails).  Concurrent first calls on one device
// may both compute it; they store the same value.
template <typename F>
int per_device_value(std::atomic<int>* cache, F make, int fallback) {
    const int dev = current_device();
    if (dev < 0) return fallback;
    int v = cache[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
    v = make();
    if (v <= 0) return fallback;
    cache[dev].store(v, std::memory_order_relaxed);
    return v;
}

// Compute units of the current device (256 without one).
int device_cu_count();

// Range-status word of the current device: kernels OR a kRange* bit into it
// when an input lies outside what a reduced-precision operand can hold;
// nyion_take_status reads and clears it.  nullptr when there is no device.
enum : unsigned { kRangePrefillV = 1u, kRangeDecodeQ = 2u };
unsigned* device_status_word();

// Records in the status word whether some of the n bf16 values of v reaches
// 65520 in magnitude (one launch on `stream`; n a multiple of 4, v 8-byte
// aligned).
int v_range_check(const uint16_t* v, long long n, hipStream_t stream);

// Device address of the no-allocation decode's scratch array on the current
// device (looked up once per device; nullptr with the error set on failure).
void* decode_scratch_ptr();

// Fills the current device's exp_q16_16 table of mojo_softmax_padic (once per
// device).
int softmax_padic_setup();

// Sets `bit` in the status word from one lane when any lane of the
// wavefront has `bad` (vector atomic on global memory).
__device__ __forceinline__ void report_range(unsigned* status, bool bad, unsigned bit) {
    const unsigned long long any = __ballot(bad);
    if (any && status && (threadIdx.x & 63) == (unsigned)__builtin_ctzll(any))
        __hip_atomic_fetch_or(status, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Split-K partials cross workgroups that may sit on different XCDs, whose
// L2s are not coherent with each other: they are stored and loaded with the
// sc1 cache policy (what agent-scope relaxed atomic loads and stores carry on
// this target) through buffer instructions, 16 bytes per instruction.
constexpr int kSc1 = 16;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t partial_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)bytes, 0x00020000);
}

// Wavefront max / sum through DPP row operations, a fixed tree (the result
// does not depend on timing): lane pairs, quads, half rows, rows, then the
// rows combined through row broadcasts; returns lane 63's result, which is
// the whole wavefront's, to every lane.  No LDS traffic.
template <bool MAX, int CTRL, int ROW_MASK>
__device__ __forceinline__ float wave_dpp_step(float x) {
    const float id = MAX ? -INFINITY : 0.0f;
    const float y = __int_as_float(
        __builtin_amdgcn_update_dpp(__float_as_int(id), __float_as_int(x), CTRL, ROW_MASK, 0xf, false));
    return MAX ? fmaxf(x, y) : x + y;
}

template <bool MAX>
__device__ __forceinline__ float wave_reduce_dpp(float x) {
    x = wave_dpp_step<MAX, 0xb1, 0xf>(x);   // quad_perm [1,0,3,2]
    x = wave_dpp_step<MAX, 0x4e, 0xf>(x);   // quad_perm [2,3,0,1]
    x = wave_dpp_step<MAX, 0x141, 0xf>(x);  // row_half_mirror
    x = wave_dpp_step<MAX, 0x140, 0xf>(x);  // row_mirror: each row's lanes hold the row's value
    x = wave_dpp_step<MAX, 0x142, 0xa>(x);  // row_bcast:15 into rows 1 and 3
    x = wave_dpp_step<MAX, 0x143, 0xc>(x);  // row_bcast:31 into rows 2 and 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 63));
}

static inline bool is_pow2(long long x) { return x > 0 && (x & (x - 1)) == 0; }
static inline int ilog2(long long x) {
    int r = 0;
    while ((1ll << r) < x) r++;
    return r;
}
static inline bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

// ------------------------------------------------------------ Q4-20B

constexpr int kQ4GroupBytes = 20;  // f16 d, f16 dmin, 16 nibble bytes
constexpr int kQ4GroupElems = 32;

__host__ __device__ constexpr int q4_row_bytes(int head_dim) {
    return ((head_dim + 31) / 32) * kQ4GroupBytes;
}

// f16 bits -> f32 (exact).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(h & 0xffffu));
}

// Dequantise one nibble exactly as dequant_block (swamp-engine/src/cache.rs:
// 385-392): f32(d) * (f32)nib + f32(dmin), two separately rounded operations.
__device__ __forceinline__ float q4_dequant(float d, float dmin, uint32_t nib) {
    return __fadd_rn(__fmul_rn(d, (float)nib), dmin);
}

// Dequantise 8 consecutive elements whose nibbles are the 4 bytes of `w`
// (element 2i in the low nibble of byte i, 2i+1 in its high nibble).
__device__ __forceinline__ void q4_dequant8(uint32_t w, float d, float dmin, float* out) {
    const uint32_t lo = w & 0x0f0f0f0fu;
    const uint32_t hi = (w >> 4) & 0x0f0f0f0fu;
    out[0] = q4_dequant(d, dmin, lo & 0xffu);
    out[1] = q4_dequant(d, dmin, hi & 0xffu);
    out[2] = q4_dequant(d, dmin, (lo >> 8) & 0xffu);
    out[3] = q4_dequant(d, dmin, (hi >> 8) & 0xffu);
    out[4] = q4_dequant(d, dmin, (lo >> 16) & 0xffu);
    out[5] = q4_dequant(d, dmin, (hi >> 16) & 0xffu);
    out[6] = q4_dequant(d, dmin, lo >> 24);
    out[7] = q4_dequant(d, dmin, hi >> 24);
}

// Dequantise 4 consecutive elements from the 2 bytes in the low half of `w`.
__device__ __forceinline__ void q4_dequant4(uint32_t w, float d, float dmin, float* out) {
    out[0] = q4_dequant(d, dmin, w & 0xfu);
    out[1] = q4_dequant(d, dmin, (w >> 4) & 0xfu);
    out[2] = q4_dequant(d, dmin, (w >> 8) & 0xfu);
    out[3] = q4_dequant(d, dmin, (w >> 12) & 0xfu);
}

// ------------------------------------------------------------ zone pages

// PagedKVCache's zone geometry (swamp-engine/src/cache.rs:20-21 zone starts
// and page sizes, 185-237 flat page ids, 593-611 page_id / slot_in_page):
// positions [0, 4096) in 32-token pages, [4096, 131072) in 128-token pages,
// [131072, ...) in 1024-token pages; flat page id = the zone's first page
// (0, 128, 1120: the pages of the zones before it) + (pos - zone start) /
// page tokens.  A page holds every layer: row (layer, kv head, slot) sits at
// ((layer * n_kv_heads + kv_head) * page_tokens + slot) rows from the page's
// start (cache.rs:700-712 f32, 728-736 Q4-20B).
constexpr int kZoneStart1 = 4096, kZoneStart2 = 131072;

struct ZonePos {
    int page;       // flat page id
    int slot;       // row within the page's (layer, kv head) block
    int page_log2;  // log2(page tokens)
};

__host__ __device__ __forceinline__ ZonePos zone_pos(int t) {
    ZonePos z;
    if (t < kZoneStart1) {
        z.page_log2 = 5;
        z.page = t >> 5;
        z.slot = t & 31;
    } else if (t < kZoneStart2) {
        z.page_log2 = 7;
        z.page = 128 + ((t - kZoneStart1) >> 7);
        z.slot = (t - kZoneStart1) & 127;
    } else {
        z.page_log2 = 10;
        z.page = 1120 + ((t - kZoneStart2) >> 10);
        z.slot = (t - kZoneStart2) & 1023;
    }
    return z;
}

// One sequence's zone pages.  Offsets and sizes are in row units (f32 or
// binary16 elements, bytes for Q4-20B).
struct ZoneMap {
    const int64_t* page_base;  // offset of each flat page in the pool, < 0 absent;
                               // nullptr: block-table geometry
    int n_pages;               // entries of page_base
    int layer_rows;            // layer * n_kv_heads
    int slot_rows;             // n_layers * n_kv_heads: rows per page slot
    int align;                 // offsets must be multiples of this
    long long pool_units;      // size of each pool
};

// Validates the host-side description of a zone pool and fills `z` (its
// page_base left null: each kernel sets its sequence's).  The offset
// alignment keeps every row on the boundary its loads and stores need:
// 16 bytes for f32 and binary16 rows, 4 bytes for Q4-20B rows.
static inline int make_zone_map(ZoneMap& z, long long pool_units, int n_pages, int n_layers,
                                int layer, int n_kv_heads, int kv_dtype, const char* what) {
    if (pool_units <= 0 || n_pages <= 0 || n_layers <= 0 || n_kv_heads <= 0)
        return set_error(NYION_ERR_INVALID, "%s: pool_units, n_pages, n_layers, n_kv_heads must be positive",
                         what);
    if (layer < 0 || layer >= n_layers)
        return set_error(NYION_ERR_INVALID, "%s: layer %d outside [0, %d)", what, layer, n_layers);
    if ((long long)n_layers * n_kv_heads > (1 << 20))
        return set_error(NYION_ERR_UNSUPPORTED, "%s: n_layers * n_kv_heads %lld", what,
                         (long long)n_layers * n_kv_heads);
    z.page_base = nullptr;
    z.n_pages = n_pages;
    z.layer_rows = layer * n_kv_heads;
    z.slot_rows = n_layers * n_kv_heads;
    z.align = kv_dtype == NYION_KV_F16 ? 8 : 4;
    z.pool_units = pool_units;
    return NYION_OK;
}

// Offset of row (t, h), or -1 when its page is past the table, absent,
// misaligned or not inside the pool.
__device__ __forceinline__ long long zone_row_offset(const ZoneMap& z, int t, int h, int row) {
    const ZonePos p = zone_pos(t);
    if (p.page >= z.n_pages) return -1;
    const long long base = z.page_base[p.page];
    const long long page_units = ((long long)z.slot_rows << p.page_log2) * row;
    if (base < 0 || base % z.align || base > z.pool_units - page_units) return -1;
    return base + ((((long long)(z.layer_rows + h)) << p.page_log2) + p.slot) * row;
}

// ------------------------------------------------------------ paged rows

// Where row (token t, kv head h) of one sequence lives.  Strides are in
// units of the row element (f32 elements, or bytes for Q4).
struct RowMap {
    const int32_t* table;  // this sequence's block table, or nullptr (block 0)
    long long block_stride;
    long long head_stride;
    int token_stride;
    int bt_log2;   // log2(block_tokens)
    int num_blocks;
    int table_len;  // entries in this sequence's table
    ZoneMap zone;   // zone.page_base set: zone geometry instead of the table
};

// Offset of the row, or -1 when the token is past the table or its block id
// is out of [0, num_blocks) (zone geometry: zone_row_offset's rules).
__device__ __forceinline__ long long row_offset(const RowMap& m, int t, int h) {
    if (m.zone.page_base) return zone_row_offset(m.zone, t, h, m.token_stride);
    int blk = 0;
    if (m.table) {
        if ((t >> m.bt_log2) >= m.table_len) return -1;
        blk = m.table[t >> m.bt_log2];
        if ((unsigned)blk >= (unsigned)m.num_blocks) return -1;
    }
    return (long long)blk * m.block_stride + (long long)h * m.head_stride +
           (long long)(t & ((1 << m.bt_log2) - 1)) * m.token_stride;
}

}  // namespace nyion
