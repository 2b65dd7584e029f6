/*
 * nyion_oracle.h — CPU restatement of the Nyion attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the reference result the HIP
 * path is compared against, and the scalar/OpenMP CPU baseline that bench.py
 * times beside the GPU.  Nothing in the product library (libnyion_hip.so)
 * links, loads or calls it; only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may.
 *
 * Every function cites the reference file:line it restates (paths relative
 * to the reference repository root).
 *
 * Pinning status (what each function is checked against; see tests/):
 *   orc_dot_avx512_order / orc_weighted_sum  : reference KATs simd.rs:190-229
 *   orc_f32_to_f16 / orc_f16_to_f32          : numpy float16 (IEEE binary16
 *                                              RNE) on every f16 bit pattern
 *   orc_q4_quantize_row / orc_q4_dequant_row : reference round-trip tests
 *                                              cache.rs:853-926,1031-1068 +
 *                                              invariants + numpy restatement
 *   orc_zone_*                               : golden page ids cache.rs:1000-1029
 *   orc_attention / _positions / _rows       : float64 brute force + closed
 *                                              forms (seq_len 1, equal keys,
 *                                              one-hot gap), importance sum
 *   orc_sparse_positions / orc_fugu_positions: hand-enumerated golden lists
 *   orc_softmax_padic / orc_exp_q16_16       : reference tests
 *                                              swamp-kernels/src/lib.rs:629-684
 *                                              + integer pipeline by hand
 *   orc_stokes_*                             : eviction-by-construction
 *   orc_rope_lut / orc_apply_rope            : float64 cos/sin of the same
 *                                              angles within f32 rounding,
 *                                              pos 0 identity, rotation
 *                                              preserves pair norms
 *   orc_q4k_unpack_scales / _dequant_block   : the reference's own block
 *                                              builder (fused_gemv_q4k.rs:812-
 *                                              828) round-tripped, and a numpy
 *                                              restatement of the 12-byte packing
 *   orc_gemv_q4k                             : closed form of the reference test
 *                                              weights (constant nibble 8,
 *                                              fused_gemv_q4k.rs:830-845) and
 *                                              float64 dequantise-then-dot
 *   orc_q6k_scale_to_f32                     : IEEE binary16 on normal values
 *                                              (numpy), the reference's own bit
 *                                              formula on exponents 0 and 31
 *   orc_q6k_dequant_block / orc_gemv_q6k     : single-element probes of the
 *                                              bit layout, the reference test
 *                                              blocks (fused_gemv_q6k.rs:329-
 *                                              356), a numpy restatement and
 *                                              float64 dequantise-then-dot
 *   orc_attention_positions importance       : equals orc_attention's over the
 *                                              full position set; float64 brute
 *                                              force; sums to n_heads
 *   orc_q4_a5_row / orc_attention_sparse_q4  : hand-built groups whose A5 order
 *                                              and writer order differ (one-hot
 *                                              q, single-position V read back),
 *                                              the 1e-8 skip on a zero row,
 *                                              float64 brute force on a tiny
 *                                              shape
 *   orc_mojo_sparse_attention_q4             : one tile (<= 64 positions) equals
 *                                              orc_attention_positions on the
 *                                              dequantised rows; equal scores
 *                                              over two tiles give the closed
 *                                              form sum(v1)/64 + sum(v2)/128 of
 *                                              the per-tile normalisation; a
 *                                              weight below 1e-8 adds nothing
 * Bit-parity of attention outputs with the Rust binary (glibc expf order,
 * rayon scheduling of the importance sum) is unpinned and not required:
 * attention parity is at tolerance.
 */
#ifndef NYION_ORACLE_H
#define NYION_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_KV_F32 = 0, ORC_KV_Q4 = 1, ORC_KV_F16 = 2 };

/* Row addressing shared by every attention restatement.
 * Row of token t, kv head h:
 *   base + table[t / block_tokens] * block_stride + h * head_stride
 *        + (t % block_tokens) * token_stride
 * Strides are in f32 elements for ORC_KV_F32, binary16 elements for
 * ORC_KV_F16 (rows widened exactly to f32 before use) and bytes for ORC_KV_Q4.
 * table == NULL means block id 0 for every token (contiguous layouts use a
 * block_tokens larger than any position). */
typedef struct orc_kv_layout {
    const void*    k_base;
    const void*    v_base;
    const int32_t* table;
    int64_t        block_tokens;
    int64_t        block_stride;
    int64_t        head_stride;
    int64_t        token_stride;
    int32_t        dtype;
    int32_t        _pad;
} orc_kv_layout;

/* simd.rs primitives */
float orc_dot_avx512_order(const float* a, const float* b, int n);
void  orc_weighted_sum(float* out, const float* v, float score, int n);

/* IEEE binary16 conversions (what `half` 2.7.1 implements) */
uint16_t orc_f32_to_f16(float f);
float    orc_f16_to_f32(uint16_t h);

/* Q4-20B codec: ceil(d/32) groups of 20 bytes per row */
int  orc_q4_row_bytes(int head_dim);
void orc_q4_quantize_row(const float* x, int head_dim, uint8_t* out);
void orc_q4_dequant_row(const uint8_t* in, int head_dim, float* out);
void orc_q4_quantize_rows(const float* x, int64_t n_rows, int head_dim, uint8_t* out);
void orc_q4_dequant_rows(const uint8_t* in, int64_t n_rows, int head_dim, float* out);

/* PagedKVCache zone arithmetic (cache.rs:17-21,185-237,593-611) */
int64_t orc_zone_index(int64_t pos);
int64_t orc_zone_block_size(int64_t pos);
int64_t orc_zone_page_id(int64_t pos, int64_t max_seq_len);
int64_t orc_zone_slot_in_page(int64_t pos);
int64_t orc_zone_page_start(int64_t pos);
int64_t orc_zone_total_pages(int64_t max_seq_len);
int64_t orc_zone_f32_offset(int64_t layer, int64_t kv_head, int64_t pos,
                            int64_t n_kv_heads, int64_t head_dim);
int64_t orc_zone_q4_offset(int64_t layer, int64_t kv_head, int64_t pos,
                           int64_t n_kv_heads, int64_t head_dim);

/* Position sets */
int orc_sparse_positions(int seq_len, int q_pos, int window, int global_stride,
                         int32_t* out, int cap);
int orc_fugu_positions(int seq_len, int q_pos, int window, int sentinel_stride,
                       const int32_t* dspark, int n_dspark, int32_t* out, int cap);

/* Attention restatements. Return 0 on success, <0 on bad arguments. */
int orc_attention(float* out, const float* q, const orc_kv_layout* kv,
                  int seq_len, int q_pos, int n_heads, int n_kv_heads,
                  int head_dim, double* importance, int nthreads);
/* importance (nullable): importance[i] += sum over heads of the probability
 * of positions[i] (f64, heads in order). */
int orc_attention_positions(float* out, const float* q, const orc_kv_layout* kv,
                            const int32_t* positions, int n_pos, int n_heads,
                            int n_kv_heads, int head_dim, double* importance,
                            int nthreads);
/* One causal attention per listed query row r: q row r, keys [0, r]. */
int orc_attention_rows(float* out, const float* q, int64_t q_row_stride,
                       int64_t out_row_stride, const orc_kv_layout* kv,
                       const int32_t* rows, int n_rows, int n_heads,
                       int n_kv_heads, int head_dim, int nthreads);

/* RoPE: init_rope_lut (swamp-engine/src/ops.rs:20-37) into lut
 * [max_ctx][head_dim/2][2], and apply_rope_ufc (ops.rs:40-79) on one
 * token's q [n_heads][D] and k [n_kv_heads][D] in place. */
void orc_rope_lut(int head_dim, int max_ctx, float* lut);
void orc_apply_rope(float* q, float* k, int pos, int n_heads, int n_kv_heads, int head_dim,
                    int max_ctx, const float* lut);

/* swamp-kernels C-ABI restatements */
int32_t orc_exp_q16_16(int32_t x_fixed);
void    orc_softmax_padic(const float* logits, float* probs, int n, float temperature);

void* orc_stokes_init(int head_dim);
int   orc_stokes_append(void* cache, int token_id, const float* key,
                        const float* value, float score);
void  orc_stokes_free(void* cache);
int   orc_stokes_count(const void* cache);
int   orc_stokes_read(const void* cache, float* keys, float* values, float* scores);

/* Q4_K weights (GGUF 144-byte blocks of 256: f16 d, f16 dmin, 12 bytes of
 * 6-bit scales/mins, 128 bytes of nibbles) and the scalar GEMV of
 * swamp-kernels/src/fused_gemv_q4k.rs */
void orc_q4k_unpack_scales(const uint8_t* sc, uint8_t* scales, uint8_t* mins);
void orc_q4k_dequant_block(const uint8_t* blk, float* out);
int  orc_gemv_q4k(const uint8_t* w, const float* x, float* out, int n_rows, int n_cols);

/* Q6_K weights (210-byte blocks of 256: ql[128], qh[64], int8 scales[16],
 * f16 d) and the scalar GEMV of swamp-kernels/src/fused_gemv_q6k.rs */
float orc_q6k_scale_to_f32(uint16_t v);
void  orc_q6k_dequant_block(const uint8_t* blk, float* out);
int   orc_gemv_q6k(const uint8_t* w, const float* x, float* out, int n_rows, int n_cols);

/* sparse_attention_q4 of the Mojo kernel library (swamp-gpu/kernels/
 * attention.mojo:38-152, loaded through swamp-gpu/src/mojo.rs:5,38): every
 * head against one K/V of f32-word Q4 rows, tiles of 64 listed positions,
 * each tile's weights normalised by the running denominator of the tiles so
 * far. */
void  orc_mojo_sparse_attention_q4(const float* q, const float* k_q4, const float* v_q4,
                                   const int32_t* positions, float* out, int n_heads,
                                   int head_dim, int n_sparse);

/* attention_sparse_q4 (swamp-engine/src/ops.rs:597-723) over Q4-20B rows
 * addressed by kv (dtype ORC_KV_Q4): attention_sparse's position set, the
 * rows read with that function's nibble order (low nibbles elements 0-15,
 * high nibbles 16-31 of each group) and fma(d, nibble, dmin), weights below
 * 1e-8 skipped.  orc_q4_a5_row is that row decode alone. */
void orc_q4_a5_row(const uint8_t* in, int head_dim, float* out);
int  orc_sparse_q4_positions(int seq_len, int q_pos, int window, int global_stride,
                             int32_t* out, int cap);
int  orc_attention_sparse_q4(float* out, const float* q, const orc_kv_layout* kv,
                             int seq_len, int q_pos, int n_heads, int n_kv_heads,
                             int head_dim, int window, int global_stride, int nthreads);

int orc_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
