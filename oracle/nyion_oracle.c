/*
 * nyion_oracle.c — CPU restatement of the Nyion attention path.
 *
 * TEST INFRASTRUCTURE ONLY (the tests' reference results and the CPU
 * baseline).  The product
 * library never links or calls this file.  Build: oracle/Makefile, which
 * compiles with -ffp-contract=off so that every multiply-then-add written
 * below stays two roundings, exactly as the Rust source (no contraction)
 * does; fused operations are spelled fmaf() where the reference uses an FMA
 * intrinsic.
 *
 * Citations are reference file:line (repository-relative).
 */
#include "nyion_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#if defined(__x86_64__) && defined(__GNUC__) && !defined(__clang__)
#define ORC_CLONES __attribute__((target_clones("arch=skylake-avx512", "arch=haswell", "default")))
#else
#define ORC_CLONES
#endif

int orc_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------------
 * simd.rs primitives
 * --------------------------------------------------------------------- */

/* dot_product_avx512 (swamp-kernels/src/simd.rs:35-68): 16 FMA lanes over
 * full 16-chunks, one 8-wide FMA into lanes 0-7 (the reference widens a
 * 256-bit load with _mm512_castps256_ps512, whose upper half is undefined;
 * it is taken as zero here), a scalar mul+add tail, then the reduction tree
 * (lanes 0-3 + 4-7) + (8-11 + 12-15), two horizontal adds, plus the tail. */
static inline float dot16(const float* a, const float* b, int n) {
    float acc[16];
    for (int l = 0; l < 16; l++) acc[l] = 0.0f;
    int i = 0;
    for (; i + 16 <= n; i += 16)
        for (int l = 0; l < 16; l++) acc[l] = fmaf(a[i + l], b[i + l], acc[l]);
    if (i + 8 <= n) {
        for (int l = 0; l < 8; l++) acc[l] = fmaf(a[i + l], b[i + l], acc[l]);
        i += 8;
    }
    float tail = 0.0f;
    for (; i < n; i++) tail = tail + a[i] * b[i];
    float s[4];
    for (int l = 0; l < 4; l++) {
        float s1 = acc[l] + acc[4 + l];
        float s2 = acc[8 + l] + acc[12 + l];
        s[l] = s1 + s2;
    }
    float h0 = s[0] + s[1];
    float h1 = s[2] + s[3];
    return (h0 + h1) + tail;
}

/* weighted_sum_avx512 (simd.rs:106-121): out = fma(score, v, out) over
 * 16-chunks, scalar out += score*v tail. */
static inline void axpy16(float* out, const float* v, float score, int n) {
    int i = 0;
    for (; i + 16 <= n; i += 16)
        for (int l = 0; l < 16; l++) out[i + l] = fmaf(score, v[i + l], out[i + l]);
    for (; i < n; i++) out[i] = out[i] + score * v[i];
}

float orc_dot_avx512_order(const float* a, const float* b, int n) { return dot16(a, b, n); }
void orc_weighted_sum(float* out, const float* v, float score, int n) { axpy16(out, v, score, n); }

/* ------------------------------------------------------------------------
 * IEEE binary16 (the `half` 2.7.1 crate's f16::from_f32 / to_f32, used at
 * cache.rs:376-383,651-652).  Round-to-nearest-even, overflow to infinity,
 * gradual underflow; NaN stays NaN with the quiet bit set.
 * --------------------------------------------------------------------- */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ex = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (ex == 0xffu) {
        if (man == 0) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7c00u | 0x200u | (man >> 13));
    }
    int e = (int)ex - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t m = man | 0x800000u;
        int shift = 14 - e; /* 14..24 */
        uint32_t hm = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (hm & 1u))) hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t hm = man >> 13;
    uint32_t rem = man & 0x1fffu;
    uint32_t h = sign | ((uint32_t)e << 10) | hm;
    if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) h++;
    return (uint16_t)h;
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t ex = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (ex == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            float v = ldexpf((float)man, -24);
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (ex == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((ex - 15u + 127u) << 23) | (man << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

/* ------------------------------------------------------------------------
 * Q4-20B codec
 * Quantise: PagedKVCache::save / save_at (cache.rs:637-663, 771-806).
 *   per 32-element group: d = max|x|/7 (0 when max|x| <= 1e-10),
 *   dmin = min x, both f32, stored as f16 LE at bytes [0,2) and [2,4);
 *   q_i = clamp(round_half_away((x_i - dmin)/d), 0, 15) with the f32 d, dmin;
 *   element i -> byte 4 + i/2, low nibble if i even.
 *   f32::max/min skip NaN, as fmaxf/fminf do.
 * Dequantise: dequant_block (cache.rs:375-394): f32(d)*nib + f32(dmin),
 *   a separate multiply and add.
 * --------------------------------------------------------------------- */
int orc_q4_row_bytes(int head_dim) { return ((head_dim + 31) / 32) * 20; }

void orc_q4_quantize_row(const float* x, int head_dim, uint8_t* out) {
    int groups = (head_dim + 31) / 32;
    for (int g = 0; g < groups; g++) {
        int start = g * 32;
        int end = start + 32 < head_dim ? start + 32 : head_dim;
        int len = end - start;
        uint8_t* blk = out + g * 20;
        float mx = 0.0f, mn = FLT_MAX;
        for (int i = 0; i < len; i++) {
            mx = fmaxf(mx, fabsf(x[start + i]));
            mn = fminf(mn, x[start + i]);
        }
        float d = (mx > 1e-10f) ? mx / 7.0f : 0.0f;
        float dmin = mn;
        uint16_t dh = orc_f32_to_f16(d), mh = orc_f32_to_f16(dmin);
        blk[0] = (uint8_t)(dh & 0xff);
        blk[1] = (uint8_t)(dh >> 8);
        blk[2] = (uint8_t)(mh & 0xff);
        blk[3] = (uint8_t)(mh >> 8);
        memset(blk + 4, 0, 16);
        for (int i = 0; i < len; i++) {
            uint8_t q = 0;
            if (d > 1e-10f) {
                float r = roundf((x[start + i] - dmin) / d);
                r = fmaxf(r, 0.0f);
                r = fminf(r, 15.0f);
                q = (uint8_t)r;
            }
            blk[4 + i / 2] |= (uint8_t)(q << ((i % 2) ? 4 : 0));
        }
    }
}

void orc_q4_dequant_row(const uint8_t* in, int head_dim, float* out) {
    int groups = (head_dim + 31) / 32;
    for (int g = 0; g < groups; g++) {
        const uint8_t* blk = in + g * 20;
        float d = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        float dmin = orc_f16_to_f32((uint16_t)(blk[2] | (blk[3] << 8)));
        for (int i = 0; i < 32; i++) {
            if (g * 32 + i >= head_dim) break;
            uint8_t b = blk[4 + i / 2];
            uint8_t nib = (i % 2 == 0) ? (uint8_t)(b & 0x0f) : (uint8_t)(b >> 4);
            float prod = d * (float)nib;
            out[g * 32 + i] = prod + dmin;
        }
    }
}

void orc_q4_quantize_rows(const float* x, int64_t n_rows, int head_dim, uint8_t* out) {
    int rb = orc_q4_row_bytes(head_dim);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < n_rows; r++)
        orc_q4_quantize_row(x + r * head_dim, head_dim, out + r * rb);
}

void orc_q4_dequant_rows(const uint8_t* in, int64_t n_rows, int head_dim, float* out) {
    int rb = orc_q4_row_bytes(head_dim);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < n_rows; r++)
        orc_q4_dequant_row(in + r * rb, head_dim, out + r * head_dim);
}

/* ------------------------------------------------------------------------
 * Zone page arithmetic (cache.rs:17-21 constants, 185-237 zone build and
 * flat ids, 593-611 page_id/page_start_for/slot_in_page, 365/689/711 f32
 * offsets, 627/665/733 Q4 offsets).
 * --------------------------------------------------------------------- */
static const int64_t ZSTART[3] = {0, 4096, 131072};
static const int64_t ZBS[3] = {32, 128, 1024};

int64_t orc_zone_index(int64_t pos) { return pos < ZSTART[1] ? 0 : (pos < ZSTART[2] ? 1 : 2); }
int64_t orc_zone_block_size(int64_t pos) { return ZBS[orc_zone_index(pos)]; }

static int64_t zone_pages(int z, int64_t max_seq_len) {
    int64_t start = ZSTART[z];
    int64_t end = z + 1 < 3 ? ZSTART[z + 1] : max_seq_len;
    int64_t cov = end > start ? end - start : 0;
    return cov > 0 ? (cov + ZBS[z] - 1) / ZBS[z] : 0;
}

int64_t orc_zone_total_pages(int64_t max_seq_len) {
    return zone_pages(0, max_seq_len) + zone_pages(1, max_seq_len) + zone_pages(2, max_seq_len);
}

int64_t orc_zone_page_id(int64_t pos, int64_t max_seq_len) {
    int z = (int)orc_zone_index(pos);
    int64_t off = 0;
    for (int i = 0; i < z; i++) off += zone_pages(i, max_seq_len);
    return off + (pos - ZSTART[z]) / ZBS[z];
}

int64_t orc_zone_slot_in_page(int64_t pos) {
    int z = (int)orc_zone_index(pos);
    return (pos - ZSTART[z]) % ZBS[z];
}

int64_t orc_zone_page_start(int64_t pos) { return pos - orc_zone_slot_in_page(pos); }

int64_t orc_zone_f32_offset(int64_t layer, int64_t kv_head, int64_t pos, int64_t n_kv_heads,
                            int64_t head_dim) {
    int64_t bs = orc_zone_block_size(pos);
    return ((layer * n_kv_heads + kv_head) * bs + orc_zone_slot_in_page(pos)) * head_dim;
}

int64_t orc_zone_q4_offset(int64_t layer, int64_t kv_head, int64_t pos, int64_t n_kv_heads,
                           int64_t head_dim) {
    int64_t bs = orc_zone_block_size(pos);
    int64_t rb = orc_q4_row_bytes((int)head_dim);
    return (layer * n_kv_heads + kv_head) * bs * rb + orc_zone_slot_in_page(pos) * rb;
}

/* ------------------------------------------------------------------------
 * Position sets
 * attention_sparse (swamp-engine/src/ops.rs:97-113):
 *   valid_end = min(q_pos, seq_len-1)
 *   window_start = valid_end > window ? valid_end - window + 1 : 0   (strict >)
 *   globals: stride*g for g < min(window_start/stride, 128)
 *   then window_start..=valid_end
 * The reference divides by global_stride unconditionally (a zero stride
 * panics there); here stride <= 0 means no globals.
 * attention_fugu (ops.rs:459-484): the same with sentinel_stride, then each
 * dspark position p <= valid_end not already present, in the given order.
 * --------------------------------------------------------------------- */
static int sparse_into(int seq_len, int q_pos, int window, int stride, int32_t* out, int cap) {
    if (seq_len <= 0 || q_pos < 0 || window < 0) return -1;
    int valid_end = q_pos < seq_len - 1 ? q_pos : seq_len - 1;
    int ws = valid_end > window ? valid_end - window + 1 : 0;
    int n = 0;
    if (stride > 0) {
        int gc = ws / stride;
        if (gc > 128) gc = 128;
        for (int g = 0; g < gc; g++) {
            if (n >= cap) return -2;
            out[n++] = stride * g;
        }
    }
    for (int t = ws; t <= valid_end; t++) {
        if (n >= cap) return -2;
        out[n++] = t;
    }
    return n;
}

int orc_sparse_positions(int seq_len, int q_pos, int window, int global_stride, int32_t* out,
                         int cap) {
    return sparse_into(seq_len, q_pos, window, global_stride, out, cap);
}

int orc_fugu_positions(int seq_len, int q_pos, int window, int sentinel_stride,
                       const int32_t* dspark, int n_dspark, int32_t* out, int cap) {
    int n = sparse_into(seq_len, q_pos, window, sentinel_stride, out, cap);
    if (n < 0) return n;
    int valid_end = q_pos < seq_len - 1 ? q_pos : seq_len - 1;
    for (int i = 0; i < n_dspark; i++) {
        int p = dspark[i];
        if (p < 0 || p > valid_end) continue;
        int present = 0;
        for (int j = 0; j < n; j++)
            if (out[j] == p) { present = 1; break; }
        if (present) continue;
        if (n >= cap) return -2;
        out[n++] = p;
    }
    return n;
}

/* ------------------------------------------------------------------------
 * Attention
 * --------------------------------------------------------------------- */
static inline int64_t row_index(const orc_kv_layout* kv, int64_t t, int64_t h) {
    int64_t blk = kv->table ? (int64_t)kv->table[t / kv->block_tokens] : 0;
    return blk * kv->block_stride + h * kv->head_stride + (t % kv->block_tokens) * kv->token_stride;
}

/* Returns a pointer to the f32 row; binary16 rows are widened into tmp, Q4
 * rows dequantised into tmp first,
 * as the reference reads Q4 pages through their f32 view (cache.rs:338-405). */
static inline const float* fetch_row(const orc_kv_layout* kv, const void* base, int64_t t,
                                     int64_t h, int head_dim, float* tmp) {
    int64_t idx = row_index(kv, t, h);
    if (kv->dtype == ORC_KV_F32) return (const float*)base + idx;
    if (kv->dtype == ORC_KV_F16) {
        const uint16_t* r = (const uint16_t*)base + idx;
        for (int d = 0; d < head_dim; d++) tmp[d] = orc_f16_to_f32(r[d]);
        return tmp;
    }
    orc_q4_dequant_row((const uint8_t*)base + idx, head_dim, tmp);
    return tmp;
}

/* One head of ops::attention / attention_tracked (ops.rs:170-278, 283-401):
 * scores for t in [0, valid_end], -inf for (valid_end, seq_len), max, exp,
 * sum in t order, multiply by 1/sum (normalise before accumulating), then
 * out = sum_t p_t V_t with weighted_sum. */
ORC_CLONES
static void head_full(float* out, const float* qh, const orc_kv_layout* kv, int kvh, int seq_len,
                      int valid_end, int head_dim, float scale, float* scores, float* tmp) {
    float mx = -INFINITY;
    for (int t = 0; t <= valid_end; t++) {
        const float* kr = fetch_row(kv, kv->k_base, t, kvh, head_dim, tmp);
        float s = dot16(qh, kr, head_dim) * scale;
        scores[t] = s;
        if (s > mx) mx = s;
    }
    for (int t = valid_end + 1; t < seq_len; t++) scores[t] = -INFINITY;
    float sum = 0.0f;
    for (int t = 0; t < seq_len; t++) {
        float e = expf(scores[t] - mx);
        scores[t] = e;
        sum += e;
    }
    float inv = 1.0f / sum;
    for (int t = 0; t < seq_len; t++) scores[t] *= inv;
    for (int d = 0; d < head_dim; d++) out[d] = 0.0f;
    for (int t = 0; t <= valid_end; t++) {
        const float* vr = fetch_row(kv, kv->v_base, t, kvh, head_dim, tmp);
        axpy16(out, vr, scores[t], head_dim);
    }
}

/* One head of attention_sparse / attention_fugu (ops.rs:126-166, 497-540):
 * softmax over exactly the listed positions, no mask. */
ORC_CLONES
static void head_positions(float* out, const float* qh, const orc_kv_layout* kv, int kvh,
                           const int32_t* pos, int n_pos, int head_dim, float scale,
                           float* scores, float* tmp) {
    float mx = -INFINITY;
    for (int i = 0; i < n_pos; i++) {
        const float* kr = fetch_row(kv, kv->k_base, pos[i], kvh, head_dim, tmp);
        float s = dot16(qh, kr, head_dim) * scale;
        scores[i] = s;
        if (s > mx) mx = s;
    }
    float sum = 0.0f;
    for (int i = 0; i < n_pos; i++) {
        float e = expf(scores[i] - mx);
        scores[i] = e;
        sum += e;
    }
    float inv = 1.0f / sum;
    for (int i = 0; i < n_pos; i++) scores[i] *= inv;
    for (int d = 0; d < head_dim; d++) out[d] = 0.0f;
    for (int i = 0; i < n_pos; i++) {
        const float* vr = fetch_row(kv, kv->v_base, pos[i], kvh, head_dim, tmp);
        axpy16(out, vr, scores[i], head_dim);
    }
}

static int check_heads(int n_heads, int n_kv_heads, int head_dim) {
    if (n_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0) return -1;
    if (n_heads % n_kv_heads != 0) return -1;
    return 0;
}

int orc_attention(float* out, const float* q, const orc_kv_layout* kv, int seq_len, int q_pos,
                  int n_heads, int n_kv_heads, int head_dim, double* importance, int nthreads) {
    if (!out || !q || !kv || seq_len <= 0 || q_pos < 0) return -1;
    if (check_heads(n_heads, n_kv_heads, head_dim)) return -1;
    int n_rep = n_heads / n_kv_heads;
    int valid_end = q_pos < seq_len - 1 ? q_pos : seq_len - 1;
    float scale = 1.0f / sqrtf((float)head_dim);
    /* Per-head probabilities are kept so that the importance sum can be
     * taken in head order (the reference adds under a Mutex in whatever
     * order rayon finishes, ops.rs:362-368). */
    float* probs = importance ? (float*)malloc(sizeof(float) * (size_t)seq_len * (size_t)n_heads) : NULL;
    if (importance && !probs) return -3;
    int err = 0;
#pragma omp parallel num_threads(nthreads > 0 ? nthreads : 1)
    {
        float* scores = (float*)malloc(sizeof(float) * (size_t)seq_len);
        float* tmp = (float*)malloc(sizeof(float) * (size_t)head_dim);
        if (!scores || !tmp) {
#pragma omp atomic write
            err = -3;
        } else {
#pragma omp for schedule(dynamic, 1)
            for (int h = 0; h < n_heads; h++) {
                head_full(out + (size_t)h * head_dim, q + (size_t)h * head_dim, kv, h / n_rep,
                          seq_len, valid_end, head_dim, scale, scores, tmp);
                if (probs) memcpy(probs + (size_t)h * seq_len, scores, sizeof(float) * (size_t)seq_len);
            }
        }
        free(scores);
        free(tmp);
    }
    if (probs) {
        if (!err)
            for (int h = 0; h < n_heads; h++)
                for (int t = 0; t < seq_len; t++) importance[t] += (double)probs[(size_t)h * seq_len + t];
        free(probs);
    }
    return err;
}

int orc_attention_positions(float* out, const float* q, const orc_kv_layout* kv,
                            const int32_t* positions, int n_pos, int n_heads, int n_kv_heads,
                            int head_dim, double* importance, int nthreads) {
    if (!out || !q || !kv || !positions || n_pos <= 0) return -1;
    if (check_heads(n_heads, n_kv_heads, head_dim)) return -1;
    int n_rep = n_heads / n_kv_heads;
    float scale = 1.0f / sqrtf((float)head_dim);
    /* importance[i] += sum over heads of the probability of positions[i],
     * added in head order as orc_attention does. */
    float* probs = importance ? (float*)malloc(sizeof(float) * (size_t)n_pos * (size_t)n_heads) : NULL;
    if (importance && !probs) return -3;
    int err = 0;
#pragma omp parallel num_threads(nthreads > 0 ? nthreads : 1)
    {
        float* scores = (float*)malloc(sizeof(float) * (size_t)n_pos);
        float* tmp = (float*)malloc(sizeof(float) * (size_t)head_dim);
        if (!scores || !tmp) {
#pragma omp atomic write
            err = -3;
        } else {
#pragma omp for schedule(dynamic, 1)
            for (int h = 0; h < n_heads; h++) {
                head_positions(out + (size_t)h * head_dim, q + (size_t)h * head_dim, kv, h / n_rep,
                               positions, n_pos, head_dim, scale, scores, tmp);
                if (probs) memcpy(probs + (size_t)h * n_pos, scores, sizeof(float) * (size_t)n_pos);
            }
        }
        free(scores);
        free(tmp);
    }
    if (probs) {
        if (!err)
            for (int h = 0; h < n_heads; h++)
                for (int i = 0; i < n_pos; i++) importance[i] += (double)probs[(size_t)h * n_pos + i];
        free(probs);
    }
    return err;
}

/* ------------------------------------------------------------------------
 * attention_sparse_q4 (swamp-engine/src/ops.rs:597-723): attention_sparse's
 * position set over Q4-20B rows, read with that function's own rules:
 *   - group g of a row is the 20 bytes at (slot * groups + g) * 20 of the
 *     (layer, kv head) page block (ops.rs:639-644), f16 d and dmin first;
 *   - the 16 nibble bytes give elements 0..15 from their low nibbles and
 *     16..31 from their high nibbles (ops.rs:653-656), where the writer
 *     (cache.rs:655-663) and dequant_block interleave them;
 *   - element = fma(d, nibble, dmin) (ops.rs:661-662, 703-704);
 *   - q.k in 16 FMA lanes over 16-element chunks, lanes added in order
 *     (ops.rs:664-674), times scale;
 *   - softmax: max, exp(s - max) summed in position order, times 1/sum
 *     (ops.rs:678-682);
 *   - out = sum of fma(v, w, out) in position order over the positions
 *     whose weight w is not below 1e-8 (ops.rs:686-720).
 * head_dim must be a multiple of 32 (the reference reads 32 q values per
 * group).  global_stride <= 0 means no globals (the reference divides by
 * it).
 * --------------------------------------------------------------------- */
void orc_q4_a5_row(const uint8_t* in, int head_dim, float* out) {
    int groups = head_dim / 32;
    for (int g = 0; g < groups; g++) {
        const uint8_t* blk = in + g * 20;
        float d = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        float dmin = orc_f16_to_f32((uint16_t)(blk[2] | (blk[3] << 8)));
        for (int j = 0; j < 16; j++) {
            uint8_t b = blk[4 + j];
            out[g * 32 + j] = fmaf(d, (float)(b & 0x0f), dmin);
            out[g * 32 + 16 + j] = fmaf(d, (float)(b >> 4), dmin);
        }
    }
}

int orc_sparse_q4_positions(int seq_len, int q_pos, int window, int global_stride, int32_t* out,
                            int cap) {
    return sparse_into(seq_len, q_pos, window, global_stride, out, cap);
}

ORC_CLONES
static void head_sparse_q4(float* out, const float* qh, const orc_kv_layout* kv, int kvh,
                           const int32_t* pos, int n_pos, int head_dim, float scale,
                           float* scores, float* tmp) {
    float mx = -INFINITY;
    for (int i = 0; i < n_pos; i++) {
        orc_q4_a5_row((const uint8_t*)kv->k_base + row_index(kv, pos[i], kvh), head_dim, tmp);
        float acc[16];
        for (int l = 0; l < 16; l++) acc[l] = 0.0f;
        for (int c = 0; c < head_dim; c += 16)
            for (int l = 0; l < 16; l++) acc[l] = fmaf(tmp[c + l], qh[c + l], acc[l]);
        float dot = 0.0f;
        for (int l = 0; l < 16; l++) dot = dot + acc[l];
        float s = dot * scale;
        scores[i] = s;
        if (s > mx) mx = s;
    }
    float sum = 0.0f;
    for (int i = 0; i < n_pos; i++) {
        float e = expf(scores[i] - mx);
        scores[i] = e;
        sum += e;
    }
    float inv = 1.0f / sum;
    for (int i = 0; i < n_pos; i++) scores[i] *= inv;
    for (int d = 0; d < head_dim; d++) out[d] = 0.0f;
    for (int i = 0; i < n_pos; i++) {
        float w = scores[i];
        if (w < 1e-8f) continue;
        orc_q4_a5_row((const uint8_t*)kv->v_base + row_index(kv, pos[i], kvh), head_dim, tmp);
        for (int d = 0; d < head_dim; d++) out[d] = fmaf(tmp[d], w, out[d]);
    }
}

int orc_attention_sparse_q4(float* out, const float* q, const orc_kv_layout* kv, int seq_len,
                            int q_pos, int n_heads, int n_kv_heads, int head_dim, int window,
                            int global_stride, int nthreads) {
    if (!out || !q || !kv || kv->dtype != ORC_KV_Q4 || head_dim % 32) return -1;
    if (check_heads(n_heads, n_kv_heads, head_dim)) return -1;
    int cap = (window > 0 ? window : 0) + 130;
    if (cap > seq_len + 1) cap = seq_len + 1;
    int32_t* pos = (int32_t*)malloc(sizeof(int32_t) * (size_t)cap);
    if (!pos) return -3;
    int n_pos = sparse_into(seq_len, q_pos, window, global_stride, pos, cap);
    if (n_pos < 0) {
        free(pos);
        return n_pos == -2 ? -3 : -1;
    }
    int n_rep = n_heads / n_kv_heads;
    float scale = 1.0f / sqrtf((float)head_dim);
    int err = 0;
    if (n_pos == 0) {
        memset(out, 0, sizeof(float) * (size_t)n_heads * (size_t)head_dim);
        free(pos);
        return 0;
    }
#pragma omp parallel num_threads(nthreads > 0 ? nthreads : 1)
    {
        float* scores = (float*)malloc(sizeof(float) * (size_t)n_pos);
        float* tmp = (float*)malloc(sizeof(float) * (size_t)head_dim);
        if (!scores || !tmp) {
#pragma omp atomic write
            err = -3;
        } else {
#pragma omp for schedule(dynamic, 1)
            for (int h = 0; h < n_heads; h++)
                head_sparse_q4(out + (size_t)h * head_dim, q + (size_t)h * head_dim, kv, h / n_rep,
                               pos, n_pos, head_dim, scale, scores, tmp);
        }
        free(scores);
        free(tmp);
    }
    free(pos);
    return err;
}

/* Prefill as the reference executes it: one ops::attention call per token
 * with seq_len = abs_pos + 1 and q_pos = abs_pos (executor.rs:132-137). */
int orc_attention_rows(float* out, const float* q, int64_t q_row_stride, int64_t out_row_stride,
                       const orc_kv_layout* kv, const int32_t* rows, int n_rows, int n_heads,
                       int n_kv_heads, int head_dim, int nthreads) {
    if (!out || !q || !kv || !rows || n_rows <= 0) return -1;
    if (check_heads(n_heads, n_kv_heads, head_dim)) return -1;
    int n_rep = n_heads / n_kv_heads;
    float scale = 1.0f / sqrtf((float)head_dim);
    int max_row = 0;
    for (int i = 0; i < n_rows; i++) {
        if (rows[i] < 0) return -1;
        if (rows[i] > max_row) max_row = rows[i];
    }
    int err = 0;
    long long total = (long long)n_rows * n_heads;
#pragma omp parallel num_threads(nthreads > 0 ? nthreads : 1)
    {
        float* scores = (float*)malloc(sizeof(float) * (size_t)(max_row + 1));
        float* tmp = (float*)malloc(sizeof(float) * (size_t)head_dim);
        if (!scores || !tmp) {
#pragma omp atomic write
            err = -3;
        } else {
#pragma omp for schedule(dynamic, 1)
            for (long long w = 0; w < total; w++) {
                int ri = (int)(w / n_heads), h = (int)(w % n_heads);
                int r = rows[ri];
                head_full(out + (size_t)r * out_row_stride + (size_t)h * head_dim,
                          q + (size_t)r * q_row_stride + (size_t)h * head_dim, kv, h / n_rep, r + 1,
                          r, head_dim, scale, scores, tmp);
            }
        }
        free(scores);
        free(tmp);
    }
    return err;
}

/* ------------------------------------------------------------------------
 * mojo_softmax_padic (swamp-kernels/src/lib.rs:181-223) following its
 * AVX-512 branch (lib.rs:110-179, 202-206), the one x86-64 AVX-512 hosts
 * take; the scalar fallback (lib.rs:209-222) is not restated.
 * --------------------------------------------------------------------- */

/* Rust `f32 as i32`: truncate toward zero, saturate, NaN -> 0. */
static int32_t sat_i32(float x) {
    if (x != x) return 0;
    if (x >= 2147483648.0f) return INT32_MAX;
    if (x <= -2147483648.0f) return INT32_MIN;
    return (int32_t)x;
}

/* exp_q16_16 (lib.rs:102-108) */
int32_t orc_exp_q16_16(int32_t x_fixed) {
    if (x_fixed < -655360) return 0;
    if (x_fixed >= 0) return 65536;
    float xr = (float)x_fixed / 65536.0f;
    float r = roundf(expf(xr) * 65536.0f);
    r = fmaxf(r, 0.0f);
    return sat_i32(r);
}

void orc_softmax_padic(const float* logits, float* probs, int n, float temperature) {
    if (!logits || !probs || n <= 0) return;
    float inv_tmp = 1.0f / fmaxf(temperature, 1e-6f);
    int32_t* fixed = (int32_t*)malloc(sizeof(int32_t) * (size_t)n);
    int32_t* e = (int32_t*)malloc(sizeof(int32_t) * (size_t)n);
    if (!fixed || !e) {
        free(fixed);
        free(e);
        return;
    }
    for (int i = 0; i < n; i++) fixed[i] = sat_i32((logits[i] * inv_tmp) * 65536.0f);
    int32_t mx = INT32_MIN;
    for (int i = 0; i < n; i++)
        if (fixed[i] > mx) mx = fixed[i];
    int64_t sum = 0;
    for (int i = 0; i < n; i++) {
        int32_t diff = (int32_t)((uint32_t)fixed[i] - (uint32_t)mx); /* wrapping, as release Rust */
        e[i] = orc_exp_q16_16(diff);
        sum += e[i];
    }
    if (sum > 0) {
        int32_t inv = (int32_t)(uint32_t)((1ull << 32) / (uint64_t)sum);
        int simd_end = (n / 16) * 16;
        for (int i = 0; i < simd_end; i++) /* _mm512_mullo_epi32 + _mm512_srli_epi32(.,16) */
            e[i] = (int32_t)(((uint32_t)e[i] * (uint32_t)inv) >> 16);
        for (int i = simd_end; i < n; i++)
            e[i] = (int32_t)(((int64_t)e[i] * (int64_t)inv) >> 16);
    }
    for (int i = 0; i < n; i++) probs[i] = (float)e[i] / 65536.0f;
    free(fixed);
    free(e);
}

/* ------------------------------------------------------------------------
 * StokesKVCacheSim + mojo_stokes_* (swamp-kernels/src/lib.rs:27-85):
 * append K, V, score; above 4096 tokens drop the first minimum-score token.
 * The reference panics on a NaN comparison (partial_cmp().unwrap()); here
 * that case returns -1 and leaves the cache unchanged past the append.
 * --------------------------------------------------------------------- */
typedef struct {
    int n, cap, head_dim;
    float *keys, *values, *scores;
} orc_stokes;

void* orc_stokes_init(int head_dim) {
    orc_stokes* c = (orc_stokes*)calloc(1, sizeof(orc_stokes));
    if (c) c->head_dim = head_dim;
    return c;
}

void orc_stokes_free(void* p) {
    orc_stokes* c = (orc_stokes*)p;
    if (!c) return;
    free(c->keys);
    free(c->values);
    free(c->scores);
    free(c);
}

int orc_stokes_append(void* p, int token_id, const float* key, const float* value, float score) {
    (void)token_id;
    orc_stokes* c = (orc_stokes*)p;
    if (!c || !key || !value) return 0;
    int hd = c->head_dim;
    if (c->n == c->cap) {
        int nc = c->cap ? c->cap * 2 : 64;
        float* k = (float*)realloc(c->keys, sizeof(float) * (size_t)nc * (size_t)hd);
        if (!k) return -3;
        c->keys = k;
        float* v = (float*)realloc(c->values, sizeof(float) * (size_t)nc * (size_t)hd);
        if (!v) return -3;
        c->values = v;
        float* s = (float*)realloc(c->scores, sizeof(float) * (size_t)nc);
        if (!s) return -3;
        c->scores = s;
        c->cap = nc;
    }
    memcpy(c->keys + (size_t)c->n * hd, key, sizeof(float) * (size_t)hd);
    memcpy(c->values + (size_t)c->n * hd, value, sizeof(float) * (size_t)hd);
    c->scores[c->n] = score;
    c->n++;
    if (c->n > 4096) {
        int mi = 0;
        for (int i = 0; i < c->n; i++)
            if (c->scores[i] != c->scores[i]) return -1;
        for (int i = 1; i < c->n; i++)
            if (c->scores[i] < c->scores[mi]) mi = i;
        size_t tail = (size_t)(c->n - mi - 1);
        memmove(c->keys + (size_t)mi * hd, c->keys + (size_t)(mi + 1) * hd, sizeof(float) * tail * hd);
        memmove(c->values + (size_t)mi * hd, c->values + (size_t)(mi + 1) * hd, sizeof(float) * tail * hd);
        memmove(c->scores + mi, c->scores + mi + 1, sizeof(float) * tail);
        c->n--;
    }
    return 0;
}

int orc_stokes_count(const void* p) { return p ? ((const orc_stokes*)p)->n : 0; }

int orc_stokes_read(const void* p, float* keys, float* values, float* scores) {
    const orc_stokes* c = (const orc_stokes*)p;
    if (!c) return -1;
    if (keys) memcpy(keys, c->keys, sizeof(float) * (size_t)c->n * c->head_dim);
    if (values) memcpy(values, c->values, sizeof(float) * (size_t)c->n * c->head_dim);
    if (scores) memcpy(scores, c->scores, sizeof(float) * (size_t)c->n);
    return c->n;
}

/* ------------------------------------------------------------------------
 * RoPE (swamp-engine/src/ops.rs:11, 20-37, 40-79)
 * --------------------------------------------------------------------- */
void orc_rope_lut(int head_dim, int max_ctx, float* lut) {
    const int half = head_dim / 2;
    for (int m = 0; m < max_ctx; m++)
        for (int k = 0; k < half; k++) {
            /* ops.rs:30-33: freq = 1 / theta^(2k/D); angle = m * freq (f32) */
            float freq = 1.0f / powf(10000.0f, (float)(2 * k) / (float)head_dim);
            float angle = (float)m * freq;
            lut[((size_t)m * half + k) * 2] = cosf(angle);
            lut[((size_t)m * half + k) * 2 + 1] = sinf(angle);
        }
}

static void rope_rows(float* x, int rows, int head_dim, const float* cs) {
    const int half = head_dim / 2;
    for (int h = 0; h < rows; h++) {
        float* v = x + (size_t)h * head_dim;
        for (int k = 0; k < half; k++) {
            /* ops.rs:70-78 */
            float a = v[2 * k], b = v[2 * k + 1];
            float c = cs[2 * k], s = cs[2 * k + 1];
            v[2 * k] = a * c - b * s;
            v[2 * k + 1] = a * s + b * c;
        }
    }
}

void orc_apply_rope(float* q, float* k, int pos, int n_heads, int n_kv_heads, int head_dim,
                    int max_ctx, const float* lut) {
    if (pos > max_ctx - 1) pos = max_ctx - 1; /* ops.rs:53 */
    const float* cs = lut + (size_t)pos * (head_dim / 2) * 2;
    rope_rows(q, n_heads, head_dim, cs);
    rope_rows(k, n_kv_heads, head_dim, cs);
}

/* ------------------------------------------------------------------ Q4_K */

/* swamp-kernels/src/fused_gemv_q4k.rs:30-43 (unpack_scales_q4k): 12 bytes
 * -> eight 6-bit scales and mins. */
void orc_q4k_unpack_scales(const uint8_t* sc, uint8_t* scales, uint8_t* mins) {
    for (int j = 0; j < 4; j++) {
        scales[j] = sc[j] & 63;
        mins[j] = sc[j + 4] & 63;
    }
    for (int j = 4; j < 8; j++) {
        scales[j] = (uint8_t)((sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4));
        mins[j] = (uint8_t)((sc[j + 4] >> 4) | ((sc[j] >> 6) << 4));
    }
}

/* One 144-byte block -> 256 weights, as the scalar GEMV forms them
 * (fused_gemv_q4k.rs:395-448): w = (d * scale) * q - (dmin * min), the two
 * products rounded to f32 first; qs pair p holds sub-block 2p in its low
 * nibbles and 2p+1 in its high nibbles. */
void orc_q4k_dequant_block(const uint8_t* blk, float* out) {
    const float d = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
    const float dmin = orc_f16_to_f32((uint16_t)(blk[2] | (blk[3] << 8)));
    uint8_t scales[8], mins[8];
    orc_q4k_unpack_scales(blk + 4, scales, mins);
    const uint8_t* qs = blk + 16;
    for (int pair = 0; pair < 4; pair++) {
        const uint8_t* qb = qs + pair * 32;
        const int se = pair * 2, so = pair * 2 + 1;
        const float sve = d * (float)(scales[se] & 0x3F), mve = dmin * (float)(mins[se] & 0x3F);
        const float svo = d * (float)(scales[so] & 0x3F), mvo = dmin * (float)(mins[so] & 0x3F);
        for (int i = 0; i < 32; i++) {
            out[se * 32 + i] = sve * (float)(qb[i] & 0x0F) - mve;
            out[so * 32 + i] = svo * (float)(qb[i] >> 4) - mvo;
        }
    }
}

/* fused_gemv_q4k_scalar (fused_gemv_q4k.rs:395-448), same accumulation
 * order: per row one f32 accumulator over blocks, pairs, the even
 * sub-block's 32 products then the odd one's. */
int orc_gemv_q4k(const uint8_t* w, const float* x, float* out, int n_rows, int n_cols) {
    if (n_cols <= 0 || n_cols % 256 || n_rows < 0) return -1;
    const int nb = n_cols / 256;
#pragma omp parallel for schedule(static)
    for (int row = 0; row < n_rows; row++) {
        float acc = 0.0f;
        for (int blk = 0; blk < nb; blk++) {
            const uint8_t* b = w + ((size_t)row * nb + blk) * 144;
            const float d = orc_f16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
            const float dmin = orc_f16_to_f32((uint16_t)(b[2] | (b[3] << 8)));
            uint8_t scales[8], mins[8];
            orc_q4k_unpack_scales(b + 4, scales, mins);
            const uint8_t* qs = b + 16;
            const float* xb = x + (size_t)blk * 256;
            for (int pair = 0; pair < 4; pair++) {
                const uint8_t* qb = qs + pair * 32;
                const int se = pair * 2;
                const float sve = d * (float)(scales[se] & 0x3F);
                const float mve = dmin * (float)(mins[se] & 0x3F);
                for (int i = 0; i < 32; i++) {
                    const float wf = sve * (float)(qb[i] & 0x0F) - mve;
                    acc += wf * xb[se * 32 + i];
                }
                const int so = pair * 2 + 1;
                const float svo = d * (float)(scales[so] & 0x3F);
                const float mvo = dmin * (float)(mins[so] & 0x3F);
                for (int i = 0; i < 32; i++) {
                    const float wf = svo * (float)(qb[i] >> 4) - mvo;
                    acc += wf * xb[so * 32 + i];
                }
            }
        }
        out[row] = acc;
    }
    return 0;
}

/* ------------------------------------------------------------------ Q6_K */

/* swamp-kernels/src/fused_gemv_q6k.rs:6-20: the reference's own f16 -> f32
 * of the block scale.  Normal values convert exactly; exponent 0 (zero and
 * subnormals) builds the bits sign | (1009 << 23, wrapped to 32 bits) |
 * mant << 13, i.e. a large negative number, and exponent 31 (inf, NaN)
 * becomes a finite value.  Restated as is. */
float orc_q6k_scale_to_f32(uint16_t v) {
    const uint32_t sign = (uint32_t)(v >> 15) << 31;
    const uint32_t e = (v >> 10) & 0x1f;
    const uint32_t mant = v & 0x3ff;
    uint32_t bits;
    if (e == 0)
        bits = sign | (uint32_t)(1009u << 23) | (mant << 13);
    else
        bits = sign | ((e + 112u) << 23) | (mant << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* One 210-byte block (ql[128], qh[64], int8 scales[16], f16 d) -> 256
 * weights d * sc * (q - 32), each product rounded left to right in f32 as
 * the scalar GEMV forms it (fused_gemv_q6k.rs:248-293): half h, l = 0..31:
 * element 128h + l + 32k takes q_k from the low (k = 0, 1) or high (k = 2, 3)
 * nibble of ql[64h + l + 32(k&1)] and bits 2k..2k+1 of qh[32h + l], and
 * scale sc[8h + l/16 + 2k]. */
void orc_q6k_dequant_block(const uint8_t* blk, float* out) {
    const float d = orc_q6k_scale_to_f32((uint16_t)(blk[208] | (blk[209] << 8)));
    for (int h = 0; h < 2; h++) {
        const uint8_t* ql = blk + 64 * h;
        const uint8_t* qh = blk + 128 + 32 * h;
        const int8_t* sc = (const int8_t*)(blk + 192 + 8 * h);
        for (int l = 0; l < 32; l++) {
            const int is = l / 16;
            const int q[4] = {(ql[l] & 0x0F) | ((qh[l] & 3) << 4),
                              (ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4),
                              (ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4),
                              (ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)};
            for (int k = 0; k < 4; k++)
                out[128 * h + l + 32 * k] = d * (float)sc[is + 2 * k] * (float)(q[k] - 32);
        }
    }
}

/* fused_gemv_q6k_scalar (fused_gemv_q6k.rs:248-293), same accumulation
 * order: per block, halves, l = 0..31, the four elements l, l+32, l+64,
 * l+96, each acc += ((d * sc) * q) * x. */
int orc_gemv_q6k(const uint8_t* w, const float* x, float* out, int n_rows, int n_cols) {
    if (n_cols <= 0 || n_cols % 256 || n_rows < 0) return -1;
    const int nb = n_cols / 256;
#pragma omp parallel for schedule(static)
    for (int row = 0; row < n_rows; row++) {
        float acc = 0.0f;
        for (int blk = 0; blk < nb; blk++) {
            const uint8_t* b = w + ((size_t)row * nb + blk) * 210;
            const float d = orc_q6k_scale_to_f32((uint16_t)(b[208] | (b[209] << 8)));
            for (int h = 0; h < 2; h++) {
                const uint8_t* ql = b + 64 * h;
                const uint8_t* qh = b + 128 + 32 * h;
                const int8_t* sc = (const int8_t*)(b + 192 + 8 * h);
                const float* xh = x + (size_t)blk * 256 + 128 * h;
                for (int l = 0; l < 32; l++) {
                    const int is = l / 16;
                    const float q1 = (float)(((ql[l] & 0x0F) | ((qh[l] & 3) << 4)) - 32);
                    const float q2 = (float)(((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32);
                    const float q3 = (float)(((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32);
                    const float q4 = (float)(((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32);
                    acc += d * (float)sc[is] * q1 * xh[l];
                    acc += d * (float)sc[is + 2] * q2 * xh[l + 32];
                    acc += d * (float)sc[is + 4] * q3 * xh[l + 64];
                    acc += d * (float)sc[is + 6] * q4 * xh[l + 96];
                }
            }
        }
        out[row] = acc;
    }
    return 0;
}

/* ------------------------------------------------------------------------
 * sparse_attention_q4 (swamp-gpu/kernels/attention.mojo):
 *   rows: position t's K (and V) row is blocks*20 f32 words at t*blocks*20
 *         (blocks = ceil(head_dim/32), 53-54); block b: word 0 d, word 1
 *         dmin, word 2 + i/2 holds the byte of elements i, i+1 as a float
 *         value, read as an integer (truncation), low nibble for even i
 *         (74-83, 104-113);
 *   k = d*nib + dmin, dot accumulated in element order (76-84),
 *   s = dot * (1/sqrt(head_dim)) (85, 141);
 *   per tile of 64 listed positions (60-63): tile max from -1e10 (66, 87),
 *   tile sum of exp(s - tile max) in order (90-92), then the running
 *   (m, d) from (-1e10, 0): new_m = max(m, tile max), d = d*exp(m - new_m)
 *   + tile_sum*exp(tile max - new_m), m = new_m (94-96);
 *   each position of the tile adds v*w to the output, w = exp(s - m)/d with
 *   the running (m, d) after this tile, skipping w < 1e-8 (99-115); the
 *   output of earlier tiles is not rescaled.
 * The library is built with -ffp-contract=off: each written multiply-add
 * keeps two roundings.
 * --------------------------------------------------------------------- */
static float mojo_q4_elem(const float* row, int i) {
    const float* blk = row + (i / 32) * 20;
    const int e = i % 32;
    const int64_t byte = (int64_t)blk[2 + e / 2];
    const int nib = (int)((byte >> ((e % 2) * 4)) & 0x0F);
    return blk[0] * (float)nib + blk[1];
}

void orc_mojo_sparse_attention_q4(const float* q, const float* k_q4, const float* v_q4,
                                  const int32_t* positions, float* out, int n_heads,
                                  int head_dim, int n_sparse) {
    const int blocks = (head_dim + 31) / 32;
    const int64_t row = (int64_t)blocks * 20;
    const float scale = 1.0f / sqrtf((float)head_dim);
    float scores[64];
    for (int h = 0; h < n_heads; h++) {
        const float* qh = q + (int64_t)h * head_dim;
        float* oh = out + (int64_t)h * head_dim;
        float m = -1e10f, d = 0.0f;
        for (int i = 0; i < head_dim; i++) oh[i] = 0.0f;
        for (int t0 = 0; t0 < n_sparse; t0 += 64) {
            const int nt = n_sparse - t0 < 64 ? n_sparse - t0 : 64;
            float tmax = -1e10f;
            for (int p = 0; p < nt; p++) {
                const float* kr = k_q4 + positions[t0 + p] * row;
                float dot = 0.0f;
                for (int i = 0; i < head_dim; i++) dot += mojo_q4_elem(kr, i) * qh[i];
                scores[p] = dot * scale;
                if (scores[p] > tmax) tmax = scores[p];
            }
            float tsum = 0.0f;
            for (int p = 0; p < nt; p++) tsum += expf(scores[p] - tmax);
            const float nm = m > tmax ? m : tmax;
            d = d * expf(m - nm) + tsum * expf(tmax - nm);
            m = nm;
            for (int p = 0; p < nt; p++) {
                const float w = expf(scores[p] - m) / d;
                if (w < 1e-8f) continue;
                const float* vr = v_q4 + positions[t0 + p] * row;
                for (int i = 0; i < head_dim; i++) oh[i] += mojo_q4_elem(vr, i) * w;
            }
        }
    }
}
