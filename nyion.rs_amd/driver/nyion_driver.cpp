// nyion_driver.cpp — a native caller of libnyion_hip.so through the C ABI
// of include/nyion_hip.h only: no HIP headers, device memory from the
// library's own arena (nyion_hma_*), plain pointers and sizes, as the Rust
// executor's binding would call it (swamp-engine/src/executor.rs:85-137
// prefill, 699-763 decode; swamp-engine/src/linear.rs:99-189 projections).
//
// It runs one paged decode step, a chunk of causal prefill and a Q4_K GEMV
// on synthetic data, recomputes each in double precision on the host (its
// own loops, independent of the library) and reports the largest error.
// Exit status: 0 all within 2e-3 absolute and 1e-3 relative to the largest
// reference value, 1 a mismatch, 2 an API error, 3 no usable device.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <vector>

#include "nyion_hip.h"

namespace {

struct Lcg {
    uint64_t s;
    explicit Lcg(uint64_t seed) : s(seed * 6364136223846793005ULL + 1442695040888963407ULL) {}
    uint32_t next() {
        s = s * 6364136223846793005ULL + 1442695040888963407ULL;
        return (uint32_t)(s >> 33);
    }
    float uniform() { return (float)((next() & 0xffffff) / 8388608.0 - 1.0); }  // [-1, 1)
};

int fail(const char* what) {
    fprintf(stderr, "nyion_driver: %s failed: %s\n", what, nyion_last_error());
    return 2;
}

struct Arena {
    void* h = nullptr;
    ~Arena() {
        if (h) nyion_hma_destroy(h);
    }
    bool alloc(size_t bytes, nyion_allocation& a) {
        return nyion_hma_alloc(h, bytes, NYION_MEM_DEVICE_LOCAL, &a) == NYION_OK;
    }
};

double report(const char* what, const std::vector<float>& got, const std::vector<double>& ref) {
    double err = 0.0, mx = 0.0;
    for (size_t i = 0; i < ref.size(); i++) {
        err = fmax(err, fabs((double)got[i] - ref[i]));
        mx = fmax(mx, fabs(ref[i]));
    }
    const double rel = mx > 0 ? err / mx : err;
    printf("nyion_driver: %-8s max-abs-err %.3e rel %.3e\n", what, err, rel);
    return (err <= 2e-3 && rel <= 1e-3) ? 0.0 : 1.0;
}

// softmax(q . K^T * scale) V in double over positions [0, n) of one head
void attend(const float* q, const std::vector<const float*>& krows,
            const std::vector<const float*>& vrows, int d, double* out) {
    const double scale = 1.0 / sqrt((double)d);
    std::vector<double> s(krows.size());
    double m = -1e300;
    for (size_t t = 0; t < krows.size(); t++) {
        double acc = 0.0;
        for (int i = 0; i < d; i++) acc += (double)q[i] * krows[t][i];
        s[t] = acc * scale;
        m = fmax(m, s[t]);
    }
    double l = 0.0;
    for (double& v : s) l += (v = exp(v - m));
    for (int i = 0; i < d; i++) out[i] = 0.0;
    for (size_t t = 0; t < krows.size(); t++)
        for (int i = 0; i < d; i++) out[i] += s[t] / l * vrows[t][i];
}

// ---------------------------------------------------------------- decode

int run_decode(Arena& ar, double& bad) {
    const int hq = 32, hkv = 4, d = 64, bt = 16, ctx = 300, nblk = 32, maxb = 24;
    Lcg rng(1);
    std::vector<int32_t> table(maxb);
    for (int i = 0; i < maxb; i++) table[i] = i;
    for (int i = maxb - 1; i > 0; i--) {  // shuffled block table
        const int j = (int)(rng.next() % (uint32_t)(i + 1));
        const int32_t t = table[i];
        table[i] = table[j];
        table[j] = t;
    }
    // pool [block][kv head][bt][d]
    const size_t pool_elems = (size_t)nblk * hkv * bt * d;
    std::vector<float> kp(pool_elems), vp(pool_elems), q((size_t)hq * d);
    for (float& x : kp) x = rng.uniform();
    for (float& x : vp) x = rng.uniform();
    for (float& x : q) x = rng.uniform();
    const int32_t ctx_len = ctx;
    const size_t ws_bytes = nyion_paged_decode_workspace_size(1, hq, hkv, d, ctx, 0, 0);
    nyion_allocation a_q, a_k, a_v, a_t, a_c, a_o, a_w;
    if (!ar.alloc(q.size() * 4, a_q) || !ar.alloc(pool_elems * 4, a_k) || !ar.alloc(pool_elems * 4, a_v) ||
        !ar.alloc(maxb * 4, a_t) || !ar.alloc(4, a_c) || !ar.alloc(q.size() * 4, a_o) ||
        !ar.alloc(ws_bytes > 0 ? ws_bytes : 256, a_w))
        return fail("decode arena");
    if (nyion_hma_upload(ar.h, &a_q, q.data(), q.size() * 4) || nyion_hma_upload(ar.h, &a_k, kp.data(), pool_elems * 4) ||
        nyion_hma_upload(ar.h, &a_v, vp.data(), pool_elems * 4) || nyion_hma_upload(ar.h, &a_t, table.data(), maxb * 4) ||
        nyion_hma_upload(ar.h, &a_c, &ctx_len, 4))
        return fail("decode upload");
    if (ws_bytes && nyion_decode_workspace_init(a_w.ptr, ws_bytes, nullptr)) return fail("workspace init");
    if (nyion_paged_decode_attention((const float*)a_q.ptr, a_k.ptr, a_v.ptr, (const int32_t*)a_t.ptr, maxb,
                                     (const int32_t*)a_c.ptr, nullptr, 1, hq, hkv, d, bt, nblk,
                                     NYION_KV_F32, 0, 0, ctx, 0.0f, (float*)a_o.ptr, a_w.ptr, ws_bytes,
                                     nullptr))
        return fail("nyion_paged_decode_attention");
    if (nyion_sync()) return fail("sync");
    std::vector<float> got(q.size());
    if (nyion_hma_download(ar.h, got.data(), &a_o, got.size() * 4)) return fail("decode download");
    std::vector<double> ref(q.size());
    for (int h = 0; h < hq; h++) {
        const int g = h / (hq / hkv);
        std::vector<const float*> kr, vr;
        for (int t = 0; t < ctx; t++) {
            const size_t off = (((size_t)table[t / bt] * hkv + g) * bt + t % bt) * d;
            kr.push_back(&kp[off]);
            vr.push_back(&vp[off]);
        }
        attend(&q[(size_t)h * d], kr, vr, d, &ref[(size_t)h * d]);
    }
    bad += report("decode", got, ref);
    return 0;
}

// --------------------------------------------------------------- prefill

uint16_t bf16_bits(float f) {  // round to nearest even
    uint32_t x;
    memcpy(&x, &f, 4);
    return (uint16_t)((x + 0x7fffu + ((x >> 16) & 1u)) >> 16);
}
float bf16_value(uint16_t b) {
    const uint32_t x = (uint32_t)b << 16;
    float f;
    memcpy(&f, &x, 4);
    return f;
}

int run_prefill(Arena& ar, double& bad) {
    const int n = 100, hq = 8, hkv = 2, d = 64;
    Lcg rng(2);
    std::vector<uint16_t> q((size_t)n * hq * d), k((size_t)n * hkv * d), v((size_t)n * hkv * d);
    for (auto& x : q) x = bf16_bits(rng.uniform());
    for (auto& x : k) x = bf16_bits(rng.uniform());
    for (auto& x : v) x = bf16_bits(rng.uniform());
    nyion_allocation a_q, a_k, a_v, a_o;
    if (!ar.alloc(q.size() * 2, a_q) || !ar.alloc(k.size() * 2, a_k) || !ar.alloc(v.size() * 2, a_v) ||
        !ar.alloc(q.size() * 4, a_o))
        return fail("prefill arena");
    if (nyion_hma_upload(ar.h, &a_q, q.data(), q.size() * 2) || nyion_hma_upload(ar.h, &a_k, k.data(), k.size() * 2) ||
        nyion_hma_upload(ar.h, &a_v, v.data(), v.size() * 2))
        return fail("prefill upload");
    if (nyion_prefill_attention_bf16((const uint16_t*)a_q.ptr, (const uint16_t*)a_k.ptr, (const uint16_t*)a_v.ptr, n,
                                     hq, hkv, d, 1, 0.0f, (float*)a_o.ptr, nullptr, nullptr, nullptr, 16, 0,
                                     NYION_KV_F32, 0, nullptr))
        return fail("nyion_prefill_attention_bf16");
    if (nyion_sync()) return fail("sync");
    std::vector<float> got(q.size());
    if (nyion_hma_download(ar.h, got.data(), &a_o, got.size() * 4)) return fail("prefill download");
    std::vector<float> qf(q.size()), kf(k.size()), vf(v.size());
    for (size_t i = 0; i < q.size(); i++) qf[i] = bf16_value(q[i]);
    for (size_t i = 0; i < k.size(); i++) kf[i] = bf16_value(k[i]);
    for (size_t i = 0; i < v.size(); i++) vf[i] = bf16_value(v[i]);
    std::vector<double> ref(q.size());
    for (int r = 0; r < n; r++)
        for (int h = 0; h < hq; h++) {
            const int g = h / (hq / hkv);
            std::vector<const float*> kr, vr;
            for (int t = 0; t <= r; t++) {  // causal: keys [0, r]
                kr.push_back(&kf[((size_t)t * hkv + g) * d]);
                vr.push_back(&vf[((size_t)t * hkv + g) * d]);
            }
            attend(&qf[((size_t)r * hq + h) * d], kr, vr, d, &ref[((size_t)r * hq + h) * d]);
        }
    bad += report("prefill", got, ref);
    return 0;
}

// ------------------------------------------------------------------ GEMV

float f16_value(uint16_t h) {  // IEEE binary16 -> float (normal values)
    const uint32_t sign = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1f, m = h & 0x3ff;
    uint32_t x = sign;
    if (e) x |= ((e + 112) << 23) | (m << 13);
    float f;
    memcpy(&f, &x, 4);
    return f;
}

int run_gemv(Arena& ar, double& bad) {
    const int rows = 300, cols = 512, nb = cols / 256;
    Lcg rng(3);
    std::vector<uint8_t> w((size_t)rows * nb * 144);
    for (auto& b : w) b = (uint8_t)rng.next();
    for (size_t blk = 0; blk < (size_t)rows * nb; blk++) {  // normal, small d and dmin
        const uint16_t d = (uint16_t)(0x0c00 | (rng.next() & 0x3ff)), dm = (uint16_t)(0x0c00 | (rng.next() & 0x3ff));
        memcpy(&w[blk * 144], &d, 2);
        memcpy(&w[blk * 144 + 2], &dm, 2);
    }
    std::vector<float> x(cols);
    for (float& v : x) v = rng.uniform();
    nyion_allocation a_w, a_x, a_o;
    if (!ar.alloc(w.size(), a_w) || !ar.alloc(cols * 4, a_x) || !ar.alloc(rows * 4, a_o)) return fail("gemv arena");
    if (nyion_hma_upload(ar.h, &a_w, w.data(), w.size()) || nyion_hma_upload(ar.h, &a_x, x.data(), cols * 4))
        return fail("gemv upload");
    if (nyion_gemv_q4k((const uint8_t*)a_w.ptr, (const float*)a_x.ptr, (float*)a_o.ptr, rows, cols, nullptr))
        return fail("nyion_gemv_q4k");
    if (nyion_sync()) return fail("sync");
    std::vector<float> got(rows);
    if (nyion_hma_download(ar.h, got.data(), &a_o, rows * 4)) return fail("gemv download");
    std::vector<double> ref(rows, 0.0);
    for (int r = 0; r < rows; r++)
        for (int b = 0; b < nb; b++) {
            const uint8_t* blk = &w[((size_t)r * nb + b) * 144];
            uint16_t db, dmb;
            memcpy(&db, blk, 2);
            memcpy(&dmb, blk + 2, 2);
            const double dd = f16_value(db), dm = f16_value(dmb);
            const uint8_t* sc = blk + 4;
            for (int j = 0; j < 8; j++) {  // GGUF Q4_K 6-bit scale / min of sub-block j
                const int s = j < 4 ? (sc[j] & 63) : ((sc[j + 4] & 0xf) | ((sc[j - 4] >> 6) << 4));
                const int mn = j < 4 ? (sc[j + 4] & 63) : ((sc[j + 4] >> 4) | ((sc[j] >> 6) << 4));
                for (int i = 0; i < 32; i++) {
                    const uint8_t byte = blk[16 + 32 * (j / 2) + i];
                    const int qv = (j & 1) ? byte >> 4 : byte & 0xf;
                    ref[r] += (dd * s * qv - dm * mn) * x[(size_t)b * 256 + 32 * j + i];
                }
            }
        }
    bad += report("gemv_q4k", got, ref);
    return 0;
}

}  // namespace

int main() {
    if (nyion_init(0) != NYION_OK) {
        fprintf(stderr, "nyion_driver: no usable device: %s\n", nyion_last_error());
        return 3;
    }
    Arena ar;
    ar.h = nyion_hma_create((size_t)64 << 20, 0);
    if (!ar.h) return fail("nyion_hma_create");
    double bad = 0.0;
    int rc;
    if ((rc = run_decode(ar, bad)) || (rc = run_prefill(ar, bad)) || (rc = run_gemv(ar, bad))) return rc;
    if (bad > 0) {
        fprintf(stderr, "nyion_driver: mismatch\n");
        return 1;
    }
    printf("nyion_driver: all results within tolerance\n");
    return 0;
}
