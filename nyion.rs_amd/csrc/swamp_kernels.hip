// swamp_kernels.hip — the swamp-kernels C-ABI (swamp-kernels/src/lib.rs)
// on the MI355X: mojo_softmax_padic and the Stokes score-evicting KV buffer.
//
// mojo_softmax_padic (lib.rs:181-223) follows the reference's AVX-512 branch
// (lib.rs:110-179), the one x86-64 AVX-512 hosts execute:
//   fixed_i = sat_i32((x_i * (1/max(T,1e-6))) * 65536)     (Rust `as i32`)
//   m = max fixed_i;  e_i = exp_q16_16(fixed_i - m)          (wrapping sub)
//   exp_q16_16(x) = 0 if x < -655360; 65536 if x >= 0;
//                   else sat_i32(max(round(expf(x/65536) * 65536), 0))
//   S = sum e_i (i64); inv = (i32)(2^32 / S)
//   p_i = (u32)(e_i * inv) >> 16   for i < 16*floor(n/16)   (vector lanes)
//   p_i = (i32)((i64)e_i * inv >> 16) for the tail            (scalar lanes)
//   probs_i = p_i / 65536
// exp_q16_16 takes one of 655360 negative inputs, so its values are a table:
// each device holds round(expf(x / 65536) * 65536) for x in [-655360, -1],
// computed once by the host with the C library's expf (the function the
// reference's f32::exp calls), which makes the whole pipeline integer-exact.
//
// StokesKVCacheSim (lib.rs:27-85): keys and values live in device memory,
// one slot per resident token; the host keeps the logical order and the
// scores (a few KB) and picks the victim when the count passes 4096: the
// first minimum score, as Iterator::min_by does.  Slots are reused, data
// never moves.
#include <limits.h>
#include <math.h>
#include <string.h>

#include <mutex>
#include <vector>

#include "common.hpp"

// Staging for mojo_softmax_padic's host arrays: logits and probabilities of
// up to kSoftmaxStage elements, one copy per device (the name is a host-side
// stand-in: softmax_stage_ptr() looks its device address up once per device).
constexpr int kSoftmaxStage = 1 << 20;
static __device__ __align__(256) float softmax_stage[2 * kSoftmaxStage];

// exp_q16_16 of x = -1 - i at index i (2.5 MiB per device; the name is a
// host-side stand-in: exp_table_ptr() looks its address up and fills it once
// per device).
constexpr int kExpEntries = 655360;
static __device__ __align__(256) int32_t exp_q16_table[kExpEntries];

namespace nyion {

// Device address of this device's staging array and the lock that
// serialises its users (the host-pointer call is synchronous).
static float* softmax_stage_ptr(std::mutex** lock) {
    static std::atomic<uintptr_t> cache[kMaxDevices];
    static std::mutex locks[kMaxDevices];
    const int dev = current_device();
    if (dev < 0) return nullptr;
    *lock = &locks[dev];
    uintptr_t v = cache[dev].load(std::memory_order_relaxed);
    if (v) return (float*)v;
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(softmax_stage));
    if (e != hipSuccess || !ptr) {
        (void)hipGetLastError();
        set_error(NYION_ERR_LAUNCH, "mojo_softmax_padic: hipGetSymbolAddress failed: %s",
                  hipGetErrorString(e));
        return nullptr;
    }
    cache[dev].store((uintptr_t)ptr, std::memory_order_relaxed);
    return (float*)ptr;
}

__device__ __forceinline__ int32_t sat_i32(float x) {
    if (x != x) return 0;
    if (x >= 2147483648.0f) return INT_MAX;
    if (x <= -2147483648.0f) return INT_MIN;
    return (int32_t)x;
}

// Host side of exp_q16_16 (swamp-kernels/src/lib.rs:102-108) for x in
// [-655360, -1]: x as f32 / 65536 (exact), expf, times 65536 (exact),
// rounded half away from zero (f32::round), max 0, as i32.
static int32_t exp_q16_16_host(int32_t x) {
    const float e = expf((float)x / 65536.0f);
    const float r = fmaxf(roundf(e * 65536.0f), 0.0f);
    return (int32_t)r;
}

// Device address of this device's exp table, filled by the first caller on
// the device (synchronous copy); nullptr with the error set on failure.
static const int32_t* exp_table_ptr() {
    static std::atomic<uintptr_t> cache[kMaxDevices];
    static std::mutex locks[kMaxDevices];
    const int dev = current_device();
    if (dev < 0) return nullptr;
    uintptr_t v = cache[dev].load(std::memory_order_acquire);
    if (v) return (const int32_t*)v;
    std::lock_guard<std::mutex> g(locks[dev]);
    v = cache[dev].load(std::memory_order_acquire);
    if (v) return (const int32_t*)v;
    void* ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(exp_q16_table));
    if (e == hipSuccess && ptr) {
        std::vector<int32_t> t(kExpEntries);
        for (int i = 0; i < kExpEntries; i++) t[i] = exp_q16_16_host(-1 - i);
        e = hipMemcpy(ptr, t.data(), sizeof(int32_t) * kExpEntries, hipMemcpyHostToDevice);
    }
    if (e != hipSuccess || !ptr) {
        (void)hipGetLastError();
        set_error(NYION_ERR_LAUNCH, "softmax_padic: exp table set-up failed: %s", hipGetErrorString(e));
        return nullptr;
    }
    cache[dev].store((uintptr_t)ptr, std::memory_order_release);
    return (const int32_t*)ptr;
}

__device__ __forceinline__ int32_t exp_q16_16(const int32_t* table, int32_t x) {
    if (x < -655360) return 0;
    if (x >= 0) return 65536;
    return table[-1 - x];
}

// One workgroup of 1024 threads; e_i is kept in `probs` (as bits) between
// the passes.
__global__ __launch_bounds__(1024) void softmax_padic_kernel(const float* logits, float* probs,
                                                             int n, float inv_tmp,
                                                             const int32_t* exp_table) {
    __shared__ int32_t smax[16];
    __shared__ long long ssum[16];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;

    int32_t mx = INT_MIN;
    for (int i = tid; i < n; i += 1024) mx = max(mx, sat_i32((logits[i] * inv_tmp) * 65536.0f));
    for (int o = 32; o > 0; o >>= 1) mx = max(mx, __shfl_xor(mx, o));
    if (lane == 0) smax[wave] = mx;
    __syncthreads();
    mx = smax[0];
    for (int w = 1; w < 16; w++) mx = max(mx, smax[w]);

    long long sum = 0;
    for (int i = tid; i < n; i += 1024) {
        const int32_t f = sat_i32((logits[i] * inv_tmp) * 65536.0f);
        const int32_t e = exp_q16_16(exp_table, (int32_t)((uint32_t)f - (uint32_t)mx));
        ((int32_t*)probs)[i] = e;
        sum += e;
    }
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
    if (lane == 0) ssum[wave] = sum;
    __syncthreads();
    sum = 0;
    for (int w = 0; w < 16; w++) sum += ssum[w];

    const int simd_end = (n / 16) * 16;
    const int32_t inv = sum > 0 ? (int32_t)(uint32_t)((1ull << 32) / (unsigned long long)sum) : 0;
    for (int i = tid; i < n; i += 1024) {
        int32_t e = ((const int32_t*)probs)[i];
        if (sum > 0) {
            if (i < simd_end)
                e = (int32_t)(((uint32_t)e * (uint32_t)inv) >> 16);
            else
                e = (int32_t)(((long long)e * (long long)inv) >> 16);
        }
        probs[i] = (float)e / 65536.0f;
    }
}

struct Stokes {
    int head_dim = 0;
    int device = 0;
    float* d_keys = nullptr;    // [kSlots][head_dim]
    float* d_values = nullptr;  // [kSlots][head_dim]
    std::vector<float> scores;  // logical order
    std::vector<int> slot;      // logical order -> device slot
    std::vector<int> free_slots;
    static constexpr int kLimit = 4096;
    static constexpr int kSlots = kLimit + 1;
};

__global__ void stokes_gather_kernel(const float* src, const int* slots, int count, int hd, float* dst) {
    const long long n = (long long)count * hd;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n;
         i += (long long)gridDim.x * blockDim.x) {
        const int t = (int)(i / hd), e = (int)(i % hd);
        dst[i] = src[(long long)slots[t] * hd + e];
    }
}

}  // namespace nyion

namespace nyion {
// Set-up of the current device's exp table (called by nyion_init).
int softmax_padic_setup() { return exp_table_ptr() ? NYION_OK : NYION_ERR_LAUNCH; }
}  // namespace nyion

using namespace nyion;

extern "C" {

int nyion_softmax_padic_dev(const float* d_logits, float* d_probs, int n, float temperature,
                            nyion_stream_t stream) {
    clear_error();
    int rc;
    if ((rc = require_device()) != NYION_OK) return rc;
    if (!d_logits || !d_probs || n <= 0)
        return set_error(NYION_ERR_INVALID, "softmax_padic: null pointer or n <= 0");
    const int32_t* table = exp_table_ptr();
    if (!table) return NYION_ERR_LAUNCH;
    const float inv_tmp = 1.0f / fmaxf(temperature, 1e-6f);
    hipLaunchKernelGGL(softmax_padic_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, d_logits,
                       d_probs, n, inv_tmp, table);
    return check_launch("softmax_padic");
}

void mojo_softmax_padic(const float* logits, float* probs, int n, float temperature) {
    if (!logits || !probs || n <= 0) return;
    clear_error();
    if (require_device() != NYION_OK) return;
    // up to kSoftmaxStage logits go through the device's staging array;
    // longer arrays through device memory allocated for the call
    std::mutex* lock = nullptr;
    float* stage = n <= kSoftmaxStage ? softmax_stage_ptr(&lock) : nullptr;
    if (n <= kSoftmaxStage && !stage) return;
    std::unique_lock<std::mutex> held;
    if (lock) held = std::unique_lock<std::mutex>(*lock);
    float* d = stage;
    if (!d && hipMalloc(&d, 2 * (size_t)n * sizeof(float)) != hipSuccess) {
        (void)hipGetLastError();
        set_error(NYION_ERR_OOM, "mojo_softmax_padic: hipMalloc failed");
        return;
    }
    float* dl = d;
    float* dp = d + (stage ? kSoftmaxStage : n);
    const bool ok = hipMemcpy(dl, logits, (size_t)n * sizeof(float), hipMemcpyDefault) == hipSuccess &&
                    nyion_softmax_padic_dev(dl, dp, n, temperature, nullptr) == NYION_OK &&
                    hipMemcpy(probs, dp, (size_t)n * sizeof(float), hipMemcpyDefault) == hipSuccess;
    if (!ok) {
        (void)hipGetLastError();
        if (nyion_last_error()[0] == 0) set_error(NYION_ERR_LAUNCH, "mojo_softmax_padic: HIP copy failed");
    }
    if (!stage) (void)hipFree(d);
}

void* mojo_stokes_init(int head_dim) {
    clear_error();
    if (require_device() != NYION_OK) return nullptr;
    Stokes* c = new Stokes();
    c->head_dim = head_dim > 0 ? head_dim : 0;
    (void)hipGetDevice(&c->device);
    if (c->head_dim) {
        const size_t bytes = (size_t)Stokes::kSlots * c->head_dim * sizeof(float);
        if (hipMalloc(&c->d_keys, bytes) != hipSuccess || hipMalloc(&c->d_values, bytes) != hipSuccess) {
            (void)hipGetLastError();
            if (c->d_keys) (void)hipFree(c->d_keys);
            delete c;
            set_error(NYION_ERR_OOM, "mojo_stokes_init: hipMalloc failed");
            return nullptr;
        }
    }
    for (int s = Stokes::kSlots - 1; s >= 0; s--) c->free_slots.push_back(s);
    return c;
}

void mojo_stokes_free(void* cache) {
    Stokes* c = (Stokes*)cache;
    if (!c) return;
    if (c->d_keys) (void)hipFree(c->d_keys);
    if (c->d_values) (void)hipFree(c->d_values);
    delete c;
}

void mojo_stokes_append(void* cache, int token_id, const float* key, const float* value, float score) {
    (void)token_id;
    Stokes* c = (Stokes*)cache;
    if (!c || !key || !value) return;
    clear_error();
    if (c->free_slots.empty()) {  // only after NaN scores blocked eviction
        set_error(NYION_ERR_INVALID, "mojo_stokes_append: cache full (NaN scores block eviction)");
        return;
    }
    const int s = c->free_slots.back();
    if (c->head_dim) {
        const size_t row = (size_t)c->head_dim * sizeof(float);
        if (hipMemcpy(c->d_keys + (size_t)s * c->head_dim, key, row, hipMemcpyDefault) != hipSuccess ||
            hipMemcpy(c->d_values + (size_t)s * c->head_dim, value, row, hipMemcpyDefault) != hipSuccess) {
            (void)hipGetLastError();
            set_error(NYION_ERR_LAUNCH, "mojo_stokes_append: copy failed");
            return;
        }
    }
    c->free_slots.pop_back();
    c->slot.push_back(s);
    c->scores.push_back(score);
    if ((int)c->scores.size() > Stokes::kLimit) {
        for (float v : c->scores)
            if (v != v) {  // the reference panics on a NaN comparison (partial_cmp().unwrap())
                set_error(NYION_ERR_INVALID, "mojo_stokes_append: NaN score, eviction skipped");
                return;
            }
        size_t mi = 0;
        for (size_t i = 1; i < c->scores.size(); i++)
            if (c->scores[i] < c->scores[mi]) mi = i;
        c->free_slots.push_back(c->slot[mi]);
        c->slot.erase(c->slot.begin() + (long)mi);
        c->scores.erase(c->scores.begin() + (long)mi);
    }
}

int nyion_stokes_count(const void* cache) {
    const Stokes* c = (const Stokes*)cache;
    return c ? (int)c->scores.size() : 0;
}

int nyion_stokes_read(const void* cache, float* keys, float* values, float* scores) {
    clear_error();
    const Stokes* c = (const Stokes*)cache;
    if (!c) return set_error(NYION_ERR_INVALID, "stokes read: null cache");
    const int n = (int)c->scores.size();
    if (scores) memcpy(scores, c->scores.data(), sizeof(float) * (size_t)n);
    if (n == 0 || c->head_dim == 0 || (!keys && !values)) return n;
    int* d_slots = nullptr;
    float* d_tmp = nullptr;
    const size_t bytes = (size_t)n * c->head_dim * sizeof(float);
    NYION_CHECK_HIP(hipMalloc(&d_slots, sizeof(int) * (size_t)n));
    if (hipMalloc(&d_tmp, bytes) != hipSuccess) {
        (void)hipGetLastError();
        (void)hipFree(d_slots);
        return set_error(NYION_ERR_OOM, "stokes read: hipMalloc failed");
    }
    int rc = NYION_OK;
    if (hipMemcpy(d_slots, c->slot.data(), sizeof(int) * (size_t)n, hipMemcpyHostToDevice) != hipSuccess)
        rc = set_error(NYION_ERR_LAUNCH, "stokes read: copy failed");
    const float* srcs[2] = {c->d_keys, c->d_values};
    float* dsts[2] = {keys, values};
    for (int w = 0; w < 2 && rc == NYION_OK; w++) {
        if (!dsts[w]) continue;
        hipLaunchKernelGGL(stokes_gather_kernel, dim3(256), dim3(256), 0, nullptr, srcs[w], d_slots, n,
                           c->head_dim, d_tmp);
        if ((rc = check_launch("stokes gather")) != NYION_OK) break;
        if (hipMemcpy(dsts[w], d_tmp, bytes, hipMemcpyDeviceToHost) != hipSuccess)
            rc = set_error(NYION_ERR_LAUNCH, "stokes read: copy failed");
    }
    (void)hipGetLastError();
    (void)hipFree(d_slots);
    (void)hipFree(d_tmp);
    return rc == NYION_OK ? n : rc;
}

}  // extern "C"
