// mojo_ffi.hip — the Mojo kernel library's sparse_attention_q4 symbol
// (swamp-gpu/src/mojo.rs:5,38 loads it from libswamp_mojo.so by name;
// semantics swamp-gpu/kernels/attention.mojo:38-152).
//
// The reference routine is a CPU kernel over host memory: every head of q
// against one K/V given as rows of f32 words (per 32-element block: d, dmin,
// then the 16 nibble bytes as float values), over an explicit position list
// walked in tiles of 64 whose weights are normalised by the running
// denominator of the tiles seen so far (earlier tiles are not rescaled), with
// weights below 1e-8 skipped.  Here the same arithmetic runs on the device:
// the call copies q, the positions and the K/V rows up to the largest listed
// position to device buffers (a per-device staging array of kMojoStage
// words, under a lock; a call that needs more allocates its buffers for the
// call), runs one wavefront per head
// (lane p scores tile position p; lane i accumulates output elements i,
// i + 64, ... over the tile's positions in list order, as the reference's
// loop does), and copies the output back.  It is not a hot path: the
// reference has no caller of it.
#include <math.h>

#include <mutex>
#include <vector>

#include "common.hpp"

// Staging for sparse_attention_q4's host arrays (q, out, K and V rows,
// positions): 16 MiB of 4-byte words, one copy per device (the name is a
// host-side stand-in: mojo_stage_ptr() looks its device address up once per
// device).
constexpr size_t kMojoStage = (size_t)1 << 22;
static __device__ __align__(256) float mojo_stage[kMojoStage];

namespace nyion {

// Device address of this device's staging array and the lock that
// serialises its users (the call is synchronous).
static float* mojo_stage_ptr(std::mutex** lock) {
    static std::atomic<uintptr_t> cache[kMaxDevices];
    static std::mutex locks[kMaxDevices];
    const int dev = current_device();
    if (dev < 0) return nullptr;
    *lock = &locks[dev];
    uintptr_t v = cache[dev].load(std::memory_order_relaxed);
    if (v) return (float*)v;
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(mojo_stage));
    if (e != hipSuccess || !ptr) {
        (void)hipGetLastError();
        set_error(NYION_ERR_LAUNCH, "sparse_attention_q4: hipGetSymbolAddress failed: %s",
                  hipGetErrorString(e));
        return nullptr;
    }
    cache[dev].store((uintptr_t)ptr, std::memory_order_relaxed);
    return (float*)ptr;
}

// Element i of a row of f32 words (attention.mojo:74-83): the word holding
// its byte is read as an integer, low nibble for even i.
__device__ __forceinline__ float mojo_elem(const float* row, int i) {
    const float* blk = row + (i / 32) * 20;
    const int e = i % 32;
    const int byte = (int)blk[2 + e / 2];
    const int nib = (byte >> ((e % 2) * 4)) & 0x0F;
    return __fadd_rn(__fmul_rn(blk[0], (float)nib), blk[1]);
}

__global__ __launch_bounds__(64) void mojo_sparse_kernel(const float* q, const float* k, const float* v,
                                                         const int32_t* positions, float* out,
                                                         int head_dim, int n_sparse, float scale) {
    __shared__ float sw[64];
    __shared__ float se[64];
    const int lane = threadIdx.x;
    const int blocks = (head_dim + 31) / 32;
    const long long row = (long long)blocks * 20;
    const float* qh = q + (long long)blockIdx.x * head_dim;
    float* oh = out + (long long)blockIdx.x * head_dim;
    constexpr int kMaxOut = 16;  // output elements per lane: head_dim <= 1024
    float acc[kMaxOut];
#pragma unroll
    for (int u = 0; u < kMaxOut; u++) acc[u] = 0.f;
    float m = -1e10f, d = 0.f;
    for (int t0 = 0; t0 < n_sparse; t0 += 64) {
        const int nt = min(64, n_sparse - t0);
        float sc = -1e10f;
        if (lane < nt) {
            const float* kr = k + positions[t0 + lane] * row;
            float dot = 0.f;
            for (int i = 0; i < head_dim; i++) dot = __fadd_rn(dot, __fmul_rn(mojo_elem(kr, i), qh[i]));
            sc = __fmul_rn(dot, scale);
        }
        float tmax = sc;  // the tile max (order-free)
        for (int o = 32; o > 0; o >>= 1) tmax = fmaxf(tmax, __shfl_xor(tmax, o));
        tmax = fmaxf(tmax, -1e10f);
        se[lane] = lane < nt ? expf(sc - tmax) : 0.f;
        __syncthreads();
        float tsum = 0.f;  // in list order, as the reference sums
        for (int p = 0; p < nt; p++) tsum = __fadd_rn(tsum, se[p]);
        const float nm = fmaxf(m, tmax);
        d = __fadd_rn(__fmul_rn(d, expf(m - nm)), __fmul_rn(tsum, expf(tmax - nm)));
        m = nm;
        sw[lane] = lane < nt ? expf(sc - m) / d : 0.f;
        __syncthreads();
        for (int p = 0; p < nt; p++) {
            const float w = sw[p];
            if (w < 1e-8f) continue;  // uniform: every lane reads the same w
            const float* vr = v + positions[t0 + p] * row;
#pragma unroll
            for (int u = 0; u < kMaxOut; u++) {
                const int i = lane + 64 * u;
                if (i < head_dim) acc[u] = __fadd_rn(acc[u], __fmul_rn(mojo_elem(vr, i), w));
            }
        }
        __syncthreads();  // se / sw are rewritten by the next tile
    }
#pragma unroll
    for (int u = 0; u < kMaxOut; u++) {
        const int i = lane + 64 * u;
        if (i < head_dim) oh[i] = acc[u];
    }
}

// Device buffers of one call, freed on every return path.
struct CallBuffers {
    std::vector<void*> ptrs;
    ~CallBuffers() {
        for (void* p : ptrs) (void)hipFree(p);
    }
    int alloc(void** p, size_t bytes) {
        if (hipMalloc(p, bytes) != hipSuccess) {
            (void)hipGetLastError();
            *p = nullptr;
            return set_error(NYION_ERR_OOM, "sparse_attention_q4: hipMalloc(%zu) failed", bytes);
        }
        ptrs.push_back(*p);
        return NYION_OK;
    }
};

static int mojo_sparse_impl(const float* q, const float* k_q4, const float* v_q4,
                            const int32_t* positions, float* out, int n_heads, int head_dim,
                            int n_sparse) {
    clear_error();
    int rc;
    if ((rc = require_device()) != NYION_OK) return rc;
    if (!q || !out || n_heads <= 0 || head_dim <= 0 || n_sparse < 0)
        return set_error(NYION_ERR_INVALID, "sparse_attention_q4: null q/out or non-positive size");
    if (head_dim > 1024)
        return set_error(NYION_ERR_UNSUPPORTED, "sparse_attention_q4: head_dim %d > 1024", head_dim);
    if (n_sparse > 0 && (!k_q4 || !v_q4 || !positions))
        return set_error(NYION_ERR_INVALID, "sparse_attention_q4: null k/v/positions");
    int max_pos = -1;
    for (int i = 0; i < n_sparse; i++) {
        if (positions[i] < 0)
            return set_error(NYION_ERR_INVALID, "sparse_attention_q4: position %d at index %d",
                             positions[i], i);
        max_pos = positions[i] > max_pos ? positions[i] : max_pos;
    }
    const size_t row_bytes = (size_t)((head_dim + 31) / 32) * 20 * sizeof(float);
    const size_t q_bytes = (size_t)n_heads * head_dim * sizeof(float);
    // rows 0..max_pos of K and of V are read; at most 2^31 positions, and the
    // pair must fit in device memory (checked by the allocation below)
    const size_t kv_bytes = n_sparse > 0 ? ((size_t)max_pos + 1) * row_bytes : 0;
    if (kv_bytes > ((size_t)1 << 36))
        return set_error(NYION_ERR_INVALID,
                         "sparse_attention_q4: position %d needs %zu bytes of K rows (limit 64 GiB)",
                         max_pos, kv_bytes);
    const size_t pos_bytes = (size_t)n_sparse * sizeof(int32_t);
    // the five arrays in 256-byte aligned pieces of the staging array when
    // they fit it, else in buffers allocated for the call
    auto up = [](size_t b) { return (b + 255) & ~(size_t)255; };
    const size_t stage_need = 2 * up(q_bytes) + 2 * up(kv_bytes) + up(pos_bytes);
    std::mutex* lock = nullptr;
    char* stage = stage_need <= kMojoStage * sizeof(float) ? (char*)mojo_stage_ptr(&lock) : nullptr;
    if (stage_need <= kMojoStage * sizeof(float) && !stage) return NYION_ERR_LAUNCH;
    std::unique_lock<std::mutex> held;
    if (lock) held = std::unique_lock<std::mutex>(*lock);
    CallBuffers buf;
    void *dq = nullptr, *dout = nullptr, *dk = nullptr, *dv = nullptr, *dpos = nullptr;
    if (stage) {
        dq = stage;
        dout = stage + up(q_bytes);
        dk = stage + 2 * up(q_bytes);
        dv = stage + 2 * up(q_bytes) + up(kv_bytes);
        dpos = stage + 2 * up(q_bytes) + 2 * up(kv_bytes);
    } else if ((rc = buf.alloc(&dq, q_bytes)) != NYION_OK || (rc = buf.alloc(&dout, q_bytes)) != NYION_OK ||
               (n_sparse > 0 && ((rc = buf.alloc(&dk, kv_bytes)) != NYION_OK ||
                                 (rc = buf.alloc(&dv, kv_bytes)) != NYION_OK ||
                                 (rc = buf.alloc(&dpos, pos_bytes)) != NYION_OK))) {
        return rc;
    }
    NYION_CHECK_HIP(hipMemcpy(dq, q, q_bytes, hipMemcpyHostToDevice));
    if (n_sparse > 0) {
        NYION_CHECK_HIP(hipMemcpy(dk, k_q4, kv_bytes, hipMemcpyHostToDevice));
        NYION_CHECK_HIP(hipMemcpy(dv, v_q4, kv_bytes, hipMemcpyHostToDevice));
        NYION_CHECK_HIP(hipMemcpy(dpos, positions, pos_bytes, hipMemcpyHostToDevice));
    }
    const float scale = 1.0f / sqrtf((float)head_dim);
    hipLaunchKernelGGL(mojo_sparse_kernel, dim3((unsigned)n_heads), dim3(64), 0, nullptr, (const float*)dq,
                       (const float*)dk, (const float*)dv, (const int32_t*)dpos, (float*)dout, head_dim,
                       n_sparse, scale);
    if ((rc = check_launch("sparse_attention_q4")) != NYION_OK) return rc;
    NYION_CHECK_HIP(hipMemcpy(out, dout, q_bytes, hipMemcpyDeviceToHost));
    return NYION_OK;
}

}  // namespace nyion

using namespace nyion;

extern "C" {

void sparse_attention_q4(uint64_t q, uint64_t k_q4, uint64_t v_q4, uint64_t positions, uint64_t out,
                         int n_heads, int head_dim, int n_sparse, int window, int global_stride) {
    (void)window;  // accepted and unused, as by the reference kernel
    (void)global_stride;
    (void)mojo_sparse_impl((const float*)(uintptr_t)q, (const float*)(uintptr_t)k_q4,
                           (const float*)(uintptr_t)v_q4, (const int32_t*)(uintptr_t)positions,
                           (float*)(uintptr_t)out, n_heads, head_dim, n_sparse);
}

}  // extern "C"
