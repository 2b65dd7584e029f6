// runtime.hip — error reporting, device selection and the HMA arena of
// libnyion_hip.so.
//
// The HMA arena follows the HeterogeneousMemoryAllocator contract
// (swamp-tensors/src/hma.rs:5-9 MemoryLocation, 30-36 Allocation, 215-221
// DeviceAllocator, 243-260 allocate): DeviceLocal memory comes from one
// hipMalloc region carved first-fit with 256-byte alignment (the paged KV
// pools and decode workspaces of one model live in it), HostPinned from one
// hipHostMalloc region, UnifiedMapped from hipMallocManaged per allocation.
// Without a device the arena behaves as the reference's allocator with no
// DeviceAllocator (hma.rs:243-260): the host region is ordinary memory and
// DeviceLocal / UnifiedMapped requests are served from it as host
// allocations (location HostPinned, no device handle).
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <map>
#include <mutex>
#include <string>

#include "arena.hpp"
#include "common.hpp"

namespace nyion {

static thread_local std::string t_err;

int set_error(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    t_err = buf;
    return code;
}

void clear_error() { t_err.clear(); }

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(NYION_ERR_LAUNCH, "%s launch: %s", what, hipGetErrorString(e));
    return NYION_OK;
}

static std::mutex g_dev_mu;
static std::map<int, int> g_dev_ok;  // device -> 1 ok, 0 not gfx950

int require_device() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) {
        (void)hipGetLastError();
        return set_error(NYION_ERR_NO_DEVICE, "no HIP device available");
    }
    {
        std::lock_guard<std::mutex> g(g_dev_mu);
        auto it = g_dev_ok.find(dev);
        if (it != g_dev_ok.end())
            return it->second ? NYION_OK
                              : set_error(NYION_ERR_NO_DEVICE, "device %d is not a gfx950", dev);
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) {
        (void)hipGetLastError();
        return set_error(NYION_ERR_NO_DEVICE, "hipGetDeviceProperties(%d) failed", dev);
    }
    const int ok = strncmp(prop.gcnArchName, "gfx950", 6) == 0;
    {
        std::lock_guard<std::mutex> g(g_dev_mu);
        g_dev_ok[dev] = ok;
    }
    return ok ? NYION_OK
              : set_error(NYION_ERR_NO_DEVICE, "device %d is %s, this library is built for gfx950",
                          dev, prop.gcnArchName);
}

// ------------------------------------------------------------- per device

int current_device() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();
        return -1;
    }
    return dev >= 0 && dev < kMaxDevices ? dev : -1;
}

int device_cu_count() {
    static std::atomic<int> cache[kMaxDevices];
    return per_device_value(
        cache,
        [] {
            int c = 0;
            if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, current_device()) !=
                hipSuccess) {
                (void)hipGetLastError();
                return 0;
            }
            return c;
        },
        256);
}

// Word 0: the sticky range flags (kRange* bits); word 1: where
// status_take_kernel leaves what it took.  Each device holds its own copy.
__device__ unsigned g_status_words[2];

unsigned* device_status_word() {
    static std::atomic<uintptr_t> cache[kMaxDevices];
    const int dev = current_device();
    if (dev < 0) return nullptr;
    uintptr_t v = cache[dev].load(std::memory_order_relaxed);
    if (v) return (unsigned*)v;
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_status_words)) != hipSuccess || !p) {
        (void)hipGetLastError();
        return nullptr;
    }
    cache[dev].store((uintptr_t)p, std::memory_order_relaxed);
    return (unsigned*)p;
}

__global__ void status_take_kernel(unsigned* w) {
    w[1] = __hip_atomic_exchange(&w[0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------- arena

struct Hma {
    std::mutex mu;
    int device = 0;
    bool no_device = false;  // host-only arena: device requests fall back to host
    Region dev, host;
    std::map<void*, size_t> managed;
};

// Bytes of the live allocation `a` names (0 if it names none).
static size_t live_bytes(Hma* h, const nyion_allocation* a) {
    if (a->location == NYION_MEM_DEVICE_LOCAL) return h->dev.live_size(a->ptr);
    if (a->location == NYION_MEM_HOST_PINNED) return h->host.live_size(a->ptr);
    if (a->location == NYION_MEM_UNIFIED_MAPPED) {
        auto it = h->managed.find(a->ptr);
        return it == h->managed.end() ? 0 : it->second;
    }
    return 0;
}

}  // namespace nyion

using namespace nyion;

extern "C" {

const char* nyion_last_error(void) { return t_err.c_str(); }

const char* nyion_version(void) { return "nyion-hip 0.1 (gfx950)"; }

int nyion_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n;
}

int nyion_init(int device) {
    clear_error();
    int n = nyion_device_count();
    if (device < 0 || device >= n)
        return set_error(NYION_ERR_NO_DEVICE, "device %d not present (%d devices)", device, n);
    NYION_CHECK_HIP(hipSetDevice(device));
    int rc;
    if ((rc = require_device()) != NYION_OK) return rc;
    // set-up of the device's scratch array (nyion_paged_decode_attention_noalloc)
    if (!decode_scratch_ptr()) return NYION_ERR_LAUNCH;
    // and of mojo_softmax_padic's exp table, so that later calls copy nothing
    return softmax_padic_setup();
}

int nyion_sync(void) {
    clear_error();
    NYION_CHECK_HIP(hipDeviceSynchronize());
    return NYION_OK;
}

int nyion_take_status(nyion_stream_t stream) {
    clear_error();
    int rc;
    if ((rc = require_device()) != NYION_OK) return rc;
    unsigned* w = device_status_word();
    if (!w) return set_error(NYION_ERR_LAUNCH, "status word of the current device is unavailable");
    hipStream_t st = (hipStream_t)stream;
    unsigned got = 0;
    {
        // word 1 carries one take's result back: takes on one device (from
        // any thread or stream) run one at a time, so each reads its own
        static std::mutex take_mu[kMaxDevices];
        std::lock_guard<std::mutex> g(take_mu[current_device()]);
        hipLaunchKernelGGL(status_take_kernel, dim3(1), dim3(1), 0, st, w);
        if ((rc = check_launch("status")) != NYION_OK) return rc;
        NYION_CHECK_HIP(hipMemcpyAsync(&got, w + 1, sizeof got, hipMemcpyDeviceToHost, st));
        NYION_CHECK_HIP(hipStreamSynchronize(st));
    }
    if (!got) return NYION_OK;
    std::string msg;
    if (got & kRangePrefillV)
        msg += "prefill: a V value of magnitude >= 65520 (or infinite) does not fit the binary16 "
               "operand of the P.V product; rows attending to it are not valid. ";
    if (got & kRangeDecodeQ)
        msg += "binary16 / Q4-20B KV decode: a q value of magnitude >= 65520 overflows the binary16 high "
               "part of q; the heads holding it are not valid. ";
    return set_error(NYION_ERR_RANGE, "%s", msg.c_str());
}

void* nyion_hma_create(size_t device_bytes, size_t host_pinned_bytes) {
    clear_error();
    Hma* h = new Hma();
    h->no_device = require_device() != NYION_OK;
    clear_error();
    if (!h->no_device) (void)hipGetDevice(&h->device);
    void* d = nullptr;
    void* p = nullptr;
    if (device_bytes && !h->no_device) {
        if (hipMalloc(&d, device_bytes) != hipSuccess) {
            (void)hipGetLastError();
            set_error(NYION_ERR_OOM, "hma: hipMalloc(%zu) failed", device_bytes);
            delete h;
            return nullptr;
        }
    }
    if (host_pinned_bytes) {
        const bool ok = h->no_device
                            ? (p = aligned_alloc(Region::kAlign, (host_pinned_bytes + Region::kAlign - 1) &
                                                                     ~(Region::kAlign - 1))) != nullptr
                            : hipHostMalloc(&p, host_pinned_bytes, hipHostMallocDefault) == hipSuccess;
        if (!ok) {
            if (!h->no_device) (void)hipGetLastError();
            if (d) (void)hipFree(d);
            set_error(NYION_ERR_OOM, "hma: host region of %zu bytes: allocation failed", host_pinned_bytes);
            delete h;
            return nullptr;
        }
    }
    h->dev.init(d, h->no_device ? 0 : device_bytes);
    h->host.init(p, host_pinned_bytes);
    return h;
}

int nyion_hma_alloc(void* hma, size_t size, int location, nyion_allocation* out) {
    clear_error();
    Hma* h = (Hma*)hma;
    if (!h || !out) return set_error(NYION_ERR_INVALID, "hma alloc: null handle/out");
    memset(out, 0, sizeof *out);
    if (location != NYION_MEM_DEVICE_LOCAL && location != NYION_MEM_HOST_PINNED &&
        location != NYION_MEM_UNIFIED_MAPPED)
        return set_error(NYION_ERR_INVALID, "hma alloc: location %d", location);
    std::lock_guard<std::mutex> g(h->mu);
    // no device: device requests are served by the host region (hma.rs:249-256)
    if (h->no_device) location = NYION_MEM_HOST_PINNED;
    void* p = nullptr;
    switch (location) {
        case NYION_MEM_DEVICE_LOCAL:
            p = h->dev.alloc(size);
            if (!p) return set_error(NYION_ERR_OOM, "hma: device arena exhausted (%zu requested, %zu/%zu used)",
                                     size, h->dev.used, h->dev.cap);
            out->device_handle = (uint64_t)(uintptr_t)p;
            break;
        case NYION_MEM_HOST_PINNED:
            p = h->host.alloc(size);
            if (!p) return set_error(NYION_ERR_OOM, "hma: host arena exhausted (%zu requested, %zu/%zu used)",
                                     size, h->host.used, h->host.cap);
            break;
        default:  // NYION_MEM_UNIFIED_MAPPED
            if (hipMallocManaged(&p, size ? size : 1) != hipSuccess) {
                (void)hipGetLastError();
                return set_error(NYION_ERR_OOM, "hma: hipMallocManaged(%zu) failed", size);
            }
            h->managed[p] = size;
            out->device_handle = (uint64_t)(uintptr_t)p;
            break;
    }
    out->ptr = p;
    out->size = size;
    out->location = location;
    return NYION_OK;
}

int nyion_hma_free(void* hma, const nyion_allocation* a) {
    clear_error();
    Hma* h = (Hma*)hma;
    if (!h || !a) return set_error(NYION_ERR_INVALID, "hma free: null handle/allocation");
    if (!a->ptr) return NYION_OK;
    std::lock_guard<std::mutex> g(h->mu);
    bool ok = false;
    if (a->location == NYION_MEM_DEVICE_LOCAL) ok = h->dev.release(a->ptr);
    else if (a->location == NYION_MEM_HOST_PINNED) ok = h->host.release(a->ptr);
    else if (a->location == NYION_MEM_UNIFIED_MAPPED) {
        auto it = h->managed.find(a->ptr);
        if (it != h->managed.end()) {
            (void)hipFree(a->ptr);
            h->managed.erase(it);
            ok = true;
        }
    }
    return ok ? NYION_OK : set_error(NYION_ERR_INVALID, "hma free: %p is not a live allocation", a->ptr);
}

// Host <-> allocation copies; host-region allocations are plain memcpy, the
// others synchronous hipMemcpy.  `bytes` may not exceed the live allocation.
static int hma_copy(void* hma, void* host, const nyion_allocation* a, size_t bytes, bool up) {
    clear_error();
    Hma* h = (Hma*)hma;
    const char* what = up ? "hma upload" : "hma download";
    if (!h || !a || !host || !a->ptr) return set_error(NYION_ERR_INVALID, "%s: null argument", what);
    size_t live;
    {
        std::lock_guard<std::mutex> g(h->mu);
        live = live_bytes(h, a);
    }
    if (live == 0) return set_error(NYION_ERR_INVALID, "%s: %p is not a live allocation", what, a->ptr);
    if (bytes > a->size || bytes > live)
        return set_error(NYION_ERR_INVALID, "%s: %zu bytes > allocation of %zu", what, bytes, a->size);
    if (a->location == NYION_MEM_HOST_PINNED) {
        if (up) memcpy(a->ptr, host, bytes);
        else memcpy(host, a->ptr, bytes);
        return NYION_OK;
    }
    if (up) NYION_CHECK_HIP(hipMemcpy(a->ptr, host, bytes, hipMemcpyHostToDevice));
    else NYION_CHECK_HIP(hipMemcpy(host, a->ptr, bytes, hipMemcpyDeviceToHost));
    return NYION_OK;
}

int nyion_hma_upload(void* hma, const nyion_allocation* dst, const void* src, size_t bytes) {
    return hma_copy(hma, (void*)src, dst, bytes, true);
}

int nyion_hma_download(void* hma, void* dst, const nyion_allocation* src, size_t bytes) {
    return hma_copy(hma, dst, src, bytes, false);
}

int nyion_hma_reset(void* hma) {
    clear_error();
    Hma* h = (Hma*)hma;
    if (!h) return set_error(NYION_ERR_INVALID, "hma reset: null handle");
    std::lock_guard<std::mutex> g(h->mu);
    h->dev.reset();
    h->host.reset();
    for (auto& kv : h->managed) (void)hipFree(kv.first);
    h->managed.clear();
    return NYION_OK;
}

int nyion_hma_stats(void* hma, int location, size_t* used, size_t* capacity) {
    clear_error();
    Hma* h = (Hma*)hma;
    if (!h) return set_error(NYION_ERR_INVALID, "hma stats: null handle");
    std::lock_guard<std::mutex> g(h->mu);
    size_t u = 0, c = 0;
    if (location == NYION_MEM_DEVICE_LOCAL) { u = h->dev.used; c = h->dev.cap; }
    else if (location == NYION_MEM_HOST_PINNED) { u = h->host.used; c = h->host.cap; }
    else if (location == NYION_MEM_UNIFIED_MAPPED) { for (auto& kv : h->managed) u += kv.second; c = u; }
    else return set_error(NYION_ERR_INVALID, "hma stats: location %d", location);
    if (used) *used = u;
    if (capacity) *capacity = c;
    return NYION_OK;
}

int nyion_hma_has_device(void* hma) {
    Hma* h = (Hma*)hma;
    return h && !h->no_device ? 1 : 0;
}

void nyion_hma_destroy(void* hma) {
    Hma* h = (Hma*)hma;
    if (!h) return;
    if (h->dev.base) (void)hipFree(h->dev.base);
    if (h->host.base) {
        if (h->no_device) free(h->host.base);
        else (void)hipHostFree(h->host.base);
    }
    for (auto& kv : h->managed) (void)hipFree(kv.first);
    delete h;
}

}  // extern "C"
