// runtime.hip — error reporting, device selection and the HMA arena of
// libnyion_hip.so.
//
// The HMA arena follows the HeterogeneousMemoryAllocator contract
// (swamp-tensors/src/hma.rs:5-9 MemoryLocation, 30-36 Allocation, 215-221
// DeviceAllocator, 243-260 allocate): DeviceLocal memory comes from one
// hipMalloc region carved first-fit with 256-byte alignment (the paged KV
// pools and decode workspaces of one model live in it), HostPinned from one
// hipHostMalloc region, UnifiedMapped from hipMallocManaged per allocation.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <map>
#include <mutex>
#include <string>

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

// ------------------------------------------------------------- arena

// First-fit free-list over one contiguous region.
struct Region {
    char* base = nullptr;
    size_t cap = 0;
    size_t used = 0;
    std::map<size_t, size_t> free_;  // offset -> size
    std::map<size_t, size_t> live;   // offset -> size

    void init(void* b, size_t c) {
        base = (char*)b;
        cap = c;
        used = 0;
        free_.clear();
        live.clear();
        if (c) free_[0] = c;
    }
    void* alloc(size_t size) {
        size = (size + 255) & ~(size_t)255;
        if (size == 0) size = 256;
        for (auto it = free_.begin(); it != free_.end(); ++it) {
            if (it->second >= size) {
                size_t off = it->first, rem = it->second - size;
                free_.erase(it);
                if (rem) free_[off + size] = rem;
                live[off] = size;
                used += size;
                return base + off;
            }
        }
        return nullptr;
    }
    bool release(void* p) {
        if (!base || (char*)p < base || (char*)p >= base + cap) return false;
        size_t off = (size_t)((char*)p - base);
        auto it = live.find(off);
        if (it == live.end()) return false;
        size_t size = it->second;
        live.erase(it);
        used -= size;
        auto nx = free_.lower_bound(off);
        if (nx != free_.end() && nx->first == off + size) {
            size += nx->second;
            free_.erase(nx);
        }
        auto pv = free_.lower_bound(off);
        if (pv != free_.begin()) {
            --pv;
            if (pv->first + pv->second == off) {
                pv->second += size;
                return true;
            }
        }
        free_[off] = size;
        return true;
    }
    void reset() { init(base, cap); }
};

struct Hma {
    std::mutex mu;
    int device = 0;
    Region dev, host;
    std::map<void*, size_t> managed;
};

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
    return require_device();
}

int nyion_sync(void) {
    clear_error();
    NYION_CHECK_HIP(hipDeviceSynchronize());
    return NYION_OK;
}

void* nyion_hma_create(size_t device_bytes, size_t host_pinned_bytes) {
    clear_error();
    if (device_bytes && require_device() != NYION_OK) return nullptr;
    Hma* h = new Hma();
    (void)hipGetDevice(&h->device);
    void* d = nullptr;
    void* p = nullptr;
    if (device_bytes) {
        if (hipMalloc(&d, device_bytes) != hipSuccess) {
            (void)hipGetLastError();
            set_error(NYION_ERR_OOM, "hma: hipMalloc(%zu) failed", device_bytes);
            delete h;
            return nullptr;
        }
    }
    if (host_pinned_bytes) {
        if (hipHostMalloc(&p, host_pinned_bytes, hipHostMallocDefault) != hipSuccess) {
            (void)hipGetLastError();
            if (d) (void)hipFree(d);
            set_error(NYION_ERR_OOM, "hma: hipHostMalloc(%zu) failed", host_pinned_bytes);
            delete h;
            return nullptr;
        }
    }
    h->dev.init(d, device_bytes);
    h->host.init(p, host_pinned_bytes);
    return h;
}

int nyion_hma_alloc(void* hma, size_t size, int location, nyion_allocation* out) {
    clear_error();
    Hma* h = (Hma*)hma;
    if (!h || !out) return set_error(NYION_ERR_INVALID, "hma alloc: null handle/out");
    memset(out, 0, sizeof *out);
    std::lock_guard<std::mutex> g(h->mu);
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
            if (!p) return set_error(NYION_ERR_OOM, "hma: pinned arena exhausted (%zu requested)", size);
            break;
        case NYION_MEM_UNIFIED_MAPPED:
            if (hipMallocManaged(&p, size ? size : 1) != hipSuccess) {
                (void)hipGetLastError();
                return set_error(NYION_ERR_OOM, "hma: hipMallocManaged(%zu) failed", size);
            }
            h->managed[p] = size;
            out->device_handle = (uint64_t)(uintptr_t)p;
            break;
        default:
            return set_error(NYION_ERR_INVALID, "hma alloc: location %d", location);
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

int nyion_hma_upload(void* hma, const nyion_allocation* dst, const void* src, size_t bytes) {
    clear_error();
    if (!hma || !dst || !src || !dst->ptr) return set_error(NYION_ERR_INVALID, "hma upload: null");
    if (bytes > dst->size) return set_error(NYION_ERR_INVALID, "hma upload: %zu > allocation %zu", bytes, dst->size);
    if (dst->location == NYION_MEM_HOST_PINNED) {
        memcpy(dst->ptr, src, bytes);
        return NYION_OK;
    }
    NYION_CHECK_HIP(hipMemcpy(dst->ptr, src, bytes, hipMemcpyHostToDevice));
    return NYION_OK;
}

int nyion_hma_download(void* hma, void* dst, const nyion_allocation* src, size_t bytes) {
    clear_error();
    if (!hma || !dst || !src || !src->ptr) return set_error(NYION_ERR_INVALID, "hma download: null");
    if (bytes > src->size) return set_error(NYION_ERR_INVALID, "hma download: %zu > allocation %zu", bytes, src->size);
    if (src->location == NYION_MEM_HOST_PINNED) {
        memcpy(dst, src->ptr, bytes);
        return NYION_OK;
    }
    NYION_CHECK_HIP(hipMemcpy(dst, src->ptr, bytes, hipMemcpyDeviceToHost));
    return NYION_OK;
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

void nyion_hma_destroy(void* hma) {
    Hma* h = (Hma*)hma;
    if (!h) return;
    if (h->dev.base) (void)hipFree(h->dev.base);
    if (h->host.base) (void)hipHostFree(h->host.base);
    for (auto& kv : h->managed) (void)hipFree(kv.first);
    delete h;
}

}  // extern "C"
