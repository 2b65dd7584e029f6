// arena.hpp — first-fit free list over one contiguous region (host code
// only; the HMA arena of runtime.hip carves its DeviceLocal and HostPinned
// regions with it).  Allocation sizes are rounded up to 256 bytes, so with a
// 256-byte aligned base every allocation is 256-byte aligned; a release
// merges the freed range with free neighbours on both sides.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <map>

namespace nyion {

struct Region {
    char* base = nullptr;
    size_t cap = 0;
    size_t used = 0;
    std::map<size_t, size_t> free_;  // offset -> size, no two adjacent
    std::map<size_t, size_t> live;   // offset -> size

    static constexpr size_t kAlign = 256;

    void init(void* b, size_t c) {
        base = (char*)b;
        cap = c;
        used = 0;
        free_.clear();
        live.clear();
        if (cap) free_[0] = cap;
    }
    // nullptr when no free range holds `size` (rounded up to 256 bytes; a
    // zero-byte request takes 256).  Sizes so large that rounding them up
    // would wrap are refused.
    void* alloc(size_t size) {
        if (size > cap) return nullptr;
        size = (size + kAlign - 1) & ~(kAlign - 1);
        if (size == 0) size = kAlign;
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
    // false when p is not the start of a live allocation of this region
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
    // size of a live allocation starting at p (0 if none)
    size_t live_size(const void* p) const {
        if (!base || (const char*)p < base) return 0;
        auto it = live.find((size_t)((const char*)p - base));
        return it == live.end() ? 0 : it->second;
    }
};

}  // namespace nyion
