// page_policy.hpp — the PagedKVCache page policy (host code only; the
// device-resident pool of kv_pool.hip turns its events into copy kernels).
// Restated from swamp-engine/src/cache.rs (lines cited per method).
#pragma once

#include <vector>

#include "host_status.hpp"

namespace nyion {

class PagePolicy {
public:
    enum State { kUnmapped = 0, kHot = 1, kCold = 2 };

    PagePolicy(int hot_limit, int cold_slots, int max_pages)
        : hot_limit_(hot_limit), cold_slots_(cold_slots), max_pages_(max_pages),
          state_(max_pages, kUnmapped), where_(max_pages, -1), prev_(max_pages, -1),
          next_(max_pages, -1), importance_(max_pages, 0.0), slot_used_(cold_slots, 0) {
        for (int b = hot_limit - 1; b >= 0; b--) free_blocks_.push_back(b);
    }

    // Pages [lo, hi] are not eviction candidates while a range is made hot
    // (hi < lo: none).
    void protect(int lo, int hi) {
        prot_lo_ = lo;
        prot_hi_ = hi;
    }

    // cache.rs:525-546 (ensure_page): pages are created in order up to p
    // (each creation evicting first when the hot tier is full), a cold page
    // is reloaded, and p becomes the most recently used.
    int ensure(int p, std::vector<nyion_page_event>& ev) {
        if (p < 0 || p >= max_pages_) return set_error(NYION_ERR_INVALID, "page %d of %d", p, max_pages_);
        int rc;
        while (p >= n_created_) {
            if (hot_count_ >= hot_limit_ && (rc = evict_one(ev)) != NYION_OK) return rc;
            if ((rc = create(ev)) != NYION_OK) return rc;
        }
        if (state_[p] == kCold && (rc = reload(p, ev)) != NYION_OK) return rc;
        touch(p);
        return NYION_OK;
    }

    // cache.rs:563-571: only created pages accumulate importance
    void record(int p, double w) {
        if (p >= 0 && p < n_created_) importance_[p] += w;
    }
    void reset() {  // cache.rs:573-580
        for (double& v : importance_) v = 0.0;
    }
    int state(int p, int* where, double* importance) const {
        if (p < 0 || p >= max_pages_) return -1;
        if (where) *where = where_[p];
        if (importance) *importance = importance_[p];
        return state_[p];
    }
    int hot_limit() const { return hot_limit_; }
    int max_pages() const { return max_pages_; }
    long long hot_count() const { return hot_count_; }
    long long cold_count() const { return cold_count_; }
    long long evictions() const { return evictions_; }
    long long reloads() const { return reloads_; }
    // most recently used first
    int lru_order(int* out, int cap) const {
        int n = 0;
        for (int p = head_; p >= 0 && n < cap; p = next_[p]) out[n++] = p;
        return n;
    }

private:
    // cache.rs:277-309: a new page is hot, zeroed, at the LRU head
    int create(std::vector<nyion_page_event>& ev) {
        if (free_blocks_.empty())
            return set_error(NYION_ERR_OOM, "kv pool: no free block for page %d (cold tier full?)",
                             n_created_);
        const int p = n_created_++;
        const int b = free_blocks_.back();
        free_blocks_.pop_back();
        state_[p] = kHot;
        where_[p] = b;
        importance_[p] = 0.0;
        hot_count_++;
        push_head(p);
        ev.push_back(nyion_page_event{NYION_PAGE_CREATE, p, b, -1});
        return NYION_OK;
    }

    // cache.rs:407-477: among the LRU tail and up to seven pages before it,
    // evict the one with the lowest importance (the first found on ties),
    // into the first free cold slot at or after the write cursor.  Pages of
    // the range being made hot are skipped (they do not count among the
    // eight): the reference would evict them and then read a missing page.
    int evict_one(std::vector<nyion_page_event>& ev) {
        if (tail_ < 0) return NYION_OK;
        int best = -1, seen = 0;
        double best_imp = 0.0;
        for (int cur = tail_; cur >= 0 && seen < 8; cur = prev_[cur]) {
            if (cur >= prot_lo_ && cur <= prot_hi_) continue;
            if (best < 0 || importance_[cur] < best_imp) {
                best_imp = importance_[cur];
                best = cur;
            }
            seen++;
        }
        if (best < 0)
            return set_error(NYION_ERR_INVALID, "kv pool: every hot page is in the range being made hot");
        int slot = -1;
        for (int i = 0; i < cold_slots_; i++) {
            const int s = (cursor_ + i) % cold_slots_;
            if (!slot_used_[s]) {
                slot = s;
                break;
            }
        }
        // the reference overwrites the slot at its cursor when every slot is
        // taken, losing that page; here that is an error
        if (slot < 0)
            return set_error(NYION_ERR_OOM, "kv pool: cold tier full (%d slots)", cold_slots_);
        slot_used_[slot] = 1;
        cursor_ = (slot + 1) % cold_slots_;
        const int b = where_[best];
        state_[best] = kCold;
        where_[best] = slot;
        hot_count_--;
        cold_count_++;
        evictions_++;
        unlink(best);
        free_blocks_.push_back(b);
        ev.push_back(nyion_page_event{NYION_PAGE_EVICT, best, b, slot});
        return NYION_OK;
    }

    // cache.rs:479-523: evict first when full, then the slot's bytes come
    // back into a block and the page is hot at the LRU head
    int reload(int p, std::vector<nyion_page_event>& ev) {
        int rc;
        if (hot_count_ >= hot_limit_ && (rc = evict_one(ev)) != NYION_OK) return rc;
        if (free_blocks_.empty()) return set_error(NYION_ERR_OOM, "kv pool: no free block for page %d", p);
        const int slot = where_[p];
        const int b = free_blocks_.back();
        free_blocks_.pop_back();
        slot_used_[slot] = 0;
        state_[p] = kHot;
        where_[p] = b;
        hot_count_++;
        cold_count_--;
        reloads_++;
        push_head(p);
        ev.push_back(nyion_page_event{NYION_PAGE_RELOAD, p, b, slot});
        return NYION_OK;
    }

    void push_head(int p) {
        prev_[p] = -1;
        next_[p] = head_;
        if (head_ >= 0) prev_[head_] = p;
        head_ = p;
        if (tail_ < 0) tail_ = p;
    }
    void unlink(int p) {
        const int a = prev_[p], c = next_[p];
        if (a >= 0) next_[a] = c;
        if (c >= 0) prev_[c] = a;
        if (head_ == p) head_ = c;
        if (tail_ == p) tail_ = a;
        prev_[p] = next_[p] = -1;
    }
    void touch(int p) {  // cache.rs:311-323
        if (head_ == p) return;
        unlink(p);
        push_head(p);
    }

    int hot_limit_, cold_slots_, max_pages_;
    std::vector<int> state_, where_, prev_, next_;
    std::vector<double> importance_;
    std::vector<char> slot_used_;
    std::vector<int> free_blocks_;
    int head_ = -1, tail_ = -1, cursor_ = 0, n_created_ = 0;
    int prot_lo_ = 0, prot_hi_ = -1;
    long long hot_count_ = 0, cold_count_ = 0, evictions_ = 0, reloads_ = 0;
};

}  // namespace nyion
