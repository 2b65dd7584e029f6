// Host-only stress of the library's CPU-side data structures -- the HMA
// arena's free list (arena.hpp) and the paged KV pool's page policy
// (page_policy.hpp) -- built with the address and undefined-behaviour
// sanitizers by tests/test_host_sanitize.py.  Random operation sequences;
// after every operation the structural invariants are checked.  Exit 0 when
// every check held.
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>

#include <map>
#include <random>
#include <set>
#include <vector>

#include "../../nyion.rs_amd/csrc/arena.hpp"
#include "../../nyion.rs_amd/csrc/page_policy.hpp"

// The library's error reporting, for this host-only build.
namespace nyion {
int set_error(int code, const char*, ...) { return code; }
void clear_error() {}
}  // namespace nyion

#define CHECK(c)                                                         \
    do {                                                                 \
        if (!(c)) {                                                      \
            fprintf(stderr, "check failed: %s (line %d)\n", #c, __LINE__); \
            exit(1);                                                     \
        }                                                                \
    } while (0)

static void check_region(const nyion::Region& r) {
    size_t live = 0, fr = 0, end = 0;
    std::map<size_t, std::pair<size_t, int>> all;  // offset -> (size, 0 live / 1 free)
    for (auto& kv : r.live) {
        CHECK(kv.first % 256 == 0 && kv.second % 256 == 0 && kv.second > 0);
        live += kv.second;
        all[kv.first] = {kv.second, 0};
    }
    for (auto& kv : r.free_) {
        CHECK(kv.second > 0);
        fr += kv.second;
        CHECK(all.count(kv.first) == 0);
        all[kv.first] = {kv.second, 1};
    }
    CHECK(live == r.used);
    CHECK(live + fr == r.cap);
    int prev_kind = -1;
    for (auto& kv : all) {  // ranges tile [0, cap) with no two free ones adjacent
        CHECK(kv.first == end);
        CHECK(!(prev_kind == 1 && kv.second.second == 1));
        end = kv.first + kv.second.first;
        prev_kind = kv.second.second;
    }
    CHECK(end == r.cap);
}

static void stress_region(unsigned seed) {
    std::mt19937 rng(seed);
    std::vector<char> mem(1 << 20);
    nyion::Region r;
    const size_t cap = (1 << 20) - 256 * (seed % 3);
    r.init(mem.data(), cap);
    std::vector<void*> live;
    for (int i = 0; i < 20000; i++) {
        const int op = rng() % 100;
        if (op < 55) {
            size_t sz = rng() % 3 == 0 ? rng() % 300 : rng() % 40000;
            if (rng() % 200 == 0) sz = (size_t)-1 - rng() % 100;  // absurd sizes are refused
            void* p = r.alloc(sz);
            if (p) {
                CHECK((char*)p >= mem.data() && (char*)p + r.live_size(p) <= mem.data() + cap);
                memset(p, 0xab, r.live_size(p));  // the whole range is writable
                live.push_back(p);
            }
        } else if (op < 95 && !live.empty()) {
            const size_t k = rng() % live.size();
            CHECK(r.release(live[k]));
            CHECK(!r.release(live[k]));  // a second free is refused
            live[k] = live.back();
            live.pop_back();
        } else if (op < 97) {
            CHECK(!r.release(mem.data() + cap + 4096));  // foreign pointers are refused
        } else {
            r.reset();
            live.clear();
        }
        check_region(r);
    }
}

static void check_policy(const nyion::PagePolicy& p, int pages) {
    std::vector<int> lru(pages);
    const int n = p.lru_order(lru.data(), pages);
    CHECK(n == p.hot_count() && n <= p.hot_limit());
    std::set<int> blocks, in_lru(lru.begin(), lru.begin() + n);
    CHECK((int)in_lru.size() == n);
    int hot = 0, cold = 0;
    for (int q = 0; q < pages; q++) {
        int where = -1;
        double imp = 0.0;
        const int st = p.state(q, &where, &imp);
        CHECK(st >= 0 && st <= 2);
        if (st == 1) {
            hot++;
            CHECK(where >= 0 && where < p.hot_limit() && blocks.insert(where).second);
            CHECK(in_lru.count(q) == 1);
        } else {
            CHECK(in_lru.count(q) == 0);
        }
        cold += st == 2;
    }
    CHECK(hot == p.hot_count() && cold == p.cold_count());
}

static void stress_policy(unsigned seed) {
    std::mt19937 rng(seed);
    const int hot = 1 + rng() % 16, cold = rng() % 64, pages = 8 + rng() % 200;
    nyion::PagePolicy p(hot, cold, pages);
    std::vector<nyion_page_event> ev;
    for (int i = 0; i < 4000; i++) {
        const int op = rng() % 100;
        if (op < 70) {
            const int first = rng() % pages;
            const int last = std::min(pages - 1, first + (int)(rng() % (hot + 1)));
            if (last - first + 1 > hot) continue;  // the library refuses such a range
            ev.clear();
            p.protect(first, last);
            int rc = NYION_OK;
            for (int q = first; q <= last && rc == NYION_OK; q++) rc = p.ensure(q, ev);
            p.protect(0, -1);
            if (rc == NYION_OK)  // the whole range ends hot
                for (int q = first; q <= last; q++) CHECK(p.state(q, nullptr, nullptr) == 1);
        } else if (op < 95) {
            p.record(rng() % pages, (rng() % 5) * 0.25);
        } else {
            p.reset();
        }
        check_policy(p, pages);
    }
}

int main() {
    for (unsigned s = 0; s < 12; s++) stress_region(s);
    for (unsigned s = 0; s < 60; s++) stress_policy(s);
    printf("host structures: all checks held\n");
    return 0;
}
