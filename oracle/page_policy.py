"""Restatement of the PagedKVCache page policy (swamp-engine/src/cache.rs).

TEST INFRASTRUCTURE ONLY: what the tests compare the policy inside the
product library's paged KV pool (nyion_page_policy_* / nyion_kv_pool_*)
against.  Nothing in the product imports it.

Followed line by line (paths relative to the reference repository root):
  cache.rs:277-309  alloc_hot_page_in_zone: a new page is hot, importance 0,
                    at the LRU head
  cache.rs:311-323  touch_lru_in_zone
  cache.rs:325-336  remove_from_lru_in_zone
  cache.rs:407-477  evict_one_page_from_zone: scan the LRU tail and up to 7
                    pages before it, keep the first strictly lower
                    importance; cold slot = first unused at or after the
                    write cursor; cursor = slot + 1
  cache.rs:479-523  reload_cold_page_in_zone: evict first when the hot count
                    has reached the limit; the slot becomes unused; the page
                    goes to the LRU head
  cache.rs:525-546  ensure_page: create pages in order up to the requested
                    one (evicting first whenever the limit is reached), reload
                    a cold page, then touch
  cache.rs:549-553  ensure_pages_hot: ensure_page over a range in order
  cache.rs:563-581  record_importance / reset_entropy
Three points are this build's own and are restated, not followed:
  * which physical block a hot page occupies (the reference allocates fresh
    host memory): blocks 0..hot_limit-1 on a LIFO free list, 0 first;
  * a full cold tier is an error (the reference overwrites the slot at its
    cursor, losing that page); so is a range larger than the hot limit;
  * while ensure() makes a range hot, the range's pages are not eviction
    candidates: the scan takes the first eight pages from the LRU tail that
    lie outside the range (the reference would evict a page of the range
    it is making hot and then read a missing page).
The reference's own tiered tests (cache.rs:951-998) stay inside one page and
do not exercise eviction; the tests pin this restatement with hand-worked
cases instead.
"""

CREATE, EVICT, RELOAD = 0, 1, 2
UNMAPPED, HOT, COLD = 0, 1, 2


class PolicyError(Exception):
    pass


class PagePolicy:
    def __init__(self, hot_limit, cold_slots, max_pages):
        self.hot_limit = hot_limit
        self.cold_slots = cold_slots
        self.max_pages = max_pages
        self.state = [UNMAPPED] * max_pages
        self.where = [-1] * max_pages
        self.importance = [0.0] * max_pages
        self.lru = []  # most recent first
        self.slot_used = [False] * cold_slots
        self.cursor = 0
        self.free = list(range(hot_limit - 1, -1, -1))
        self.n_created = 0
        self.hot_count = 0
        self.protected = range(0)

    # cache.rs:277-309
    def _create(self, ev):
        if not self.free:
            raise PolicyError("no free block")
        p = self.n_created
        self.n_created += 1
        b = self.free.pop()
        self.state[p], self.where[p], self.importance[p] = HOT, b, 0.0
        self.hot_count += 1
        self.lru.insert(0, p)
        ev.append((CREATE, p, b, -1))

    # cache.rs:407-477
    def _evict_one(self, ev):
        if not self.lru:
            return
        cands = [p for p in reversed(self.lru) if p not in self.protected][:8]  # tail first
        if not cands:
            raise PolicyError("every hot page is in the range being made hot")
        best = cands[0]
        for c in cands[1:]:
            if self.importance[c] < self.importance[best]:
                best = c
        slot = None
        for i in range(self.cold_slots):
            s = (self.cursor + i) % self.cold_slots
            if not self.slot_used[s]:
                slot = s
                break
        if slot is None:
            raise PolicyError("cold tier full")
        self.slot_used[slot] = True
        self.cursor = (slot + 1) % self.cold_slots
        b = self.where[best]
        self.state[best], self.where[best] = COLD, slot
        self.hot_count -= 1
        self.lru.remove(best)
        self.free.append(b)
        ev.append((EVICT, best, b, slot))

    # cache.rs:479-523
    def _reload(self, p, ev):
        if self.hot_count >= self.hot_limit:
            self._evict_one(ev)
        if not self.free:
            raise PolicyError("no free block")
        slot = self.where[p]
        b = self.free.pop()
        self.slot_used[slot] = False
        self.state[p], self.where[p] = HOT, b
        self.hot_count += 1
        self.lru.insert(0, p)
        ev.append((RELOAD, p, b, slot))

    # cache.rs:525-546
    def _ensure_page(self, p, ev):
        if not 0 <= p < self.max_pages:
            raise PolicyError("page out of range")
        while p >= self.n_created:
            if self.hot_count >= self.hot_limit:
                self._evict_one(ev)
            self._create(ev)
        if self.state[p] == COLD:
            self._reload(p, ev)
        if self.lru[0] != p:  # cache.rs:311-323
            self.lru.remove(p)
            self.lru.insert(0, p)

    # cache.rs:549-553
    def ensure(self, first, last=None):
        """Returns (ok, events); events up to a failure are kept."""
        last = first if last is None else last
        ev = []
        if first > last or last - first + 1 > self.hot_limit:
            return False, ev
        self.protected = range(first, last + 1)
        try:
            for q in range(first, last + 1):
                self._ensure_page(q, ev)
        except PolicyError:
            return False, ev
        finally:
            self.protected = range(0)
        return True, ev

    # cache.rs:563-571
    def record(self, page, weight):
        if 0 <= page < self.n_created:
            self.importance[page] += weight

    # cache.rs:573-580
    def reset(self):
        self.importance = [0.0] * self.max_pages
