// kv_pool.hip — device-resident paged KV pool with host spill.
//
// The reference keeps KV pages in host RAM and spills cold pages to a file
// (swamp-engine/src/cache.rs:251-274 cold store, 277-309 page allocation,
// 311-336 LRU, 407-477 eviction, 479-523 reload, 525-553 ensure_page /
// ensure_pages_hot, 563-581 importance).  Here the hot tier is HBM and the
// cold tier pinned host memory:
//
//   page p        = tokens [p*bt, (p+1)*bt) of the sequence, every layer
//   hot page      = one physical block b of every layer's K and V pool
//                   (pool layout [layer][block][kv head][bt][row], so block b
//                   of all layers is 2 * n_layers contiguous runs)
//   cold page     = one slot of the pinned host store, [layer][K|V][block]
//   block table   = device int32 [max_pages]: b for a hot page, -1 otherwise
//                   (the decode and KV-write kernels' table for this sequence)
//
// The policy (which page to evict, where it goes) is the reference's, in a
// host class of its own with a C ABI (PagePolicy below) so that it can be
// checked without a GPU; the pool turns its events into one copy kernel
// each on the caller's stream.
#include <stdlib.h>
#include <string.h>

#include <vector>

#include "common.hpp"
#include "page_policy.hpp"

namespace nyion {

// ------------------------------------------------------------ pool

// Moves (or zeroes) block b of every layer's K and V pool: 16 bytes per
// thread over 2 * n_layers runs of block_bytes.
//   dir 0: zero the device block; 1: device -> host slot; 2: host slot -> device
struct PageMoveArgs {
    unsigned char* k;  // pool bases [layer][block][...]
    unsigned char* v;
    unsigned char* host;  // slot base [layer][2][block_bytes]
    long long layer_stride;
    long long block_off;
    long long block_bytes;
    int n_layers;
    int dir;
};

typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void page_move_kernel(PageMoveArgs a) {
    const long long per_run = a.block_bytes / 16;
    const long long n = per_run * 2 * a.n_layers;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n;
         i += (long long)gridDim.x * blockDim.x) {
        const long long run = i / per_run;
        const long long off = (i - run * per_run) * 16;
        const int layer = (int)(run >> 1);
        unsigned char* dev = ((run & 1) ? a.v : a.k) + layer * a.layer_stride + a.block_off + off;
        unsigned char* hst = a.host + run * a.block_bytes + off;
        if (a.dir == 0)
            *(u32x4v*)dev = u32x4v{0u, 0u, 0u, 0u};
        else if (a.dir == 1)
            *(u32x4v*)hst = *(const u32x4v*)dev;
        else
            *(u32x4v*)dev = *(const u32x4v*)hst;
    }
}

struct KvPool {
    PagePolicy policy;
    int n_layers, n_kv_heads, head_dim, block_tokens, kv_dtype;
    long long row_bytes, block_bytes, layer_stride, slot_bytes;
    unsigned char* k = nullptr;  // device
    unsigned char* v = nullptr;
    unsigned char* cold = nullptr;   // pinned host [slot][layer][2][block_bytes]
    int32_t* table_dev = nullptr;    // device [max_pages]
    int32_t* table_host = nullptr;   // pinned mirror
    std::vector<nyion_page_event> events;

    KvPool(int hot, int cold_slots, int max_pages) : policy(hot, cold_slots, max_pages) {}
};

static void free_pool(KvPool* p) {
    if (!p) return;
    if (p->k) (void)hipFree(p->k);
    if (p->v) (void)hipFree(p->v);
    if (p->table_dev) (void)hipFree(p->table_dev);
    if (p->cold) (void)hipHostFree(p->cold);
    if (p->table_host) (void)hipHostFree(p->table_host);
    delete p;
}

static int move_page(KvPool* p, int block, int slot, int dir, hipStream_t st) {
    PageMoveArgs a;
    a.k = p->k;
    a.v = p->v;
    a.host = slot >= 0 ? p->cold + slot * p->slot_bytes : nullptr;
    a.layer_stride = p->layer_stride;
    a.block_off = (long long)block * p->block_bytes;
    a.block_bytes = p->block_bytes;
    a.n_layers = p->n_layers;
    a.dir = dir;
    const long long n = p->block_bytes / 16 * 2 * p->n_layers;
    long long g = (n + 255) / 256;
    if (g > 1024) g = 1024;
    hipLaunchKernelGGL(page_move_kernel, dim3((unsigned)g), dim3(256), 0, st, a);
    return check_launch("kv pool page move");
}

// Pages first..last made hot in order (ensure_pages_hot, cache.rs:549-553);
// the events of every step are kept even when a later one fails.
static int policy_ensure_range(PagePolicy* pp, int first, int last, std::vector<nyion_page_event>& ev) {
    if (first > last || last - first + 1 > pp->hot_limit())
        return set_error(NYION_ERR_INVALID, "page policy: range [%d, %d] exceeds the %d hot pages",
                         first, last, pp->hot_limit());
    pp->protect(first, last);
    int rc = NYION_OK;
    for (int q = first; q <= last && rc == NYION_OK; q++) rc = pp->ensure(q, ev);
    pp->protect(0, -1);
    return rc;
}

// Block table entries written from kernel arguments (no host staging buffer
// that a later call could overwrite while a copy is in flight).
constexpr int kTableUpdates = 32;
struct TableUpdate {
    int32_t* table;
    int page[kTableUpdates];
    int block[kTableUpdates];
    int n;
};

__global__ void table_update_kernel(TableUpdate u) {
    const int i = threadIdx.x;
    if (i < u.n) u.table[u.page[i]] = u.block[i];
}

}  // namespace nyion

using namespace nyion;

extern "C" {

// ---------------------------------------------------------------- policy ABI

void* nyion_page_policy_create(int hot_limit, int cold_slots, int max_pages) {
    clear_error();
    if (hot_limit <= 0 || cold_slots < 0 || max_pages <= 0) {
        set_error(NYION_ERR_INVALID, "page policy: hot %d cold %d pages %d", hot_limit, cold_slots,
                  max_pages);
        return nullptr;
    }
    return new PagePolicy(hot_limit, cold_slots, max_pages);
}

void nyion_page_policy_destroy(void* h) { delete (PagePolicy*)h; }

int nyion_page_policy_ensure(void* h, int first_page, int last_page, nyion_page_event* events,
                             int max_events, int* n_events) {
    clear_error();
    if (!h || !n_events) return set_error(NYION_ERR_INVALID, "page policy: null handle");
    std::vector<nyion_page_event> ev;
    const int rc = policy_ensure_range((PagePolicy*)h, first_page, last_page, ev);
    const int n = (int)ev.size();
    *n_events = n;
    if (events)
        for (int i = 0; i < n && i < max_events; i++) events[i] = ev[i];
    if (rc != NYION_OK) return rc;
    if (events && n > max_events)
        return set_error(NYION_ERR_INVALID, "page policy: %d events for %d entries", n, max_events);
    return NYION_OK;
}

int nyion_page_policy_record(void* h, int page, double weight) {
    clear_error();
    if (!h) return set_error(NYION_ERR_INVALID, "page policy: null handle");
    ((PagePolicy*)h)->record(page, weight);
    return NYION_OK;
}

int nyion_page_policy_reset(void* h) {
    clear_error();
    if (!h) return set_error(NYION_ERR_INVALID, "page policy: null handle");
    ((PagePolicy*)h)->reset();
    return NYION_OK;
}

int nyion_page_policy_state(void* h, int page, int* where, double* importance) {
    if (!h) return -1;
    return ((PagePolicy*)h)->state(page, where, importance);
}

int nyion_page_policy_lru(void* h, int* pages, int cap) {
    if (!h || !pages) return -1;
    return ((PagePolicy*)h)->lru_order(pages, cap);
}

// ------------------------------------------------------------------ pool ABI

void* nyion_kv_pool_create(int n_layers, int n_kv_heads, int head_dim, int block_tokens,
                           int kv_dtype, int hot_blocks, int cold_slots, int max_pages) {
    clear_error();
    if (require_device() != NYION_OK) return nullptr;
    if (n_layers <= 0 || n_kv_heads <= 0 || head_dim <= 0 || head_dim % 8 || !is_pow2(block_tokens) ||
        hot_blocks <= 0 || cold_slots < 0 || max_pages <= 0 ||
        (kv_dtype != NYION_KV_F32 && kv_dtype != NYION_KV_Q4_20B && kv_dtype != NYION_KV_F16)) {
        set_error(NYION_ERR_INVALID, "kv pool: layers %d heads %d dim %d bt %d dtype %d hot %d cold %d "
                  "pages %d", n_layers, n_kv_heads, head_dim, block_tokens, kv_dtype, hot_blocks,
                  cold_slots, max_pages);
        return nullptr;
    }
    KvPool* p = new KvPool(hot_blocks, cold_slots, max_pages);
    p->n_layers = n_layers;
    p->n_kv_heads = n_kv_heads;
    p->head_dim = head_dim;
    p->block_tokens = block_tokens;
    p->kv_dtype = kv_dtype;
    p->row_bytes = kv_dtype == NYION_KV_F32   ? 4LL * head_dim
                   : kv_dtype == NYION_KV_F16 ? 2LL * head_dim
                                              : q4_row_bytes(head_dim);
    p->block_bytes = p->row_bytes * block_tokens * n_kv_heads;
    if (p->block_bytes % 16) {
        set_error(NYION_ERR_UNSUPPORTED, "kv pool: block of %lld bytes (not a multiple of 16)",
                  p->block_bytes);
        free_pool(p);
        return nullptr;
    }
    p->layer_stride = p->block_bytes * hot_blocks;
    p->slot_bytes = 2 * p->block_bytes * n_layers;
    const size_t pool_bytes = (size_t)(p->layer_stride * n_layers);
    if (hipMalloc((void**)&p->k, pool_bytes) != hipSuccess ||
        hipMalloc((void**)&p->v, pool_bytes) != hipSuccess ||
        hipMalloc((void**)&p->table_dev, sizeof(int32_t) * max_pages) != hipSuccess ||
        hipHostMalloc((void**)&p->table_host, sizeof(int32_t) * max_pages, hipHostMallocDefault) !=
            hipSuccess ||
        (cold_slots > 0 && hipHostMalloc((void**)&p->cold, (size_t)(p->slot_bytes * cold_slots),
                                         hipHostMallocDefault) != hipSuccess)) {
        (void)hipGetLastError();
        set_error(NYION_ERR_OOM, "kv pool: %zu device bytes x2, %lld host bytes", pool_bytes,
                  p->slot_bytes * cold_slots);
        free_pool(p);
        return nullptr;
    }
    for (int i = 0; i < max_pages; i++) p->table_host[i] = -1;
    if (hipMemcpy(p->table_dev, p->table_host, sizeof(int32_t) * max_pages, hipMemcpyHostToDevice) !=
        hipSuccess) {
        (void)hipGetLastError();
        set_error(NYION_ERR_LAUNCH, "kv pool: table upload");
        free_pool(p);
        return nullptr;
    }
    return p;
}

void nyion_kv_pool_destroy(void* h) {
    if (!h) return;
    (void)hipDeviceSynchronize();
    free_pool((KvPool*)h);
}

int nyion_kv_pool_layer(void* h, int layer, void** k_pool, void** v_pool) {
    clear_error();
    KvPool* p = (KvPool*)h;
    if (!p || layer < 0 || layer >= p->n_layers || !k_pool || !v_pool)
        return set_error(NYION_ERR_INVALID, "kv pool: layer %d", layer);
    *k_pool = p->k + layer * p->layer_stride;
    *v_pool = p->v + layer * p->layer_stride;
    return NYION_OK;
}

const int32_t* nyion_kv_pool_table(void* h) { return h ? ((KvPool*)h)->table_dev : nullptr; }

void* nyion_kv_pool_policy(void* h) { return h ? (void*)&((KvPool*)h)->policy : nullptr; }

int nyion_kv_pool_ensure(void* h, int first_page, int last_page, nyion_stream_t stream) {
    clear_error();
    KvPool* p = (KvPool*)h;
    if (!p) return set_error(NYION_ERR_INVALID, "kv pool: null handle");
    hipStream_t st = (hipStream_t)stream;
    p->events.clear();
    const int rc = policy_ensure_range(&p->policy, first_page, last_page, p->events);
    // replay whatever the policy did, also when it stopped on an error, so
    // that device memory and the table match it; in order on one stream, a
    // block's spill precedes its reuse
    TableUpdate u{};
    u.table = p->table_dev;
    int mrc = NYION_OK;
    for (const nyion_page_event& e : p->events) {
        if (mrc == NYION_OK) {
            if (e.kind == NYION_PAGE_CREATE)
                mrc = move_page(p, e.block, -1, 0, st);
            else if (e.kind == NYION_PAGE_EVICT)
                mrc = move_page(p, e.block, e.slot, 1, st);
            else
                mrc = move_page(p, e.block, e.slot, 2, st);
        }
        u.page[u.n] = e.page;
        u.block[u.n] = e.kind == NYION_PAGE_EVICT ? -1 : e.block;
        if (++u.n == kTableUpdates) {
            hipLaunchKernelGGL(table_update_kernel, dim3(1), dim3(kTableUpdates), 0, st, u);
            u.n = 0;
        }
    }
    if (u.n > 0) hipLaunchKernelGGL(table_update_kernel, dim3(1), dim3(kTableUpdates), 0, st, u);
    const int lrc = check_launch("kv pool table update");
    if (rc != NYION_OK) return rc;
    return mrc != NYION_OK ? mrc : lrc;
}

// The executor's importance hand-off (executor.rs:751-755): every position
// whose attention weight sum exceeds `threshold` adds it to its page
// (record_importance, cache.rs:563-571).
int nyion_kv_pool_record_importance(void* h, const double* importance, int n_positions,
                                    double threshold) {
    clear_error();
    KvPool* p = (KvPool*)h;
    if (!p || (!importance && n_positions > 0) || n_positions < 0)
        return set_error(NYION_ERR_INVALID, "kv pool: importance arguments");
    for (int t = 0; t < n_positions; t++)
        if (importance[t] > threshold) p->policy.record(t / p->block_tokens, importance[t]);
    return NYION_OK;
}

int nyion_kv_pool_stats(void* h, int64_t* hot, int64_t* cold, int64_t* evictions,
                        int64_t* reloads) {
    clear_error();
    KvPool* p = (KvPool*)h;
    if (!p) return set_error(NYION_ERR_INVALID, "kv pool: null handle");
    if (hot) *hot = p->policy.hot_count();
    if (cold) *cold = p->policy.cold_count();
    if (evictions) *evictions = p->policy.evictions();
    if (reloads) *reloads = p->policy.reloads();
    return NYION_OK;
}

// Host view of one cold slot (pinned memory; the caller synchronises the
// stream of the evicting call first).
const void* nyion_kv_pool_cold_slot(void* h, int slot) {
    KvPool* p = (KvPool*)h;
    if (!p || !p->cold || slot < 0) return nullptr;
    return p->cold + slot * p->slot_bytes;
}

}  // extern "C"
