/*
 * nyion_hip.h — C ABI of the MI355X (gfx950) attention path for Nyion.
 *
 * One shared library, libnyion_hip.so, built with hipcc --offload-arch=gfx950.
 * Plain pointers and sizes only.  Every entry point returns an int status
 * (0 = NYION_OK, < 0 = error) and leaves a message in nyion_last_error()
 * (thread-local), so a binding can map "!= 0" to the reference's `false` /
 * GpuError::NotAvailable and take its CPU fallback
 * (swamp-engine/src/executor.rs:709-764, swamp-gpu/src/lib.rs:618-624).
 * The exceptions are the swamp-kernels symbols (mojo_*), which keep the
 * reference's void/handle signatures and silent-return-on-null behaviour.
 *
 * Device pointers ("d_" or pool arguments) must point into memory on the
 * current HIP device.  Streams are hipStream_t passed as void* (NULL = the
 * default stream).  Calls are asynchronous on that stream unless stated.
 * No entry point allocates device memory on the attention hot path: split-K
 * partial results go into a caller-provided workspace.
 *
 * KV pool layout (paged):   [num_blocks][n_kv_heads][block_tokens][row]
 *   row = head_dim f32 (NYION_KV_F32), head_dim binary16 (NYION_KV_F16) or
 *   ceil(head_dim/32)*20 bytes of the
 *   reference's Q4-20B groups (NYION_KV_Q4_20B: f16 d, f16 dmin, 16 nibble
 *   bytes; element i of a group in byte 4+i/2, low nibble when i is even;
 *   swamp-engine/src/cache.rs:637-663, 375-394).
 *   Attention over binary16 rows multiplies them on binary16 matrix cores:
 *   q is split into binary16 high and low parts (so |q| must stay below
 *   65504) and the softmax weights are rounded to binary16 (relative error
 *   <= 2^-12 per weight) before the product with V.
 *   Token t of sequence b lives in block block_tables[b*max_blocks_per_seq +
 *   t/block_tokens], slot t%block_tokens.  block_tokens is a power of two.
 */
#ifndef NYION_HIP_H
#define NYION_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* nyion_stream_t; /* hipStream_t */

enum nyion_status {
    NYION_OK = 0,
    NYION_ERR_INVALID = -1,     /* bad argument (null, size, alignment, shape) */
    NYION_ERR_UNSUPPORTED = -2, /* valid but not implemented for this shape */
    NYION_ERR_NO_DEVICE = -3,   /* no HIP device / not gfx950 */
    NYION_ERR_OOM = -4,         /* allocation failed (arena or HIP) */
    NYION_ERR_LAUNCH = -5,      /* HIP launch or runtime error */
    NYION_ERR_WORKSPACE = -6,   /* caller workspace too small */
    NYION_ERR_RANGE = -7        /* an input exceeded a reduced-precision operand (nyion_take_status) */
};

/* KV row formats: f32; the reference's Q4-20B groups; IEEE binary16 (the
 * f16 caches of the reference's CUDA path, fused_attention.cu:534-545;
 * written with round-to-nearest-even, read exactly). */
enum nyion_kv_dtype { NYION_KV_F32 = 0, NYION_KV_Q4_20B = 1, NYION_KV_F16 = 2 };

/* ---------------------------------------------------------------- runtime */

/* Thread-local message of the last failing call on this thread ("" if none). */
const char* nyion_last_error(void);
/* Selects `device`, checks it is gfx950.  Replaces gpu_init()
 * (swamp-gpu/src/lib.rs:626). */
int nyion_init(int device);
int nyion_device_count(void);
/* Waits for all work on the current device (gpu_sync, fused_attention.cu:181-189). */
int nyion_sync(void);
/* Library version string. */
const char* nyion_version(void);

/* Range report of the current device.  Kernels that carry an input in a
 * narrower format than the reference's f32 record, in a per-device sticky
 * word, when an input does not fit it: prefill's V (binary16 in the P.V
 * product: |v| >= 65520 or infinite) and the q of decode over binary16 or
 * Q4-20B pools (binary16 high part: |q| >= 65520).  This call orders itself after the work on
 * `stream`, waits for it, takes (reads and clears) the word and returns
 * NYION_OK, or NYION_ERR_RANGE with nyion_last_error() naming what
 * overflowed since the last take.  The word is per device, not per stream:
 * work on other streams of the device lands in the same word.  Takes on one
 * device from several threads are serialised by the library, so each report
 * reaches exactly one taker.  No
 * counterpart in the reference, whose CPU path computes in f32 throughout
 * (swamp-engine/src/ops.rs:170-278). */
int nyion_take_status(nyion_stream_t stream);

/* ------------------------------------------------------ decode attention */

/* The ComputeGraph Attention node, executed now on `stream`.
 * Replaces ComputeNodeOp::Attention {d_q, d_k, d_v, d_scores, d_out, n_heads,
 * n_kv_heads, seq_len, head_dim, kv_stride} (swamp-gpu/src/compute_graph.rs:14-25)
 * recorded by GpuComputeContext::add_attention_node (swamp-gpu/src/lib.rs:505-519)
 * and run by submit_and_wait (lib.rs:479-489).
 * Semantics: ops::attention (swamp-engine/src/ops.rs:170-278) for one query
 * token at q_pos = seq_len-1: out[h] = softmax(q[h].K[kv(h)]^T / sqrt(D)) V,
 * kv(h) = h / (n_heads/n_kv_heads).
 * Layout: d_q, d_out [n_heads][head_dim] f32; d_k, d_v [n_kv_heads][kv_stride][row].
 * d_scores: optional f32 scratch of at least n_heads*seq_len floats (the
 * node's scores buffer: ScratchBuffers::d_scores holds n_heads*window_size,
 * swamp-gpu/src/lib.rs:317; the CUDA path n_heads*seq_len,
 * fused_attention.cu:206), 256-byte aligned; when given, its first
 * nyion_attention_node_scratch_bytes(...) bytes hold the split-K partial
 * results, when NULL the node runs one workgroup per (kv head, group of up
 * to 16 q heads). */
int nyion_attention_node(const float* d_q, const void* d_k, const void* d_v,
                         float* d_scores, float* d_out, uint32_t n_heads,
                         uint32_t n_kv_heads, uint32_t seq_len, uint32_t head_dim,
                         uint32_t kv_stride, int kv_dtype, nyion_stream_t stream);

/* Bytes at the start of a node's d_scores buffer (n_heads*seq_len floats)
 * that nyion_attention_node uses for its split-K partials and counters:
 * never more than 4*n_heads*seq_len; 0 when the node runs whole segments.
 * Host only (on a machine without a device it plans for 256 compute units).
 * Same sizing rule as the node; no counterpart in the reference. */
size_t nyion_attention_node_scratch_bytes(uint32_t n_heads, uint32_t n_kv_heads, uint32_t seq_len,
                                          uint32_t head_dim);

/* Project ABI names of the unlinked CUDA file, same arguments (f32 KV,
 * [n_kv_heads][kv_stride][head_dim]): gpu_attention_device
 * (swamp-gpu/kernels/fused_attention.cu:194-204) and gpu_attention_streamed
 * (fused_attention.cu:483-494).  Return 0 / -1 as those did.  The CUDA
 * originals allocated an n_heads*seq_len scores buffer per call; here the
 * node's split-K scratch is a device buffer per (device, stream), allocated
 * by the first call on that stream that needs more than it holds and kept
 * until the process ends (so the first call on a stream may not be inside
 * a graph capture).  Calls on one stream are ordered by it; calls on
 * different streams use different buffers and may overlap.  A buffer that
 * must grow is replaced after the stream's queued work has finished. */
int gpu_attention_device(const float* d_q, const float* d_k_cache, const float* d_v_cache,
                         float* d_output, int n_heads, int n_kv_heads, int seq_len,
                         int head_dim, int kv_stride);
int gpu_attention_streamed(const float* d_q, const float* d_k_cache, const float* d_v_cache,
                           float* d_output, int n_heads, int n_kv_heads, int seq_len,
                           int head_dim, int kv_stride, nyion_stream_t stream);

/* The node captured once into a HIP graph and replayed (the project ABI of
 * fused_attention.cu:595-663: gpu_graph_create_attention,
 * gpu_graph_replay_attention, gpu_graph_destroy).  Every argument is fixed at
 * creation; d_scores (n_heads*seq_len floats, 256-byte aligned, or NULL)
 * is the node's scratch as for nyion_attention_node, its counters cleared
 * inside the graph by a fill kernel.  create returns NULL on error (message
 * in nyion_last_error()); replay returns 0 / -1.  Replays of one graph on
 * different streams must not overlap (they share d_scores and d_output). */
void* gpu_graph_create_attention(const float* d_q, const float* d_k_cache,
                                 const float* d_v_cache, float* d_scores, float* d_output,
                                 int n_heads, int n_kv_heads, int seq_len, int head_dim,
                                 int kv_stride);
int gpu_graph_replay_attention(void* graph_handle, nyion_stream_t stream);
void gpu_graph_destroy(void* graph_handle);

/* The same two on binary16 K/V caches (NYION_KV_F16 rows, [n_kv_heads]
 * [kv_stride][head_dim], 8-byte aligned): gpu_attention_streamed_half
 * (fused_attention.cu:534-545) and gpu_graph_create_attention_half
 * (fused_attention.cu:672-717).  K/V values are used as stored (binary16
 * products, f32 accumulation; q and the softmax weights as in the pool
 * layout note above).  gpu_attention_streamed_half takes its split-K
 * scratch as gpu_attention_streamed does. */
int gpu_attention_streamed_half(const float* d_q, const uint16_t* d_k_cache,
                                const uint16_t* d_v_cache, float* d_output, int n_heads,
                                int n_kv_heads, int seq_len, int head_dim, int kv_stride,
                                nyion_stream_t stream);
void* gpu_graph_create_attention_half(const float* d_q, const uint16_t* d_k_cache,
                                      const uint16_t* d_v_cache, float* d_scores,
                                      float* d_output, int n_heads, int n_kv_heads, int seq_len,
                                      int head_dim, int kv_stride);

/* Batched paged GQA decode with split-K partitions and a log-sum-exp merge.
 * Replaces the CPU decode call of the executor (executor.rs:739-763):
 *   window <= 0           : ops::attention / attention_tracked semantics
 *                           (ops.rs:170-278, 283-401) over [0, valid_end],
 *                           valid_end = min(q_pos, ctx_len-1);
 *   window > 0            : ops::attention_sparse (ops.rs:85-168): globals
 *                           global_stride*g, g < min(window_start/stride, 128)
 *                           (none when global_stride <= 0), then the window
 *                           [window_start, valid_end], window_start =
 *                           valid_end-window+1 if valid_end > window else 0.
 *   kv_dtype Q4_20B       : the values of dequant_block (cache.rs:375-394):
 *                           V dequantised exactly so, K's products taken
 *                           per 32-element group as d*(nib.q) + dmin*sum(q);
 *                           multiplied on binary16 matrix cores with q and V
 *                           split into high and low parts and the weights
 *                           rounded to binary16 (|q| < 65504).
 *   kv_dtype F16          : K/V binary16 rows multiplied as stored, q split
 *                           into binary16 high and low parts, the weights
 *                           rounded to binary16 (|q| < 65504).
 * d_q, d_out: [batch][n_heads][head_dim] f32.  ctx_lens[batch] (>= 1);
 * q_pos[batch] or NULL (= ctx_len-1).  max_ctx: host upper bound of ctx_lens,
 * sizes the grid.  scale <= 0 means 1/sqrt(head_dim).
 * head_dim in {64, 128}; n_heads % n_kv_heads == 0.
 * d_workspace: >= nyion_paged_decode_workspace_size(...) bytes (256-byte
 * aligned), or NULL when that size is 0.  It holds the split-K partials and
 * per-(sequence, kv head, head group) arrival counters: it must be zero-filled before its
 * first use (nyion_decode_workspace_init, or any zeroing) and is left with
 * the counters at zero by every call.  Calls that run concurrently need
 * separate workspaces. */
size_t nyion_paged_decode_workspace_size(int batch, int n_heads, int n_kv_heads, int head_dim,
                                         int max_ctx, int window, int global_stride);
int nyion_paged_decode_attention(const float* d_q, const void* k_pool, const void* v_pool,
                                 const int32_t* block_tables, int max_blocks_per_seq,
                                 const int32_t* ctx_lens, const int32_t* q_pos, int batch,
                                 int n_heads, int n_kv_heads, int head_dim, int block_tokens,
                                 int num_blocks, int kv_dtype, int window, int global_stride,
                                 int max_ctx, float scale, float* d_out, void* d_workspace,
                                 size_t workspace_bytes, nyion_stream_t stream);

/* No counterpart in the reference: nyion_paged_decode_attention for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops and harnesses that forbid hipMalloc).  Same arguments and
 * results without the workspace: the split-K partials and arrival counters
 * live in a device array the library owns, NYION_DECODE_SCRATCH_BYTES per
 * device, held until the process ends (its device address is looked up by
 * nyion_init, or by the first call on a device).  The call allocates
 * nothing; it clears the array's counters with a fill kernel on `stream`
 * before the decode.  A call whose workspace
 * (nyion_paged_decode_workspace_size) exceeds the array returns
 * NYION_ERR_WORKSPACE.  All calls on one device share the array, which keeps
 * the last call's contents: calls that overlap in time on one device (other
 * streams or threads) race and must be serialised by the caller. */
#define NYION_DECODE_SCRATCH_BYTES (32u << 20)
int nyion_paged_decode_attention_noalloc(const float* d_q, const void* k_pool, const void* v_pool,
                                         const int32_t* block_tables, int max_blocks_per_seq,
                                         const int32_t* ctx_lens, const int32_t* q_pos, int batch,
                                         int n_heads, int n_kv_heads, int head_dim,
                                         int block_tokens, int num_blocks, int kv_dtype, int window,
                                         int global_stride, int max_ctx, float scale, float* d_out,
                                         nyion_stream_t stream);

/* Tracked decode: the executor's Full decode call, ops::attention_tracked
 * (ops.rs:283-401, called at executor.rs:742-749).  Same arguments and
 * output as nyion_paged_decode_attention, plus
 *   d_importance [batch][importance_stride] f64: importance[b][t] +=
 *     sum over q heads of the normalised probability of position t (f32
 *     probabilities accumulated in f64), for every attended t; other
 *     entries are left as they are.  importance_stride >= max_ctx.
 *   d_scores [batch][n_heads][scores_stride] f32 scratch, scores_stride >=
 *     max_ctx + 2: receives the scaled scores (log2 units) of the attended
 *     positions and, in its last two entries per row, the head's softmax
 *     max and denominator.
 * Two launches on `stream` (the decode, then the importance sum). */
int nyion_paged_decode_attention_tracked(
    const float* d_q, const void* k_pool, const void* v_pool, const int32_t* block_tables,
    int max_blocks_per_seq, const int32_t* ctx_lens, const int32_t* q_pos, int batch, int n_heads,
    int n_kv_heads, int head_dim, int block_tokens, int num_blocks, int kv_dtype, int window,
    int global_stride, int max_ctx, float scale, float* d_out, void* d_workspace,
    size_t workspace_bytes, float* d_scores, int scores_stride, double* d_importance,
    int importance_stride, nyion_stream_t stream);

/* The two launches of nyion_paged_decode_attention_tracked as separate calls
 * (no counterpart in the reference, whose attention_tracked is one CPU
 * routine, ops.rs:283-401): for GPU executors that run the importance sum
 * on a second stream, beside whatever follows the decode on the first (the
 * next layer's decode leaves most CUs idle at small batch).
 *   _scores: the tracked decode's first launch -- the same arguments and
 *     results as the tracked call, less the importance.
 *   _importance: the second -- importance[b][t] += sum over q heads of the
 *     normalised probability of t, from d_scores as _scores left it, for
 *     the positions the decode with the same ctx_lens, q_pos, window,
 *     global_stride and max_ctx attended.
 * Issued on one stream, _scores then _importance give the tracked call's
 * results bit for bit.  On two streams the caller orders _importance after
 * _scores (an event), and keeps d_scores unchanged until _importance has
 * run (one scores buffer per call in flight). */
int nyion_paged_decode_attention_scores(
    const float* d_q, const void* k_pool, const void* v_pool, const int32_t* block_tables,
    int max_blocks_per_seq, const int32_t* ctx_lens, const int32_t* q_pos, int batch, int n_heads,
    int n_kv_heads, int head_dim, int block_tokens, int num_blocks, int kv_dtype, int window,
    int global_stride, int max_ctx, float scale, float* d_out, void* d_workspace,
    size_t workspace_bytes, float* d_scores, int scores_stride, nyion_stream_t stream);
int nyion_paged_decode_importance(const int32_t* ctx_lens, const int32_t* q_pos, int batch,
                                  int n_heads, int window, int global_stride, int max_ctx,
                                  const float* d_scores, int scores_stride, double* d_importance,
                                  int importance_stride, nyion_stream_t stream);

/* Pipelined tracked decode (no counterpart in the reference): one launch
 * that runs this call's decode with its scores, as
 * nyion_paged_decode_attention_scores, and on workgroups past the decode's
 * the importance sum of the previous call's scores d_prev_scores into
 * d_prev_importance [batch][importance_stride >= max_ctx] -- the previous
 * call being one with the same ctx_lens, q_pos, batch, n_heads, window,
 * global_stride and max_ctx, such as the previous layer of the same decode
 * step, and d_prev_scores a different buffer from d_scores with the same
 * scores_stride.  d_prev_scores
 * NULL: no importance sum (the first layer); after the last layer,
 * nyion_paged_decode_importance sums its scores.  A step of L layers is then
 * L + 1 launches instead of 2L, with results equal to the tracked call's,
 * layer by layer, bit for bit. */
int nyion_paged_decode_attention_tracked_pipelined(
    const float* d_q, const void* k_pool, const void* v_pool, const int32_t* block_tables,
    int max_blocks_per_seq, const int32_t* ctx_lens, const int32_t* q_pos, int batch, int n_heads,
    int n_kv_heads, int head_dim, int block_tokens, int num_blocks, int kv_dtype, int window,
    int global_stride, int max_ctx, float scale, float* d_out, void* d_workspace,
    size_t workspace_bytes, float* d_scores, int scores_stride, const float* d_prev_scores,
    double* d_prev_importance, int importance_stride, nyion_stream_t stream);

/* Decode over explicit position lists (ops::attention_fugu, ops.rs:445-541,
 * whose list is the sparse set plus DSPark positions; also the Mojo
 * sparse_attention_q4 FFI, swamp-gpu/src/mojo.rs:5).  Softmax over exactly
 * the listed positions.  positions: [batch][max_positions] int32,
 * n_positions[batch]; every listed position must be < that sequence's length
 * in its block table. */
size_t nyion_paged_decode_positions_workspace_size(int batch, int n_heads, int n_kv_heads,
                                                   int head_dim, int max_positions);
int nyion_paged_decode_attention_positions(
    const float* d_q, const void* k_pool, const void* v_pool, const int32_t* block_tables,
    int max_blocks_per_seq, const int32_t* positions, const int32_t* n_positions,
    int max_positions, int batch, int n_heads, int n_kv_heads, int head_dim, int block_tokens,
    int num_blocks, int kv_dtype, float scale, float* d_out, void* d_workspace,
    size_t workspace_bytes, nyion_stream_t stream);

/* ------------------------------------------------- reference-shaped zones */

/* A cache laid out as PagedKVCache's (swamp-engine/src/cache.rs:20-21 zone
 * starts and page sizes, 185-237 flat page ids, 593-611 page_id /
 * slot_in_page, 700-747 page pointers): positions [0, 4096) in 32-token
 * pages, [4096, 131072) in 128-token pages, [131072, ...) in 1024-token
 * pages, flat page ids 0.., 128.., 1120.. by zone.  A page holds every
 * layer: row (layer, kv_head, slot) of a page of `bs` tokens starts
 * ((layer * n_kv_heads + kv_head) * bs + slot) rows into the page, a row
 * being head_dim f32 / binary16 elements or ceil(head_dim/32)*20 Q4-20B
 * bytes (cache.rs:365, 689, 711 f32; 627, 665, 733 Q4).
 *
 * The reference keeps one heap pointer per page (k_pages / v_pages,
 * cache.rs:33-36); here pages live in two device pools of pool_units units
 * each (elements for f32 / binary16, bytes for Q4-20B) and page_base[p]
 * holds flat page p's offset in units, the same in the K and the V pool.
 * A page whose offset is negative (absent), not a multiple of 4 units (f32,
 * Q4-20B) or 8 units (binary16), or whose extent passes pool_units is
 * absent: decode skips its rows, the gather returns NaN for them, the write
 * leaves them unwritten. */

/* Flat page id and page size (tokens) of position pos (host helpers for
 * building page_base; page_id of cache.rs:593-598, block_size_for
 * cache.rs:235-237).  pos < 0 gives -1. */
int64_t nyion_zone_page_id(int64_t pos);
int nyion_zone_page_tokens(int64_t pos);

/* PagedKVCache::save_at for one layer (cache.rs:749-811; f32 copy, Q4-20B
 * quantised byte-identically to save): tokens start_pos .. start_pos +
 * n_tokens - 1 from k, v [n_tokens][n_kv_heads][head_dim] f32. */
int nyion_zone_kv_write(void* k_pool, void* v_pool, int64_t pool_units, const int64_t* page_base,
                        int n_pages, int n_layers, int layer, int n_kv_heads, int head_dim,
                        int kv_dtype, int start_pos, int n_tokens, const float* k, const float* v,
                        nyion_stream_t stream);

/* Tokens [0, n_tokens) of one layer of a zone pool (the rows k_page_ptr /
 * v_page_ptr address, cache.rs:705-725, Q4 dequantised as dequant_block)
 * as [n_kv_heads][n_tokens][head_dim] f32, like nyion_kv_gather. */
int nyion_zone_kv_gather(const void* pool, int64_t pool_units, const int64_t* page_base,
                         int n_pages, int n_layers, int layer, int n_kv_heads, int head_dim,
                         int kv_dtype, int n_tokens, float* out, nyion_stream_t stream);

/* nyion_paged_decode_attention over one layer of zone pools: ops::attention
 * / ops::attention_sparse semantics as documented there, reading K/V
 * through k_page_ptr / v_page_ptr's addressing (ops.rs:210, 221).
 * page_bases: [batch][max_pages_per_seq] int64; max_ctx must be covered by
 * the table (nyion_zone_page_id(max_ctx - 1) < max_pages_per_seq); each
 * pool holds at least 32 rows (pool_units >= 32 * row).  The
 * workspace is sized by nyion_paged_decode_workspace_size with the same
 * arguments. */
int nyion_zone_decode_attention(const float* d_q, const void* k_pool, const void* v_pool,
                                int64_t pool_units, const int64_t* page_bases, int max_pages_per_seq,
                                int n_layers, int layer, const int32_t* ctx_lens,
                                const int32_t* q_pos, int batch, int n_heads, int n_kv_heads,
                                int head_dim, int kv_dtype, int window, int global_stride,
                                int max_ctx, float scale, float* d_out, void* d_workspace,
                                size_t workspace_bytes, nyion_stream_t stream);

/* ops::attention_sparse_q4 (swamp-engine/src/ops.rs:597-723) over one layer
 * of zone pools of Q4-20B rows (pool_bytes bytes each, page_bases as for
 * nyion_zone_decode_attention).  Per sequence b: valid_end = min(q_pos[b],
 * ctx_lens[b] - 1) (q_pos null: ctx_lens[b] - 1); the positions are
 * attention_sparse's (global_stride * i for i < min(window_start /
 * global_stride, 128), then window_start .. valid_end, window_start =
 * valid_end - window + 1 when valid_end > window, else 0; global_stride <= 0
 * gives no globals where the reference divides by it).  Rows are read with
 * that function's own rules: group g of the row is the 20 bytes at (slot *
 * groups + g) * 20 of the (layer, kv head) block of the position's page,
 * its nibble bytes give elements 0-15 (low nibbles) and 16-31 (high
 * nibbles), element = fma(d, nibble, dmin); q.k in the reference's 16-lane
 * FMA order times 1/sqrt(head_dim); weights below 1e-8 are skipped.  Rows
 * of absent pages are skipped.  head_dim 64 or 128, at most 32 q heads per
 * kv head; max_ctx >= every ctx_lens[b] and covered by the table; q and
 * out 16-byte aligned.  The workspace (256-byte aligned) is sized by
 * nyion_attention_sparse_q4_workspace_size and zero-filled before its first
 * use (nyion_decode_workspace_init); every call leaves its arrival counters
 * at zero.  Calls sharing a workspace must not overlap. */
size_t nyion_attention_sparse_q4_workspace_size(int batch, int n_heads, int n_kv_heads, int head_dim,
                                                int window, int max_ctx);
int nyion_attention_sparse_q4(const float* d_q, const void* k_pool, const void* v_pool,
                              int64_t pool_bytes, const int64_t* page_bases, int max_pages_per_seq,
                              int n_layers, int layer, const int32_t* ctx_lens, const int32_t* q_pos,
                              int batch, int n_heads, int n_kv_heads, int head_dim, int window,
                              int global_stride, int max_ctx, float* d_out, void* d_workspace,
                              size_t workspace_bytes, nyion_stream_t stream);

/* ------------------------------------------ per-layer ring and Fugu policy */

/* Sliding-window KV rings of the GPU decode path: PerLayerGpuState
 * (swamp-engine/src/scheduler.rs:36-178).  One ring of `window` slots per
 * layer, [n_kv_heads][window][head_dim] f32 on the device, zero-filled.
 *   upload_kv (upload_kv_async, scheduler.rs:103-117): host k, v
 *     [n_kv_heads][head_dim] of token `pos` -> slot pos % window;
 *   attention (execute_attention_async + sync, scheduler.rs:119-178): host q
 *     [n_heads][head_dim] -> host out, the Attention node over
 *     min(seq_len, window) slots; returns when out is written.
 * Unlike the reference (one f16 ring shared by every layer), each layer has
 * its own f32 ring.  Calls on one state are not thread-safe. */
void* nyion_layer_state_create(int window, int n_heads, int n_kv_heads, int head_dim,
                               int n_layers);
int   nyion_layer_state_upload_kv(void* state, int layer, const float* h_k, const float* h_v,
                                  int pos);
int   nyion_layer_state_attention(void* state, int layer, const float* h_q, float* h_out,
                                  int pos, int seq_len);
int   nyion_layer_state_sync(void* state);
void  nyion_layer_state_destroy(void* state);

/* FuguOrchestrator::decide_attention (swamp-engine/src/fugu.rs:129-170):
 * the attention variant of one step (host function, no device needed).
 * Fields are those of SystemSnapshot (fugu.rs:64-73) and FuguOrchestrator
 * (fugu.rs:79-117) that the decision reads. */
typedef struct nyion_system_snapshot {
    int64_t seq_len;
    double  dspark_accept_rate;
    int32_t is_prefill;
    int32_t predictive_throttle;
} nyion_system_snapshot;
typedef struct nyion_fugu_config {
    int64_t sparse_attention_threshold; /* 512 */
    int32_t sparse_window;              /* 256 */
    int32_t sparse_random_samples;      /* 32 */
    int32_t n_heads;
    int32_t head_dim;
} nyion_fugu_config;
enum nyion_attention_kind {
    NYION_ATTN_FULL = 0,          /* attention_tracked: nyion_paged_decode_attention_tracked */
    NYION_ATTN_SPARSE = 1,        /* attention_sparse: window, global stride 64 */
    NYION_ATTN_SPARSE_DSPARK = 2  /* attention_fugu: nyion_fugu_positions + _positions decode */
};
typedef struct nyion_attention_strategy {
    int32_t kind;
    int32_t window;
    int32_t num_random;
    int32_t sentinel_stride;
    int32_t num_dspark;
    int32_t _pad;
} nyion_attention_strategy;
/* FuguOrchestrator::new defaults (fugu.rs:103-117). */
int nyion_fugu_config_default(int n_heads, int head_dim, nyion_fugu_config* cfg);
int nyion_fugu_decide_attention(const nyion_system_snapshot* state, const nyion_fugu_config* cfg,
                                nyion_attention_strategy* out);

/* The attention_fugu position set (ops.rs:463-484), built on the device for
 * nyion_paged_decode_attention_positions: per sequence, sentinels
 * sentinel_stride*g (g < min(window_start/sentinel_stride, 128)), the window
 * [window_start, valid_end], then each DSPark position <= valid_end not
 * already present, in input order.  d_dspark [batch][dspark_stride] int32
 * (n_dspark used per row); d_positions [batch][max_positions], with
 * max_positions >= 128 + window + 1 + n_dspark; d_n_positions [batch]. */
int nyion_fugu_positions(const int32_t* d_ctx_lens, const int32_t* d_q_pos, int batch, int window,
                         int sentinel_stride, const int32_t* d_dspark, int n_dspark,
                         int dspark_stride, int32_t* d_positions, int max_positions,
                         int32_t* d_n_positions, nyion_stream_t stream);

/* Zero-fills a decode workspace on `stream` (a fill kernel, so it may be
 * recorded into a HIP graph).  Needed once before first use. */
int nyion_decode_workspace_init(void* d_workspace, size_t workspace_bytes, nyion_stream_t stream);

/* Decode work split.  The decode grid cuts the concatenated 16-token tile
 * lists of all (sequence, kv head, head group) segments into equal ranges, one
 * per workgroup; the grid is sized for `tokens` per workgroup (a power of two
 * in 64..4096; 0 restores the default: the launch's tokens divided by the CU
 * count, within 128..256) and capped at the workgroups the device holds
 * resident.  A launch of at most 64 segments cuts each segment into pieces
 * of that many tokens instead; by default a piece of small rows (4-bit, or
 * binary16 at head_dim 64) doubles while its K+V stays within 96 KiB and the
 * launch keeps 128 workgroups, and the pieces are then raised to one
 * workgroup per CU where each keeps 16 tiles.  Process-wide; for tuning.
 * The getter
 * returns the tokens per workgroup the current setting gives for `batch`
 * sequences of max_len tokens of f32 KV. */
int nyion_set_decode_partition_tokens(int tokens);
int nyion_get_decode_partition_tokens(int batch, int n_kv_heads, int head_dim, int max_len);

/* ----------------------------------------------------- prefill attention */

/* Causal prefill of one chunk on MFMA (bf16 in, f32 accumulate, f32 out).
 * Replaces the per-token ops::attention loop of prefill_slice
 * (executor.rs:106-137) for a chunk that is the whole prefix (pos_offset 0):
 * row i attends to keys [0, i] of the chunk.  Layout: q [n][n_heads][D],
 * k, v [n][n_kv_heads][D] bf16 (raw uint16 bits); out [n][n_heads][D] f32.
 * causal = 0 attends to all n keys.  head_dim 128 or 64.
 * When k_pool is non-NULL, the chunk's K/V are also written into the paged
 * cache at positions start_pos.. (the save_at loop, executor.rs:106-111),
 * widened to f32 or quantised to Q4-20B per kv_dtype.  Keys before the
 * chunk are not attended here; a chunk that continues a cached prefix uses
 * nyion_prefill_attention_bf16_ctx. */
int nyion_prefill_attention_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v, int n,
                                 int n_heads, int n_kv_heads, int head_dim, int causal,
                                 float scale, float* out, void* k_pool, void* v_pool,
                                 const int32_t* block_table, int block_tokens, int num_blocks,
                                 int kv_dtype, int start_pos, nyion_stream_t stream);

/* Chunked prefill after a cached prefix: prefill_slice with pos_offset =
 * n_hist (executor.rs:106-137), where row i of the chunk (absolute position
 * n_hist + i) attends to all n_hist history keys and to keys [0, i] of the
 * chunk (causal = 0: all n).  k_hist, v_hist [n_hist][n_kv_heads][D] bf16
 * hold the history (nyion_kv_gather_bf16 builds them from the paged cache);
 * n_hist = 0 is nyion_prefill_attention_bf16.  The other arguments are those
 * of nyion_prefill_attention_bf16; the KV write normally uses start_pos =
 * n_hist. */
int nyion_prefill_attention_bf16_ctx(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                     const uint16_t* k_hist, const uint16_t* v_hist, int n_hist,
                                     int n, int n_heads, int n_kv_heads, int head_dim, int causal,
                                     float scale, float* out, void* k_pool, void* v_pool,
                                     const int32_t* block_table, int block_tokens,
                                     int num_blocks, int kv_dtype, int start_pos,
                                     nyion_stream_t stream);

/* --------------------------------------------------------------- KV cache */

/* Writes n_tokens tokens of one sequence at positions start_pos.. into the
 * paged pools.  k, v: [n_tokens][n_kv_heads][head_dim] f32 (device).
 * Replaces PagedKVCache::save / save_at (cache.rs:613-679, 749-811) and the
 * CUDA gpu_copy_kv_layer / kernel_kv_save (fused_attention.cu:288-310,
 * 1462-1472).  Q4_20B quantises on device byte-identically to save(). */
int nyion_kv_write(void* k_pool, void* v_pool, const int32_t* block_table, int block_tokens,
                   int num_blocks, int n_kv_heads, int head_dim, int kv_dtype, int start_pos,
                   int n_tokens, const float* k, const float* v, nyion_stream_t stream);

/* One new token per sequence (the decode-step save of executor.rs:702):
 * k, v [batch][n_kv_heads][head_dim]; token written at positions[b]. */
int nyion_kv_append_batch(void* k_pool, void* v_pool, const int32_t* block_tables,
                          int max_blocks_per_seq, const int32_t* positions, int batch,
                          int block_tokens, int num_blocks, int n_kv_heads, int head_dim,
                          int kv_dtype, const float* k, const float* v, nyion_stream_t stream);

/* RoPE table of init_rope_lut (swamp-engine/src/ops.rs:20-37): d_lut
 * [max_ctx][head_dim/2][2] f32 = (cos, sin) of m * 10000^(-2k/head_dim),
 * computed on the host with the C library's powf/cosf/sinf (what the
 * reference's f32::powf/cos/sin call) and copied; returns when copied. */
int nyion_rope_lut_init(float* d_lut, int head_dim, int max_ctx, nyion_stream_t stream);

/* Decode-step QKV epilogue in one launch: apply_rope_ufc (ops.rs:40-64) on
 * q [batch][n_heads][D] (in place) and k [batch][n_kv_heads][D] at
 * positions[b] (table row min(pos, max_ctx-1)), then the rotated k and v
 * written into the paged pools at positions[b] (the save of executor.rs:
 * 699-702, Q4-20B quantised as nyion_kv_write does).  k and v are not
 * modified. */
int nyion_rope_kv_append(float* d_q, const float* d_k, const float* d_v, const float* d_lut,
                         int max_ctx, const int32_t* positions, int batch, int n_heads,
                         int n_kv_heads, int head_dim, void* k_pool, void* v_pool,
                         const int32_t* block_tables, int max_blocks_per_seq, int block_tokens,
                         int num_blocks, int kv_dtype, nyion_stream_t stream);

/* Debug/validation kernels sharing the decode kernels' index and unpack code:
 * gather tokens [0, n_tokens) of one sequence into [n_kv_heads][n_tokens][D]
 * f32 (dequantising Q4), and row-wise Q4-20B dequantise / quantise. */
int nyion_kv_gather(const void* pool, const int32_t* block_table, int block_tokens,
                    int num_blocks, int n_kv_heads, int head_dim, int kv_dtype, int n_tokens,
                    float* out, nyion_stream_t stream);
/* Tokens [0, n_tokens) of one sequence's paged K (or V) cache (the rows
 * ops::attention reads, ops.rs:170-278, through cache.rs's page lookup) as
 * [n_tokens][n_kv_heads][D] bf16, rounded to nearest even (Q4-20B
 * dequantised first): the history operand of
 * nyion_prefill_attention_bf16_ctx.  out 16-byte aligned. */
int nyion_kv_gather_bf16(const void* pool, const int32_t* block_table, int block_tokens,
                         int num_blocks, int n_kv_heads, int head_dim, int kv_dtype, int n_tokens,
                         uint16_t* out, nyion_stream_t stream);
int nyion_q4_dequant(const uint8_t* in, int64_t n_rows, int head_dim, float* out,
                     nyion_stream_t stream);
int nyion_q4_quantize(const float* in, int64_t n_rows, int head_dim, uint8_t* out,
                      nyion_stream_t stream);

/* ------------------------------------------------------ Q4_K weight GEMV */

/* out[r] = sum_j W[r][j] x[j] for a GGUF Q4_K matrix W (n_rows rows of
 * n_cols/256 blocks of 144 bytes: f16 d, f16 dmin, 12 bytes of 6-bit
 * scales/mins, 128 nibble bytes), f32 x and out, all device memory.
 * Replaces swamp_fused_gemv_q4k / fused_gemv_q4k
 * (swamp-kernels/src/fused_gemv_q4k.rs:59-99, 903-927), the Q4_K arm of
 * forward_linear (swamp-engine/src/linear.rs:99-189), with the f32
 * semantics of its scalar path (395-448).  n_cols a positive multiple of
 * 256; W and x 16-byte aligned.  out is written, not accumulated. */
int nyion_gemv_q4k(const uint8_t* d_w, const float* d_x, float* d_out, int n_rows, int n_cols,
                   nyion_stream_t stream);

/* Up to four matrices of n_cols columns that share x in one launch
 * (fused_gemv_q4k_multi, fused_gemv_q4k.rs:330-390; the executor's q/k/v
 * and gate/up projections).  d_ws, d_outs, row_counts are host arrays of
 * n_mats entries. */
int nyion_gemv_q4k_multi(const uint8_t* const* d_ws, const float* d_x, float* const* d_outs,
                         const int32_t* row_counts, int n_mats, int n_cols,
                         nyion_stream_t stream);

/* batch inputs against one matrix, W read once per four inputs
 * (fused_gemv_q4k_batched, fused_gemv_q4k.rs:456-485, the Q4_K arm of
 * forward_linear_batch, linear.rs:301-354): x [batch][x_stride] (x_stride
 * >= n_cols, a multiple of 4), out [batch][out_stride] (>= n_rows).  Each
 * output row equals nyion_gemv_q4k of its input bit for bit. */
int nyion_gemv_q4k_batched(const uint8_t* d_w, const float* d_x, int64_t x_stride, float* d_out,
                           int64_t out_stride, int n_rows, int n_cols, int batch,
                           nyion_stream_t stream);

/* ------------------------------------------------------ Q6_K weight GEMV */

/* out[r] = sum_j W[r][j] x[j] for a GGUF Q6_K matrix W (n_rows rows of
 * n_cols/256 blocks of 210 bytes: ql[128], qh[64], int8 scales[16], f16 d).
 * Replaces fused_gemv_q6k (swamp-kernels/src/fused_gemv_q6k.rs:22-43), the
 * Q6_K arm of forward_linear (swamp-engine/src/linear.rs:173-189), with the
 * f32 semantics of its scalar path (248-293), including its own f16
 * conversion of d (11-20: exact for normal values; zero and subnormal d
 * become about -2e34, infinities and NaNs finite values).  n_cols a positive
 * multiple of 256; W 2-byte aligned, x 16-byte aligned.  out is written. */
int nyion_gemv_q6k(const uint8_t* d_w, const float* d_x, float* d_out, int n_rows, int n_cols,
                   nyion_stream_t stream);

/* batch inputs against one Q6_K matrix, W read once per four inputs (the
 * Q6_K arm of fallback_gemv, linear.rs:437-465); strides and bit-for-bit
 * equality with the single call as for nyion_gemv_q4k_batched. */
int nyion_gemv_q6k_batched(const uint8_t* d_w, const float* d_x, int64_t x_stride, float* d_out,
                           int64_t out_stride, int n_rows, int n_cols, int batch,
                           nyion_stream_t stream);

/* ------------------------------------------- mixed Q4_K / Q6_K GEMV lists */

/* One GEMV of a list: the reference's (raw, x, out, n_rows, n_cols,
 * block_size) tuple of forward_gemvs_ring (linear.rs:472-525); block_bytes
 * 144 is Q4_K, 210 Q6_K (the is_q4k switch of forward_gemvs,
 * linear.rs:379-432).  Device pointers. */
typedef struct nyion_gemv_spec {
    const uint8_t* w;
    const float* x;
    float* out;
    int32_t n_rows;
    int32_t n_cols;
    int32_t block_bytes;
    int32_t reserved; /* 0 */
} nyion_gemv_spec;

/* Every spec of a host array: out = W x.  Specs of one format, n_cols and x
 * share a launch (up to four each; a Q4_K_M layer's q/k with its Q6_K v take
 * two launches).  All specs are checked before the first launch; a spec with
 * n_rows 0 is skipped.  No spec's out may overlap another spec's x or W. */
int nyion_gemv_specs(const nyion_gemv_spec* specs, int n_specs, nyion_stream_t stream);

/* ------------------------------------------- paged KV pool with host spill */

/* One step of the page policy.  CREATE: a new page took block `block`
 * (zeroed); EVICT: the page left block `block` for cold slot `slot`;
 * RELOAD: the page came back from cold slot `slot` into block `block`. */
enum { NYION_PAGE_CREATE = 0, NYION_PAGE_EVICT = 1, NYION_PAGE_RELOAD = 2 };
typedef struct nyion_page_event {
    int32_t kind;
    int32_t page;
    int32_t block;
    int32_t slot;
} nyion_page_event;

/* The PagedKVCache page policy (swamp-engine/src/cache.rs:277-336 page
 * creation and LRU, 407-477 eviction, 479-523 reload, 525-553 ensure_page /
 * ensure_pages_hot, 563-581 importance), host only: at most hot_limit hot
 * pages (physical blocks 0..hot_limit-1); eviction takes the lowest
 * importance among the LRU tail and the seven pages before it, into the
 * first free cold slot at or after a write cursor.  A full cold tier is an
 * error (the reference overwrites a used slot).  ensure makes pages
 * first..last hot in order (creating pages up to last as the reference
 * does) and reports the events; the range may not exceed hot_limit pages.
 * state returns 0 unmapped, 1 hot (where = block), 2 cold (where = slot),
 * -1 out of range; lru lists hot pages, most recent first. */
void* nyion_page_policy_create(int hot_limit, int cold_slots, int max_pages);
void  nyion_page_policy_destroy(void* policy);
int   nyion_page_policy_ensure(void* policy, int first_page, int last_page,
                               nyion_page_event* events, int max_events, int* n_events);
int   nyion_page_policy_record(void* policy, int page, double weight);
int   nyion_page_policy_reset(void* policy);
int   nyion_page_policy_state(void* policy, int page, int* where, double* importance);
int   nyion_page_policy_lru(void* policy, int* pages, int cap);

/* Device-resident paged KV cache of one sequence with a pinned-host cold
 * tier: the PagedKVCache contract (cache.rs) with HBM as the hot tier in
 * place of host RAM and pinned host memory in place of the cold file.  K
 * and V pools [n_layers][hot_blocks][n_kv_heads][block_tokens][row] (f32 or
 * Q4-20B rows) and the cold store are allocated at create.  ensure makes
 * pages first..last hot on `stream` (spill, reload and zeroing as copy
 * kernels on that stream) and updates the device block table
 * (nyion_kv_pool_table: [max_pages] int32, -1 for pages not in HBM), which
 * the decode and KV-write entry points take with max_blocks_per_seq =
 * max_pages and num_blocks = hot_blocks.  record_importance is the
 * executor's hand-off (executor.rs:751-755): positions whose importance
 * exceeds `threshold` add it to their page.  nyion_kv_pool_policy exposes
 * the pool's policy to the nyion_page_policy_state/lru queries (not to
 * ensure: that would leave device memory behind).  cold_slot gives the host
 * bytes of a slot ([layer][K|V][block bytes]). */
void*          nyion_kv_pool_create(int n_layers, int n_kv_heads, int head_dim, int block_tokens,
                                    int kv_dtype, int hot_blocks, int cold_slots, int max_pages);
void           nyion_kv_pool_destroy(void* pool);
int            nyion_kv_pool_layer(void* pool, int layer, void** k_pool, void** v_pool);
const int32_t* nyion_kv_pool_table(void* pool);
void*          nyion_kv_pool_policy(void* pool);
int            nyion_kv_pool_ensure(void* pool, int first_page, int last_page, nyion_stream_t stream);
int            nyion_kv_pool_record_importance(void* pool, const double* importance,
                                               int n_positions, double threshold);
int            nyion_kv_pool_stats(void* pool, int64_t* hot, int64_t* cold, int64_t* evictions,
                                   int64_t* reloads);
const void*    nyion_kv_pool_cold_slot(void* pool, int slot);

/* --------------------------------------------------------- HMA arena */

/* The HeterogeneousMemoryAllocator contract (swamp-tensors/src/hma.rs:5-9,
 * 30-36, 215-260): DeviceLocal allocations are carved from one hipMalloc
 * region (first-fit free list, 256-byte aligned; a free merges with free
 * neighbours), HostPinned from one hipHostMalloc region the same way,
 * UnifiedMapped from hipMallocManaged per allocation.  A full region is
 * NYION_ERR_OOM with a message.  Without a device (no HIP device, or not a
 * gfx950) create still succeeds, as the reference's allocator without a
 * DeviceAllocator (hma.rs:243-260): the host region is ordinary memory, and
 * DeviceLocal and UnifiedMapped requests fall back to it, returned as
 * HostPinned allocations with device_handle 0; nyion_hma_has_device tells
 * the two modes apart.  upload/download copy at most the live allocation's
 * size; reset frees every allocation at once. */
enum nyion_mem_location {
    NYION_MEM_HOST_PINNED = 0,
    NYION_MEM_DEVICE_LOCAL = 1,
    NYION_MEM_UNIFIED_MAPPED = 2
};
typedef struct nyion_allocation {
    void*    ptr;
    size_t   size;
    int32_t  location;
    int32_t  _pad;
    uint64_t device_handle; /* device address (0 for host pinned) */
} nyion_allocation;

void* nyion_hma_create(size_t device_bytes, size_t host_pinned_bytes);
int   nyion_hma_alloc(void* hma, size_t size, int location, nyion_allocation* out);
int   nyion_hma_free(void* hma, const nyion_allocation* a);
int   nyion_hma_upload(void* hma, const nyion_allocation* dst, const void* src, size_t bytes);
int   nyion_hma_download(void* hma, void* dst, const nyion_allocation* src, size_t bytes);
int   nyion_hma_reset(void* hma);
int   nyion_hma_stats(void* hma, int location, size_t* used, size_t* capacity);
int   nyion_hma_has_device(void* hma);
void  nyion_hma_destroy(void* hma);

/* ------------------------------------------------- swamp-kernels C-ABI */

/* Same symbols and signatures as swamp-kernels/src/lib.rs:36-85,181-223.
 * Host pointers; null arguments or n <= 0 return silently, as there.
 * mojo_softmax_padic runs the Q16.16 pipeline of the reference's AVX-512
 * branch on the GPU and returns when probs is written; up to 2^20 logits are
 * staged through a device array the library holds (8 MiB per device, calls
 * on one device take turns), longer arrays through device memory allocated
 * and freed by the call. */
void  mojo_softmax_padic(const float* logits, float* probs, int n, float temperature);
void* mojo_stokes_init(int head_dim);
void  mojo_stokes_append(void* cache, int token_id, const float* key, const float* value,
                         float score);
void  mojo_stokes_free(void* cache);

/* Device form of mojo_softmax_padic: d_logits, d_probs device f32[n]. */
int nyion_softmax_padic_dev(const float* d_logits, float* d_probs, int n, float temperature,
                            nyion_stream_t stream);
/* Stokes introspection: token count, and copies of the resident keys, values
 * and scores into host buffers ([count][head_dim], [count][head_dim], [count]). */
int nyion_stokes_count(const void* cache);
int nyion_stokes_read(const void* cache, float* keys, float* values, float* scores);

/* ------------------------------------------------------ Mojo kernel FFI */

/* The symbol the reference loads from libswamp_mojo.so
 * (swamp-gpu/src/mojo.rs:5,38: extern "C" fn(u64 x 5, i32 x 5)), with the
 * semantics of swamp-gpu/kernels/attention.mojo:38-152.  Host pointers passed
 * as integers: q [n_heads][head_dim] f32, k_q4 and v_q4 one K and one V
 * shared by all heads, row t at t * ceil(head_dim/32) * 20 f32 words (per
 * 32-element block: d, dmin, then the 16 nibble bytes as float values, low
 * nibble first), positions [n_sparse] int32 (>= 0), out [n_heads][head_dim]
 * f32.  Per head: scores dot(k, q) / sqrt(head_dim); tiles of 64 listed
 * positions; each tile's weights are exp(s - m) / d with the running (m, d)
 * after that tile (the output of earlier tiles is not rescaled), weights
 * below 1e-8 skipped.  window and global_stride are accepted and unused, as
 * in the reference.  The call copies its operands through a per-device
 * 16 MiB staging array (calls on one device take turns); a call whose q,
 * out, K/V rows up to the largest position and positions need more copies
 * through device memory it allocates and frees for the call.  It returns
 * when out is written.  On an error out is left unchanged and
 * nyion_last_error() says why. */
void  sparse_attention_q4(uint64_t q, uint64_t k_q4, uint64_t v_q4, uint64_t positions, uint64_t out,
                          int n_heads, int head_dim, int n_sparse, int window, int global_stride);

#ifdef __cplusplus
}
#endif
#endif /* NYION_HIP_H */
