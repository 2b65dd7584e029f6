// layer_state.hip — per-layer sliding-window KV rings and the Fugu attention
// policy of the GPU decode path.
//
// Ring state.  PerLayerGpuState (swamp-engine/src/scheduler.rs:36-178) keeps
// a device ring of `window` K/V slots: upload_kv_async writes token `pos` at
// slot pos % window (107-116) and execute_attention_async runs the Attention
// node over min(seq_len, window) slots (140-147), then copies the output back
// (160-167).  Here every layer has its own ring, laid out as the node reads
// it, [n_kv_heads][window][head_dim] f32, and the node is
// nyion_attention_node with the ring's scores buffer as split-K scratch.
// (In the reference all layers share one f16 ring that receives raw f32
// bytes; the intended sliding-window semantics are what is kept.)
//
// Policy.  FuguOrchestrator::decide_attention (swamp-engine/src/fugu.rs:
// 129-170) picks Full / Sparse / SparseWithDSPark per decode step; the
// executor maps them to attention_tracked, attention_sparse (global stride
// 64) and attention_fugu (executor.rs:742-763).  The DSPark position set of
// attention_fugu (ops.rs:463-484) is built on the device, one sequence per
// workgroup, for nyion_paged_decode_attention_positions.
#include <string.h>

#include "common.hpp"

namespace nyion {

struct LayerState {
    int window, n_heads, n_kv_heads, head_dim, n_layers;
    float* k = nullptr;       // [n_layers][n_kv_heads][window][head_dim]
    float* v = nullptr;
    float* q = nullptr;       // [n_heads][head_dim]
    float* out = nullptr;     // [n_heads][head_dim]
    float* scores = nullptr;  // [n_heads][window]: split-K scratch of the node
    hipStream_t stream = nullptr;
    size_t layer_floats() const { return (size_t)n_kv_heads * window * head_dim; }
};

// attention_fugu position set of one sequence (ops.rs:445-541): sentinels
// stride*g (g < min(ws/stride, 128)), the window [ws, valid_end], then each
// DSPark position <= valid_end not already present, in input order.
__global__ __launch_bounds__(256) void fugu_positions_kernel(
    const int32_t* ctx_lens, const int32_t* q_pos, int window, int sentinel_stride,
    const int32_t* dspark, int n_dspark, int dspark_stride, int32_t* positions, int max_positions,
    int32_t* n_positions) {
    const int b = blockIdx.x;
    const int len = ctx_lens[b];
    const int qp = q_pos ? q_pos[b] : len - 1;
    int32_t* out = positions + (long long)b * max_positions;
    if (len <= 0 || qp < 0) {
        if (threadIdx.x == 0) n_positions[b] = 0;
        return;
    }
    const int ve = min(qp, len - 1);
    const int ws = ve > window ? ve - window + 1 : 0;  // strict '>' (ops.rs:468)
    const int n_sent = sentinel_stride > 0 ? min(ws / sentinel_stride, 128) : 0;
    const int n_win = ve - ws + 1;
    const int base = n_sent + n_win;
    for (int i = threadIdx.x; i < base && i < max_positions; i += 256)
        out[i] = i < n_sent ? i * sentinel_stride : ws + (i - n_sent);
    // DSPark extras: one thread keeps the order and the first-occurrence rule
    if (threadIdx.x == 0) {
        const int32_t* dp = dspark + (long long)b * dspark_stride;
        int n = base;
        for (int i = 0; i < n_dspark; i++) {
            const int p = dp[i];
            if (p < 0 || p > ve) continue;
            bool present = (p >= ws) ||
                           (n_sent > 0 && p % sentinel_stride == 0 && p / sentinel_stride < n_sent);
            for (int k = 0; k < i && !present; k++) present = dp[k] == p;
            if (present) continue;
            if (n < max_positions) out[n] = p;
            n++;
        }
        n_positions[b] = min(n, max_positions);
    }
}

}  // namespace nyion

using namespace nyion;

extern "C" {

void* nyion_layer_state_create(int window, int n_heads, int n_kv_heads, int head_dim,
                               int n_layers) {
    clear_error();
    if (require_device() != NYION_OK) return nullptr;
    if (window <= 0 || n_heads <= 0 || n_kv_heads <= 0 || n_layers <= 0 ||
        n_heads % n_kv_heads || (head_dim != 64 && head_dim != 128)) {
        set_error(NYION_ERR_INVALID, "layer state: window %d heads %d/%d head_dim %d layers %d",
                  window, n_heads, n_kv_heads, head_dim, n_layers);
        return nullptr;
    }
    LayerState* s = new LayerState{window, n_heads, n_kv_heads, head_dim, n_layers};
    const size_t kv = s->layer_floats() * n_layers * sizeof(float);
    bool ok = hipMalloc(&s->k, kv) == hipSuccess && hipMalloc(&s->v, kv) == hipSuccess &&
              hipMalloc(&s->q, (size_t)n_heads * head_dim * sizeof(float)) == hipSuccess &&
              hipMalloc(&s->out, (size_t)n_heads * head_dim * sizeof(float)) == hipSuccess &&
              hipMalloc(&s->scores, (size_t)n_heads * window * sizeof(float)) == hipSuccess &&
              hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking) == hipSuccess;
    // zeroed rings: slots never written read as zeros, never as stale memory
    ok = ok && hipMemset(s->k, 0, kv) == hipSuccess && hipMemset(s->v, 0, kv) == hipSuccess;
    if (!ok) {
        (void)hipGetLastError();
        set_error(NYION_ERR_OOM, "layer state: device allocation of %zu bytes failed", 2 * kv);
        if (s->stream) (void)hipStreamDestroy(s->stream);
        (void)hipFree(s->k);
        (void)hipFree(s->v);
        (void)hipFree(s->q);
        (void)hipFree(s->out);
        (void)hipFree(s->scores);
        delete s;
        return nullptr;
    }
    return s;
}

int nyion_layer_state_upload_kv(void* state, int layer, const float* h_k, const float* h_v,
                                int pos) {
    clear_error();
    LayerState* s = (LayerState*)state;
    if (!s || !h_k || !h_v) return set_error(NYION_ERR_INVALID, "layer state upload: null argument");
    if (layer < 0 || layer >= s->n_layers || pos < 0)
        return set_error(NYION_ERR_INVALID, "layer state upload: layer %d pos %d", layer, pos);
    const size_t slot = (size_t)(pos % s->window);
    const size_t row = (size_t)s->head_dim * sizeof(float);
    const size_t off = (size_t)layer * s->layer_floats() + slot * s->head_dim;
    // [n_kv_heads][D] host rows -> ring rows of each head (pitch window*D)
    NYION_CHECK_HIP(hipMemcpy2DAsync(s->k + off, row * s->window, h_k, row, row, s->n_kv_heads,
                                     hipMemcpyHostToDevice, s->stream));
    NYION_CHECK_HIP(hipMemcpy2DAsync(s->v + off, row * s->window, h_v, row, row, s->n_kv_heads,
                                     hipMemcpyHostToDevice, s->stream));
    return NYION_OK;
}

int nyion_layer_state_attention(void* state, int layer, const float* h_q, float* h_out, int pos,
                                int seq_len) {
    clear_error();
    LayerState* s = (LayerState*)state;
    (void)pos;
    if (!s || !h_q || !h_out) return set_error(NYION_ERR_INVALID, "layer state attention: null argument");
    if (layer < 0 || layer >= s->n_layers)
        return set_error(NYION_ERR_INVALID, "layer state attention: layer %d", layer);
    const int attn_len = seq_len < s->window ? seq_len : s->window;
    if (attn_len <= 0) return set_error(NYION_ERR_INVALID, "layer state attention: seq_len %d", seq_len);
    const size_t qbytes = (size_t)s->n_heads * s->head_dim * sizeof(float);
    NYION_CHECK_HIP(hipMemcpyAsync(s->q, h_q, qbytes, hipMemcpyHostToDevice, s->stream));
    const size_t off = (size_t)layer * s->layer_floats();
    int rc = nyion_attention_node(s->q, s->k + off, s->v + off, s->scores, s->out,
                                  (uint32_t)s->n_heads, (uint32_t)s->n_kv_heads, (uint32_t)attn_len,
                                  (uint32_t)s->head_dim, (uint32_t)s->window, NYION_KV_F32,
                                  s->stream);
    if (rc != NYION_OK) return rc;
    NYION_CHECK_HIP(hipMemcpyAsync(h_out, s->out, qbytes, hipMemcpyDeviceToHost, s->stream));
    NYION_CHECK_HIP(hipStreamSynchronize(s->stream));
    return NYION_OK;
}

int nyion_layer_state_sync(void* state) {
    clear_error();
    LayerState* s = (LayerState*)state;
    if (!s) return set_error(NYION_ERR_INVALID, "layer state sync: null state");
    NYION_CHECK_HIP(hipStreamSynchronize(s->stream));
    return NYION_OK;
}

void nyion_layer_state_destroy(void* state) {
    LayerState* s = (LayerState*)state;
    if (!s) return;
    (void)hipStreamSynchronize(s->stream);
    (void)hipStreamDestroy(s->stream);
    (void)hipFree(s->k);
    (void)hipFree(s->v);
    (void)hipFree(s->q);
    (void)hipFree(s->out);
    (void)hipFree(s->scores);
    delete s;
}

int nyion_fugu_config_default(int n_heads, int head_dim, nyion_fugu_config* cfg) {
    clear_error();
    if (!cfg) return set_error(NYION_ERR_INVALID, "fugu config: null");
    memset(cfg, 0, sizeof *cfg);
    cfg->sparse_attention_threshold = 512;  // FuguOrchestrator::new (fugu.rs:104-117)
    cfg->sparse_window = 256;
    cfg->sparse_random_samples = 32;
    cfg->n_heads = n_heads;
    cfg->head_dim = head_dim;
    return NYION_OK;
}

int nyion_fugu_decide_attention(const nyion_system_snapshot* state, const nyion_fugu_config* cfg,
                                nyion_attention_strategy* out) {
    clear_error();
    if (!state || !cfg || !out) return set_error(NYION_ERR_INVALID, "fugu decide: null argument");
    memset(out, 0, sizeof *out);
    if (state->is_prefill) {
        out->kind = NYION_ATTN_FULL;
        return NYION_OK;
    }
    // thermal-aware threshold: predictive throttle goes sparse earlier
    const long long thr = state->predictive_throttle
                              ? (cfg->sparse_attention_threshold > 256
                                     ? cfg->sparse_attention_threshold - 256
                                     : 0)
                              : cfg->sparse_attention_threshold;
    if ((long long)state->seq_len <= thr) {
        out->kind = NYION_ATTN_FULL;
        return NYION_OK;
    }
    out->window = state->predictive_throttle ? cfg->sparse_window / 2 : cfg->sparse_window;
    int dspark = 0;
    if (state->dspark_accept_rate > 0.0 && state->seq_len > 2048)
        dspark = cfg->n_heads < 4 ? 4 : (cfg->n_heads > 64 ? 64 : cfg->n_heads);
    if (dspark > 0) {
        out->kind = NYION_ATTN_SPARSE_DSPARK;
        out->sentinel_stride = cfg->head_dim;
        out->num_dspark = dspark;
    } else {
        out->kind = NYION_ATTN_SPARSE;
        out->num_random = cfg->sparse_random_samples;
    }
    return NYION_OK;
}

int nyion_fugu_positions(const int32_t* d_ctx_lens, const int32_t* d_q_pos, int batch, int window,
                         int sentinel_stride, const int32_t* d_dspark, int n_dspark,
                         int dspark_stride, int32_t* d_positions, int max_positions,
                         int32_t* d_n_positions, nyion_stream_t stream) {
    clear_error();
    int rc;
    if ((rc = require_device()) != NYION_OK) return rc;
    if (!d_ctx_lens || !d_positions || !d_n_positions || (n_dspark > 0 && !d_dspark))
        return set_error(NYION_ERR_INVALID, "fugu positions: null argument");
    if (batch <= 0 || window < 0 || n_dspark < 0 || max_positions <= 0 ||
        (n_dspark > 0 && dspark_stride < n_dspark))
        return set_error(NYION_ERR_INVALID, "fugu positions: batch %d window %d dspark %d/%d max %d",
                         batch, window, n_dspark, dspark_stride, max_positions);
    if ((long long)max_positions < 128LL + window + 1 + n_dspark)
        return set_error(NYION_ERR_INVALID,
                         "fugu positions: max_positions %d < 128 + window + 1 + n_dspark (%lld)",
                         max_positions, 128LL + window + 1 + n_dspark);
    if (batch > 65535) return set_error(NYION_ERR_UNSUPPORTED, "fugu positions: batch %d", batch);
    hipLaunchKernelGGL(fugu_positions_kernel, dim3(batch), dim3(256), 0, (hipStream_t)stream,
                       d_ctx_lens, d_q_pos, window, sentinel_stride, d_dspark, n_dspark,
                       dspark_stride, d_positions, max_positions, d_n_positions);
    return check_launch("fugu positions");
}

}  // extern "C"
