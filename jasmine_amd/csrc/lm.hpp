// Private state of the decoder LM runner (jas_lm_*), shared by the runner (lm.hip) and the
// weight-file reader/writer (lm_io.hip).
#pragma once
#include "gemm.hpp"

#include <map>
#include <string>
#include <vector>

#define TRY(x)                                   \
    do {                                         \
        jas_status s_ = (x);                     \
        if (s_ != JAS_OK) return s_;             \
    } while (0)

namespace jas {

// A stacked weight tensor: `layers` matrices of [rows][cols]; packed matrices use the
// MFMA-native layout of weight_pack_offset with rows padded to a multiple of 16.
// bf16 (packed only): 2-byte elements in the pair-tile layout; offsets and strides stay in
// float (4-byte) units of the arena, so a bf16 layer occupies half as many of them.
struct Tensor {
    size_t off = 0, count = 0;
    int layers = 1, rows = 1, cols = 1;
    bool packed = false, bf16 = false;
    long lstride() const
    {
        // bf16 packed layers use the pair-tile layout: K padded to a multiple of 32
        const long elems = (long)(packed ? (rows + 15) / 16 * 16 : rows) * (bf16 ? k32_of(cols) : cols);
        return bf16 ? elems / 2 : elems;
    }
};

} // namespace jas

struct jas_lm {
    jas_lm_config cfg{};
    hipStream_t stream = nullptr;
    float *arena = nullptr;
    size_t arena_count = 0;
    std::map<std::string, jas::Tensor> tensors;
    // KV cache
    float *kc = nullptr, *vc = nullptr;  // bf16 elements when cfg.kv_bf16
    long kv_layer = 0, kv_sb = 0, kv_sh = 0;  // in elements
    // decode buffers [max_batch][...]
    float *x = nullptr, *h = nullptr, *q = nullptr, *att = nullptr, *ff = nullptr, *logits = nullptr;
    int32_t *ids = nullptr, *pos = nullptr, *seqlens = nullptr, *hist = nullptr;
    int hist_cap = 0;
    // device-side decode state for graph replay: [0] next position, [1] first position of
    // the current jas_lm_generate call (its id history is indexed from there)
    int32_t *dstate = nullptr;
    // the LM head's per-workgroup greedy picks (allocated once: graph-safe)
    float *amax_v = nullptr;
    int *amax_i = nullptr;
    // one decode step captured as a HIP graph (for this batch size and id-history buffer)
    hipGraphExec_t graph = nullptr;
    bool use_graph = true;
    int graph_B = 0, graph_cap = 0;
    const int32_t *graph_hist = nullptr;
    void *attn_ws = nullptr;
    unsigned *attn_ctr = nullptr;  // [max_batch * n_head] split-arrival counters (zero between steps)
    double2 *rope_tab = nullptr;  // LLaMA: [max_ctx][dh / 2] (cos, sin) for the QKV epilogue
    float *part = nullptr;  // K-split partials of the residual projections [split][16][d]
    int ks_o = 1, ks_d = 1;
    size_t attn_ws_bytes = 0;
    // prefill buffers (grown on demand)
    float *pX = nullptr, *pH = nullptr, *pQKV = nullptr, *pATT = nullptr, *pG = nullptr, *pU = nullptr, *pFF = nullptr;
    int32_t *pIds = nullptr, *pPos = nullptr;
    long p_tokens = 0;
    int B = 0;         // active batch
    int position = 0;  // tokens already in the cache
    // profiling
    bool prof = false;
    std::vector<hipEvent_t> ev;
    std::vector<int> ev_cls;
    size_t ev_used = 0;
    // jas_lm_project's last launch on the caller's stream: the runner's stream waits on it
    hipEvent_t proj_done = nullptr;

    const float *W(const char *n) const
    {
        auto it = tensors.find(n);
        return it == tensors.end() || it->second.count == 0 ? nullptr : arena + it->second.off;
    }
    // layer l of a stacked tensor (nullptr when the model kind lacks it)
    const float *LW(const char *n, int l) const
    {
        auto it = tensors.find(n);
        if (it == tensors.end() || it->second.count == 0) return nullptr;
        return arena + it->second.off + (long)l * it->second.lstride();
    }
    int dh() const { return cfg.d_model / cfg.n_head; }
    bool wbf16() const { return cfg.weight_bf16 != 0; }
    size_t kv_es() const { return cfg.kv_bf16 ? 2 : 4; }
    // layer l of a KV cache (element type per cfg.kv_bf16)
    float *kv_layer_ptr(float *base, int l) const { return (float *)((char *)base + (size_t)l * kv_layer * kv_es()); }
};
