// kvmem_hooks.cpp -- KVMem's llama.cpp hook entry points and memory-factory
// hook over RecallMemory (include/kvmem_hip/llama_kvmem_hooks.h).
//
// Execution states (llama-kvmem-hooks.h:48-58): each holds the parameters,
// the bound recall memory and the attention samples of one target context;
// a thread uses the state it activated, else the process-wide default.
#include "kvmem_hip/llama_kvmem_hooks.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <stdexcept>

struct llama_kvmem_execution_state {
    llama_kvmem_params params{};
    std::string disk_dir;  // owns params.payload_disk_dir
    kvmem_hip::RecallMemory *memory = nullptr;
    struct Attention {
        const ggml_tensor *q, *k, *mask;
        float scale, softcap;
        int layer;
    };
    std::vector<Attention> attention;
    std::unique_ptr<kvmem_hip::AttentionSamplerHip> sampler;
    std::vector<double> masses;
    uint32_t mass_samples = 0;
};

namespace {

llama_kvmem_params default_params() {
    llama_kvmem_params p{};
    p.enabled = false;
    p.method = 1;
    p.lrfu_lambda = 0.5;
    p.lrfu_top_fraction = 0.9;
    p.graph_alpha = 0.2;
    p.query_begin = -1;
    p.query_end = -1;
    p.force_pos = -1;
    return p;
}

llama_kvmem_execution_state &default_state() {
    static llama_kvmem_execution_state s{default_params()};
    return s;
}
thread_local llama_kvmem_execution_state *t_state = nullptr;
llama_kvmem_execution_state &state() { return t_state ? *t_state : default_state(); }

std::mutex g_bridge_mutex;
kvmem_hip::EngineBridge &bridge() {
    static kvmem_hip::EngineBridge b;
    return b;
}

// Hooks run inside the engine's C code paths: no exception crosses them.
template <class F> void guarded(const char *what, F &&f) {
    try {
        f();
    } catch (const std::exception &e) {
        std::fprintf(stderr, "kvmem_hip %s: %s\n", what, e.what());
    }
}

uint32_t ceil_div(uint64_t a, uint32_t b) { return uint32_t((a + b - 1) / b); }
uint32_t align_up(uint64_t a, uint32_t b) { return uint32_t((a + b - 1) / b * b); }

kvmem_hip::AttentionTensor attention_view(const kvmem_hip::TensorView &v) {
    kvmem_hip::AttentionTensor a;
    a.data = v.data;
    a.type = v.type;
    for (int i = 0; i < 3; ++i) {
        a.ne[i] = v.ne[i];
        a.nb[i] = v.nb[i];
    }
    return a;
}

// The attention samples of the harvested graph: every 128th row of the
// ubatch and its last, page masses added per page.
void harvest_attention(llama_kvmem_execution_state &st, uint32_t block_tokens) {
    if (st.attention.empty()) return;
    auto &b = bridge();
    if (!b.tensor_view) return;
    if (!st.sampler) st.sampler = std::make_unique<kvmem_hip::AttentionSamplerHip>();
    for (const auto &a : st.attention) {
        kvmem_hip::TensorView q, k, m;
        if (!b.tensor_view(a.q, q) || !b.tensor_view(a.k, k) || !b.tensor_view(a.mask, m)) continue;
        const uint32_t rows = uint32_t(q.ne[1]);
        std::vector<uint32_t> sample;
        for (uint32_t r = 127; r < rows; r += 128) sample.push_back(r);
        if (rows && (sample.empty() || sample.back() != rows - 1)) sample.push_back(rows - 1);
        std::vector<std::vector<float>> out;
        if (!st.sampler->score(attention_view(q), attention_view(k), attention_view(m), a.scale, a.softcap,
                               block_tokens, sample, out))
            continue;
        for (const auto &row : out) {
            if (st.masses.size() < row.size()) st.masses.resize(row.size(), 0.0);
            for (size_t p = 0; p < row.size(); ++p) st.masses[p] += row[p];
            ++st.mass_samples;
        }
    }
    st.attention.clear();
}

}  // namespace

// ---- parameters and execution states ---------------------------------------------
extern "C" void llama_kvmem_set_params(const llama_kvmem_params *params) {
    auto &st = state();
    st.params = params ? *params : default_params();
    st.disk_dir = st.params.payload_disk_dir ? st.params.payload_disk_dir : "";
    st.params.payload_disk_dir = params && params->payload_disk_dir ? st.disk_dir.c_str() : nullptr;
}
extern "C" const llama_kvmem_params *llama_kvmem_get_params(void) { return &state().params; }

extern "C" llama_kvmem_execution_state *llama_kvmem_execution_create(void) {
    auto *s = new llama_kvmem_execution_state;
    s->params = default_params();
    return s;
}
extern "C" void llama_kvmem_execution_free(llama_kvmem_execution_state *s) {
    if (!s) return;
    if (t_state == s) t_state = nullptr;
    delete s;
}
extern "C" llama_kvmem_execution_state *llama_kvmem_execution_exchange(llama_kvmem_execution_state *s) {
    llama_kvmem_execution_state *previous = t_state;
    t_state = s;
    return previous;
}

// ---- capture hook -------------------------------------------------------------------
extern "C" bool llama_kvmem_eval_callback(ggml_tensor *, bool, void *) { return false; }

extern "C" void llama_kvmem_register_capture(ggml_tensor *t, int il, char which) {
    if (auto *m = state().memory) m->register_capture(t, il, which);
}

extern "C" void llama_kvmem_capture_attention(ggml_context *, ggml_cgraph *, ggml_tensor *q, ggml_tensor *k,
                                              ggml_tensor *mask, float scale, float max_bias, float softcap,
                                              int layer) {
    auto &st = state();
    if (!st.memory || !q || !k || !mask || max_bias != 0.0f || !st.memory->owns_layer(layer)) return;
    st.attention.push_back({q, k, mask, scale, softcap, layer});
}

extern "C" void llama_kvmem_capture_on_new_graph(int is_mtp) {
    auto &st = state();
    if (is_mtp || !st.memory) return;
    st.memory->capture_on_new_graph();
    st.attention.clear();
}

extern "C" void llama_kvmem_harvest_ubatch(ggml_backend_sched *sched, int is_mtp) {
    auto &st = state();
    if (is_mtp || !st.memory) return;
    guarded("harvest", [&] {
        auto &b = bridge();
        if (b.synchronize && sched) b.synchronize(sched);
        st.memory->harvest([&b](const void *t, kvmem_hip::TensorView &v) {
            return b.tensor_view && b.tensor_view(static_cast<const ggml_tensor *>(t), v);
        });
        harvest_attention(st, st.memory->config().block_tokens);
    });
}

// llama-kvmem-capture.cpp:87-105: with a memory bound, its Query span; else
// the parameters' span for retrieval.
extern "C" bool llama_kvmem_ubatch_needs_q_capture(uint32_t n_tokens, uint32_t n_pos, const llama_pos *pos) {
    (void)n_pos;
    auto &st = state();
    if (st.memory) return st.memory->query_overlaps(n_tokens, pos);
    const auto &p = st.params;
    if (!p.enabled || p.method != 1 || p.query_begin < 0 || !n_tokens) return false;
    if (!pos) return true;
    const int32_t end = p.query_end > 0 ? p.query_end : (1 << 30);
    for (uint32_t i = 0; i < n_tokens; ++i)
        if (pos[i] >= p.query_begin && pos[i] < end) return true;
    return false;
}

extern "C" bool llama_kvmem_capture_can_reuse(uint32_t n_tokens, uint32_t n_pos, const llama_pos *pos, int is_mtp) {
    auto *m = state().memory;
    return is_mtp || !m || m->capture_can_reuse(n_tokens, n_pos, pos);
}
extern "C" uint64_t llama_kvmem_capture_stamp(void) {
    auto *m = state().memory;
    return m ? m->capture_stamp() : 0;
}
extern "C" bool llama_kvmem_want_prefill_capture(void) {
    auto *m = state().memory;
    return m && m->want_prefill_capture();
}
extern "C" bool llama_kvmem_want_q_capture(uint32_t n_tokens, uint32_t n_pos, const llama_pos *pos) {
    auto *m = state().memory;
    return m && m->want_q_capture() && llama_kvmem_ubatch_needs_q_capture(n_tokens, n_pos, pos);
}
extern "C" void llama_kvmem_reset_query(void) {
    if (auto *m = state().memory) m->reset_query();
}
extern "C" bool llama_kvmem_want_decode_mean(void) {
    auto *m = state().memory;
    return m && m->want_decode_mean();
}
extern "C" void llama_kvmem_end_prefill_capture(void) {
    if (auto *m = state().memory) m->end_prefill_capture();
}
extern "C" void llama_kvmem_pin_working_set(void) {
    if (auto *m = state().memory) m->pin_working_set();
}

// ---- memory factory ---------------------------------------------------------------------
namespace kvmem_hip {

void set_engine_bridge(EngineBridge b) {
    std::lock_guard<std::mutex> lock(g_bridge_mutex);
    bridge() = std::move(b);
}

RecallMemory *current_memory() { return state().memory; }
void bind_memory(RecallMemory *m) { state().memory = m; }
void unbind_memory(RecallMemory *m) {
    auto &st = state();
    if (st.memory == m) {
        st.memory = nullptr;
        st.attention.clear();
    }
}

std::vector<double> take_attention_masses() {
    auto &st = state();
    std::vector<double> out = std::move(st.masses);
    if (st.mass_samples)
        for (double &v : out) v /= st.mass_samples;
    st.masses.clear();
    st.mass_samples = 0;
    return out;
}

// kvmem_compute_pool's token plan (llama-memory-kvmem.cpp:719-736) and the
// store bands of make_runtime_cfg: pages of block_tokens (0 -> 32) over the
// context; a budget (0 -> the whole context) aligned to pages; sink_tokens
// (0 -> one page) and recent_tokens rounded up to pages; the Query span.
RecallMemoryConfig plan_recall_memory(const llama_kvmem_params &p, const ModelFacts &f) {
    RecallMemoryConfig c;
    c.device = f.device;
    c.n_layer = f.n_layer;
    c.layers = f.attention_layers;
    c.query_heads = f.query_heads;
    c.kv_heads = f.kv_heads;
    c.head_dim = f.head_dim;
    c.block_tokens = p.block_tokens ? p.block_tokens : 32u;
    const uint32_t ctx_tokens = align_up(std::max<uint32_t>(f.n_ctx_seq, 1), c.block_tokens);
    c.max_pages = ctx_tokens / c.block_tokens;
    const uint32_t budget = p.budget ? align_up(p.budget, c.block_tokens) : ctx_tokens;
    c.budget_pages = budget >= ctx_tokens ? 0 : budget / c.block_tokens;
    c.sink_pages = p.sink_tokens ? ceil_div(p.sink_tokens, c.block_tokens) : 1;
    c.recent_pages = ceil_div(p.recent_tokens, c.block_tokens);
    c.aggregation = p.score_agg == 1 ? GqaScoreAggregation::Max : GqaScoreAggregation::Mean;
    c.tie = TieRule::HigherFirst;
    c.retrieval = p.method == 1;
    c.query_begin = p.query_begin;
    c.query_end = p.query_end;
    const int64_t span = p.query_begin >= 0 && p.query_end > p.query_begin ? int64_t(p.query_end) - p.query_begin : 256;
    c.max_query_rows = uint32_t(std::min<int64_t>(std::max<int64_t>(span, 1), 4096));
    c.model = f.model;
    return c;
}

}  // namespace kvmem_hip

// llama_memory_kvmem_maybe_create (llama-memory-kvmem.cpp:909-955): the
// decline rules in the reference's order, then a RecallMemory the engine
// wraps.  MTP drafts, companions and sliding-window models keep the
// engine's native cache here.
llama_memory_i *llama_memory_kvmem_maybe_create(const llama_model &model, const llama_memory_params &params,
                                                const llama_cparams &cparams) {
    auto &st = state();
    if (!st.params.enabled) return nullptr;
    kvmem_hip::EngineBridge b;
    {
        std::lock_guard<std::mutex> lock(g_bridge_mutex);
        b = bridge();
    }
    if (!b.describe || !b.wrap) {
        std::fprintf(stderr, "kvmem_hip: no engine bridge registered; KVMem declines\n");
        return nullptr;
    }
    kvmem_hip::ModelFacts f;
    if (!b.describe(model, params, cparams, f)) return nullptr;
    if (f.companion || f.mtp_context) return nullptr;
    if (f.recurrent) {
        std::fprintf(stderr, "kvmem_hip: KVMem skips purely recurrent models\n");
        return nullptr;
    }
    if (f.n_seq_max > 1) {
        std::fprintf(stderr, "kvmem_hip: KVMem requires n_seq_max=1 (got %u)\n", f.n_seq_max);
        return nullptr;
    }
    if (f.sliding_window) {
        std::fprintf(stderr, "kvmem_hip: KVMem skips sliding-window models\n");
        return nullptr;
    }
    llama_memory_i *out = nullptr;
    guarded("memory factory", [&] {
        auto mem = std::make_unique<kvmem_hip::RecallMemory>(kvmem_hip::plan_recall_memory(st.params, f));
        kvmem_hip::RecallMemory *raw = mem.get();
        out = b.wrap(std::move(mem), f);
        if (out) kvmem_hip::bind_memory(raw);
    });
    return out;
}
