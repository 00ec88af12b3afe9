/* llama_kvmem_hooks.h -- KVMem's llama.cpp hook entry points on the MI355X
 * recall path, with the reference's names and signatures:
 *
 *   attn-qk capture hook   src/adapter/llama-kvmem-hooks.h:43-98 (params,
 *                          execution states, register / new graph /
 *                          harvest / reuse / stamp / capture predicates)
 *   memory-factory hook    llama_memory_kvmem_maybe_create,
 *                          backends/patches/llamacpp-kvmem.patch:2102, 2403
 *                          (C++ linkage, below)
 *
 * The hooks drive a kvmem_hip::RecallMemory bound to the calling thread's
 * execution state: captured K goes into the device page sums straight from
 * the engine's tensor, the Query span's rows stay on the device.  ggml and
 * llama types are opaque here; the engine registers a bridge (C++, below)
 * that reads its tensors and describes its model, a few lines compiled with
 * the engine's headers.  The reference needs none because it includes ggml;
 * this library does not, so it has no compile-time dependency on one engine
 * revision. */
#ifndef KVMEM_HIP_LLAMA_KVMEM_HOOKS_H
#define KVMEM_HIP_LLAMA_KVMEM_HOOKS_H

#include <stdbool.h>
#include <stdint.h>

struct ggml_tensor;
struct ggml_context;
struct ggml_cgraph;
struct ggml_backend_sched;
typedef int32_t llama_pos;
typedef int32_t llama_token;

#ifdef __cplusplus
extern "C" {
#endif

/* Field for field llama_kvmem_params (llama-kvmem-hooks.h:21-46). */
struct llama_kvmem_params {
    bool enabled;
    uint32_t block_tokens;  /* 0 -> 32 */
    uint32_t budget;        /* tokens; 0 -> n_ctx (every page) */
    uint32_t gen_reserve;   /* tokens; 0 -> 256 */
    uint32_t sink_tokens;   /* 0 -> one block */
    uint32_t recent_tokens;
    int32_t method;         /* 0 recency, 1 retrieval */
    bool lrfu;
    double lrfu_lambda;
    double lrfu_top_fraction;
    int32_t score_agg;      /* 0 mean, 1 max within a GQA group */
    bool query_meanq_cosine;
    double graph_alpha;
    int32_t query_begin;    /* original token position, -1 = unset */
    int32_t query_end;      /* exclusive, -1 = end of prompt */
    int32_t force_pos;
    float gpu_memory_ratio;
    float gpu_high_watermark;
    float gpu_low_watermark;
    uint64_t cpu_bytes;
    bool harvest_v;
    uint64_t payload_host_bytes;
    uint64_t payload_disk_bytes;
    const char *payload_disk_dir;
    int32_t mtp_state;
};

/* Parameters of the calling thread's execution state (NULL: defaults,
 * disabled); read by the memory factory. */
void llama_kvmem_set_params(const struct llama_kvmem_params *params);
const struct llama_kvmem_params *llama_kvmem_get_params(void);

/* Isolated hook and recall state for one target context.  Activate before
 * creating or using its context, on every calling thread; never active on
 * two threads at once.  Exchanging NULL restores the process-wide default. */
struct llama_kvmem_execution_state;
struct llama_kvmem_execution_state *llama_kvmem_execution_create(void);
void llama_kvmem_execution_free(struct llama_kvmem_execution_state *state);
struct llama_kvmem_execution_state *llama_kvmem_execution_exchange(struct llama_kvmem_execution_state *state);

/* Always false: the harvest runs after the whole ubatch, so ggml never
 * splits the graph for this library. */
bool llama_kvmem_eval_callback(struct ggml_tensor *t, bool ask, void *user_data);

/* Graph build: a node to read after the graph runs ('k' pre-RoPE K, 'q'
 * Query, 'v' ignored) for layer il. */
void llama_kvmem_register_capture(struct ggml_tensor *t, int il, char which);
/* Graph build: one layer's attention operands for the attention-feedback
 * sampler (sampled page masses, read after the graph runs; max_bias != 0 is
 * declined as in the reference).  ctx and graph are not used: no node is
 * added. */
void llama_kvmem_capture_attention(struct ggml_context *ctx, struct ggml_cgraph *graph, struct ggml_tensor *q,
                                   struct ggml_tensor *k, struct ggml_tensor *mask, float scale, float max_bias,
                                   float softcap, int layer);
/* A new graph starts: forget the previous graph's registrations.  is_mtp:
 * the MTP draft's graph (no capture here). */
void llama_kvmem_capture_on_new_graph(int is_mtp);
/* After the ubatch's graph: synchronizes the scheduler (through the
 * bridge) and harvests the registered nodes. */
void llama_kvmem_harvest_ubatch(struct ggml_backend_sched *sched, int is_mtp);
/* True when the ubatch overlaps the Query span and Q nodes are needed. */
bool llama_kvmem_ubatch_needs_q_capture(uint32_t n_tokens, uint32_t n_pos, const llama_pos *pos);
/* False when the last graph's capture topology does not fit this ubatch. */
bool llama_kvmem_capture_can_reuse(uint32_t n_tokens, uint32_t n_pos, const llama_pos *pos, int is_mtp);
/* Topology stamp of the last target graph; 0 when no memory is bound. */
uint64_t llama_kvmem_capture_stamp(void);
bool llama_kvmem_want_prefill_capture(void);
bool llama_kvmem_want_q_capture(uint32_t n_tokens, uint32_t n_pos, const llama_pos *pos);
void llama_kvmem_reset_query(void);
bool llama_kvmem_want_decode_mean(void);
void llama_kvmem_end_prefill_capture(void);
void llama_kvmem_pin_working_set(void);

#ifdef __cplusplus
}  /* extern "C" */

#include <functional>
#include <memory>
#include <string>
#include <vector>

#include "kvmem_hip/kvmem_memory.hpp"

struct llama_model;
struct llama_memory_params;
struct llama_cparams;
struct llama_memory_i;

/* The memory-factory hook, called first in llama_model::create_memory:
 * nullptr declines (KVMem disabled in this execution state, an MTP draft,
 * recurrent or sliding-window models, more than one sequence), else the
 * engine's memory object around a RecallMemory planned from the model and
 * the execution state's parameters, bound to the execution state. */
llama_memory_i *llama_memory_kvmem_maybe_create(const llama_model &model, const llama_memory_params &params,
                                                const llama_cparams &cparams);

namespace kvmem_hip {

/* What the factory needs to know of a model (from llama_model and the
 * memory and context parameters). */
struct ModelFacts {
    uint32_t n_layer = 0;
    std::vector<uint32_t> attention_layers;  // layers with KV (empty: all)
    uint32_t query_heads = 0, kv_heads = 0, head_dim = 0;
    uint32_t n_ctx_seq = 0, n_seq_max = 1;
    bool mtp_context = false;  // the MTP draft context
    bool companion = false;    // a draft companion keeping its native cache
    bool recurrent = false;    // purely recurrent architecture
    bool sliding_window = false;
    int device = 0;
    std::string model;
};

/* The engine side: compiled with the engine's headers (INTEGRATION.md
 * shows the llama.cpp version). */
struct EngineBridge {
    std::function<bool(const llama_model &, const llama_memory_params &, const llama_cparams &, ModelFacts &)>
        describe;
    // the engine's llama_memory_i owning the recall memory
    std::function<llama_memory_i *(std::unique_ptr<RecallMemory>, const ModelFacts &)> wrap;
    std::function<bool(const ggml_tensor *, TensorView &)> tensor_view;
    std::function<void(ggml_backend_sched *)> synchronize;
};
void set_engine_bridge(EngineBridge bridge);

/* The memory plan the factory derives from the parameters (block size,
 * budget, sink and recent bands, Query span), exposed for the engine and
 * tests. */
RecallMemoryConfig plan_recall_memory(const llama_kvmem_params &params, const ModelFacts &facts);

/* The recall memory bound to the calling thread's execution state (the
 * factory binds the memory it creates; the engine's memory object unbinds
 * it when it is destroyed). */
RecallMemory *current_memory();
void bind_memory(RecallMemory *memory);
void unbind_memory(RecallMemory *memory);

/* Page masses of the attention samples harvested since the last call
 * (mean over sampled rows and layers, one value per page), then cleared. */
std::vector<double> take_attention_masses();

}  // namespace kvmem_hip
#endif  /* __cplusplus */

#endif
