// kvmem_memory.hpp -- the memory-backend side of KVMem's contract for the
// recall path, and the recall memory object behind the llama.cpp hooks.
//
//   contract types       kvmem/include/kvmem/memory_contract.hpp:27-140
//   MemoryTransfer /     memory_contract.hpp:175-195
//   MemoryBackend
//   RecallMemory         the recall part of llama_memory_kvmem
//                        (src/adapter/llama-memory-kvmem.cpp: register_capture
//                        :2952-2963, capture_on_new_graph :2965-2971,
//                        capture_can_reuse :2973-2987, capture_stamp
//                        :2989-3010, harvest_pending / harvest_capture
//                        :3566-3583, 3832-3880, query_contains / query_overlaps
//                        :4713-4725, score_retrieval :4604-4653), built on
//                        the device: captured K goes into GPU running sums
//                        straight from the engine's tensor, captured Query rows
//                        stay on the device, scoring and selection run there,
//                        and a prepared working set is restored by one gather.
// Errors: MemoryError with the contract's codes for plans and transfers,
// std::invalid_argument for geometry, std::runtime_error for device failures.
#pragma once

#include "kvmem_hip/kvmem_hip.hpp"

#include <functional>
#include <memory>
#include <string>
#include <vector>

namespace kvmem_hip {

// ---- contract types (memory_contract.hpp:27-140), field for field ----------
struct BackendIdentity {
    std::string backend, revision, model, state_schema;
    bool operator==(const BackendIdentity &o) const {
        return backend == o.backend && revision == o.revision && model == o.model && state_schema == o.state_schema;
    }
};
struct SessionIdentity {
    uint64_t id = 0;
    uint64_t incarnation = 0;
    bool operator==(const SessionIdentity &o) const { return id == o.id && incarnation == o.incarnation; }
};
struct MemoryCapabilities {
    uint32_t page_tokens = 0;
    uint64_t max_position = 0;
    bool native_payload = false;
    bool sparse_view = false;
    bool original_rope_positions = false;
    bool pre_rope_statistics = false;
    bool state_checkpoint = false;
    bool asynchronous_transfer = false;
};
struct MemoryDescriptor {
    BackendIdentity identity;
    PayloadLayout layout;
    MemoryCapabilities capabilities;
};
struct BlockDescriptor {
    SessionIdentity session;
    uint64_t id = 0;
    uint64_t original_start = 0;
    uint32_t valid_tokens = 0;
    uint64_t content_version = 0;
    uint64_t statistics_version = 0;
    bool operator==(const BlockDescriptor &o) const {
        return session == o.session && id == o.id && original_start == o.original_start &&
               valid_tokens == o.valid_tokens && content_version == o.content_version &&
               statistics_version == o.statistics_version;
    }
};
struct BlockCopies {
    BlockDescriptor block;
    uint64_t host_version = 0;  // zero: no host copy; smaller: stale copy
};
struct MemoryStamp {
    bool valid = false;
    SessionIdentity session;
    uint64_t history_revision = 0;
    uint64_t view_version = 0;
    uint64_t frontier = 0;
    uint64_t execution_history = 0;
    bool operator==(const MemoryStamp &o) const {
        return valid == o.valid && session == o.session && history_revision == o.history_revision &&
               view_version == o.view_version && frontier == o.frontier && execution_history == o.execution_history;
    }
};
struct MemorySnapshot {
    MemoryStamp stamp;
    std::vector<BlockCopies> blocks;  // the whole logical catalog, chronological
    std::vector<uint64_t> resident;   // ids of the current device view
};
struct ViewBlock {
    BlockDescriptor block;
    uint64_t compact_start = 0;  // attention address only
};
struct ExecutionView {
    MemoryStamp stamp;
    std::vector<ViewBlock> blocks;
    uint64_t visible_tokens = 0;
};
struct MemoryBudget {
    uint64_t selected_tokens = 0;
    uint64_t reserve_tokens = 0;
    uint64_t device_tokens = 0;
    uint64_t host_payload_bytes = 0;
};
struct WorkingSetPlan {
    MemoryStamp expected;
    MemoryBudget budget;
    ExecutionView next;
    std::vector<uint64_t> mandatory;
    std::vector<BlockDescriptor> evict;
    std::vector<BlockDescriptor> spill;
    std::vector<BlockDescriptor> restore;
    uint64_t device_tokens_required = 0;
    uint64_t host_payload_bytes_required = 0;
};

// memory_contract.hpp:175-195: every operation is required; prepare gives
// the strong guarantee, poll never blocks, abort drains before releasing.
class MemoryTransfer {
public:
    virtual ~MemoryTransfer() = default;
    virtual void start_spill() = 0;
    virtual TransferPoll poll() = 0;
    virtual void start_restore() = 0;
    virtual void publish(const ExecutionView &) = 0;
    virtual AbortResult abort() noexcept = 0;
};
class MemoryBackend {
public:
    virtual ~MemoryBackend() = default;
    virtual MemoryDescriptor descriptor() const = 0;
    virtual MemorySnapshot snapshot() const = 0;
    virtual MemoryStamp stamp() const noexcept = 0;
    virtual std::unique_ptr<MemoryTransfer> prepare(const WorkingSetPlan &) = 0;
    virtual void invalidate() noexcept = 0;
};

// ---- the recall memory object ----------------------------------------------
// An engine tensor as the hooks read it (ggml's order: ne[0] the head dim,
// ne[1] heads, ne[2] tokens; nb[] byte strides).
struct TensorView {
    const void *data = nullptr;
    kvr_format type = KVR_FMT_F32;  // F32, F16 or BF16 for captured K and Q
    int64_t ne[4] = {0, 0, 0, 0};
    size_t nb[4] = {0, 0, 0, 0};
};
// Resolves a registered tensor to its view after the graph has run; false
// when the tensor is not readable on this memory's device.
using TensorResolver = std::function<bool(const void *tensor, TensorView &view)>;

struct RecallMemoryConfig {
    int device = 0;
    uint32_t n_layer = 0;           // model layers
    std::vector<uint32_t> layers;   // attention layers served (empty: all n_layer)
    uint32_t query_heads = 0, kv_heads = 0, head_dim = 0;
    uint32_t block_tokens = 32;     // page size in tokens
    uint32_t max_pages = 0;         // history capacity in pages
    uint32_t budget_pages = 0;      // pages selected (0: every page)
    uint32_t sink_pages = 1, recent_pages = 0;
    GqaScoreAggregation aggregation = GqaScoreAggregation::Mean;
    TieRule tie = TieRule::HigherFirst;  // kvmem_store.cpp:444-446
    int32_t query_begin = -1, query_end = -1;  // Query span of positions; end <= 0: open
    uint32_t max_query_rows = 64;   // Query rows kept per layer
    bool retrieval = true;          // method 1 (retrieval); false: recency only
    std::string model;              // identity for the descriptor
};

class RecallMemory final : public MemoryBackend {
public:
    explicit RecallMemory(const RecallMemoryConfig &config);
    ~RecallMemory() override;
    RecallMemory(const RecallMemory &) = delete;
    RecallMemory &operator=(const RecallMemory &) = delete;

    const RecallMemoryConfig &config() const;
    bool owns_layer(int il) const;
    kvr_context *context() const;

    // ---- capture (attn-qk hook) ----
    // Positions of the next ubatch, in token order (one queue entry per
    // ubatch, consumed by its harvest).
    void note_ubatch(std::vector<int32_t> positions);
    // A graph node to read after the graph runs: 'k' (pre-RoPE K), 'q'
    // (Query) or 'v' (ignored).  Layers this memory does not serve are
    // ignored.
    void register_capture(const void *tensor, int il, char which);
    void capture_on_new_graph();
    // After the ubatch's graph has run: every captured K goes into its
    // layer's page running sums on the device, straight from the tensor, and
    // the Query rows inside the Query span into the layer's device Query
    // rows.  K tensors must hold the ubatch's tokens at consecutive positions.
    void harvest(const TensorResolver &resolve);

    bool query_contains(int32_t pos) const;
    bool query_overlaps(uint32_t n, const int32_t *pos) const;
    bool want_prefill_capture() const;
    bool want_q_capture() const;
    bool want_decode_mean() const;
    bool capture_can_reuse(uint32_t n_tokens, uint32_t n_pos, const int32_t *pos) const;
    uint64_t capture_stamp() const;
    void reset_query();
    void end_prefill_capture();
    void pin_working_set();
    void set_query_span(int32_t begin, int32_t end);

    // ---- recall ----
    uint64_t frontier() const;           // one past the largest position captured
    uint32_t pages() const;              // pages over the frontier
    uint32_t query_rows(uint32_t layer) const;
    // fp16 summaries of every page so far (the finalize of the running sums)
    PageSummaries summaries();
    // page_softmax_scores of the captured Query over the pages, on the device
    // (scores stay in device memory; a host copy is returned)
    std::vector<double> score();
    // query_fixed_blocks + pick_scored_blocks of the last score(): ascending ids
    std::vector<uint32_t> select();
    // Device copies of the last score() and select(): scores [pages],
    // selection [budget], count [1].
    const double *device_scores() const;
    const uint32_t *device_selection() const;
    const uint32_t *device_count() const;

    // Pinned history of one served layer (K and V planes; each plane's slots
    // hold the layer's slot array), where restore reads the pages' bytes.
    void set_history(uint32_t layer, const kvr_plane &k, const kvr_plane &v);

    // ---- MemoryBackend ----
    MemoryDescriptor descriptor() const override;
    MemorySnapshot snapshot() const override;
    MemoryStamp stamp() const noexcept override;
    // The next view's blocks are the selected pages, in ascending id order;
    // the transfer gathers them into slot s = rank of the page in the view.
    // MemoryError: Stale (expected stamp or block versions differ),
    // InvalidSession (after invalidate), BudgetExceeded (more pages than
    // slots), Unsupported (no history for a served layer), InvalidPlan.
    std::unique_ptr<MemoryTransfer> prepare(const WorkingSetPlan &plan) override;
    void invalidate() noexcept override;

    // Published view ids (ascending), for tests and the engine's attention.
    std::vector<uint64_t> resident() const;

private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
    friend class RecallPlanTransfer;
};

}  // namespace kvmem_hip
