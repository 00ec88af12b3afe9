// kvmem_hip.hpp -- C++ host layer of the MI355X recall path, over the C ABI
// of kvrecall.h.  It keeps the shapes of KVMem's own host interfaces for this
// path so an adapter can swap them in:
//   PageSoftmaxHip       for PageSoftmaxCuda  (kvmem/include/kvmem/page_softmax_cuda.hpp:10-32)
//   query_score_frame    (kvmem/include/kvmem/graph_recall.hpp:18-28, graph_recall.cpp:269-293)
//   kvmem_stagein_* / kvmem_d2d_batched / kvmem_meank_*
//                        for src/adapter/llama-kvmem-stagein.h:12-68 (bool + stderr)
//   RecallTransfer       the MemoryTransfer contract (kvmem/include/kvmem/memory_contract.hpp:175-187)
//   SummaryCapture       the capture side of the attn-qk hook (src/adapter/llama-kvmem-hooks.h:74-98)
//   GraphRecallHip::propagate_query_scores  (kvmem/include/kvmem/graph_recall.hpp:119-121)
//   LrfuHistoryHip       for LrfuHistory (kvmem/include/kvmem/lrfu.hpp:43-101)
// Errors follow the reference: std::invalid_argument for geometry and
// operand errors, std::length_error for workspace limits, std::runtime_error
// for device failures.  Reference paths are relative to the KVMem 0.19.0 tree.
#pragma once

#include "kvrecall.h"

#include <cstddef>
#include <cstdint>
#include <functional>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace kvmem_hip {

enum class GqaScoreAggregation { Mean, Max, MaxLogit };
enum class TieRule { LowerFirst, HigherFirst };

// Errors of the memory-backend contract (memory_contract.hpp:14-25): record
// layouts, working-set plans and transfers throw these, with the code a
// caller dispatches on.
enum class MemoryErrorCode {
    InvalidPlan, Unsupported, BudgetExceeded, Stale, Pending, TransferFailed, Disconnected, InvalidSession
};
class MemoryError : public std::runtime_error {
public:
    MemoryError(MemoryErrorCode code, const std::string &message) : std::runtime_error(message), code_(code) {}
    MemoryErrorCode code() const noexcept { return code_; }

private:
    MemoryErrorCode code_;
};

// One accepted logical index: page starts/counts and the score and transport
// masks (graph_recall.hpp:18-24).
struct QueryScoreFrame {
    std::vector<uint64_t> starts;
    std::vector<uint32_t> counts;
    std::vector<uint8_t> score_mask;
    std::vector<uint8_t> transport_mask;
    uint64_t accepted_through = 0;
};

// graph_recall.cpp:269-293: pages of `block_tokens` over `accepted_through`
// tokens; when there are more pages than the budget, sink and recent pages
// leave the softmax and every page is a transport candidate except the
// fixed ones.
QueryScoreFrame query_score_frame(uint64_t accepted_through, uint32_t block_tokens, uint32_t budget_blocks,
                                  uint32_t sink_blocks, uint32_t recent_blocks,
                                  const std::vector<uint32_t> &fixed_blocks);

// Host binary32 Query rows in layer/row/head/channel order; rows beyond
// layer_rows[layer] are absent (graph_recall.hpp:30-38).
struct PageQueryView {
    const float *data = nullptr;
    const uint32_t *layer_rows = nullptr;
    uint32_t layers = 0, rows = 0, query_heads = 0, kv_heads = 0, head_dim = 0;
    const float *const *layer_data = nullptr;  // optional per-layer storage
    float attention_scale = 0;                 // 0 selects 1/sqrt(head_dim)
};

// A borrowed device Query of one layer, strides in bytes
// (native_layer_query.hpp:12-25).
enum class NativeQueryScalar { Float32, Float16, BFloat16 };
struct NativeCurrentLayerQuery {
    const void *data = nullptr;
    size_t bytes = 0;
    uint32_t layer = 0, rows = 0, query_heads = 0, kv_heads = 0, head_dim = 0;
    float attention_scale = 0;
    NativeQueryScalar scalar = NativeQueryScalar::Float32;
    size_t row_stride = 0, head_stride = 0, dimension_stride = 0;
};
// Positive, non-overlapping strides within `bytes` (native_layer_query.hpp:36-58).
void validate_native_layer_query(const NativeCurrentLayerQuery &q);

// Device-resident page summaries, the GPU stand-in for RawKvStore's mean-K:
// per layer fp16 [pages][kv_heads*head_dim] (the recall_fp16 values), as
// written by kvr_summary_build / kvr_summary_finalize.
struct PageSummaries {
    std::vector<const uint16_t *> layers;
    uint32_t pages = 0, page_tokens = 0, kv_heads = 0, head_dim = 0;
};

// Host binary32 page means, the form RawKvStore keeps (mean_k,
// raw_kv_store.cpp:606-625): `read(page, layer, out)` writes the `width`
// (= kv_heads*head_dim) means of the page starting at token
// page*block_tokens, for pages where `has(page)` holds.
struct HostMeanSource {
    uint32_t layers = 0, width = 0, block_tokens = 0;
    std::function<bool(uint32_t page)> has;
    std::function<void(uint32_t page, uint32_t layer, float *out)> read;
    // tokens the page's mean covers in `layer` (mean_k_tokens), for the
    // current-layer coverage check
    std::function<uint32_t(uint32_t page, uint32_t layer)> tokens;
};

// Media (image) token ranges [first, end) in recording order
// (KvMemStore::set_media_ranges, kvmem/include/kvmem/kvmem_store.hpp:504).
using MediaRanges = std::vector<std::pair<uint32_t, uint32_t>>;

// KvMemStore::query_fixed_blocks (kvmem/src/host/kvmem_store.cpp:381-408)
// for a store of `pages` pages of page_tokens tokens holding total_tokens
// tokens: every page when the budget is 0 or covers them all; else sink,
// last media range and mandatory pages with their whole media groups
// (std::runtime_error when they do not fit, std::invalid_argument for a
// page outside the store), then recent pages while they fit.
std::vector<uint32_t> query_fixed_blocks(uint32_t pages, uint32_t budget, uint32_t sink, uint32_t recent,
                                         const MediaRanges &media, uint32_t page_tokens, uint64_t total_tokens,
                                         const std::vector<uint32_t> &mandatory);

// The page-softmax scorer (page_softmax_cuda.hpp:10-32): synchronous on
// return, owned by one adapter, one device.
class PageSoftmaxHip {
public:
    explicit PageSoftmaxHip(int device);
    // Device bytes of a borrowed workspace for up to `max_blocks` pages;
    // score() then never allocates and rejects larger calls before a launch.
    static size_t workspace_bytes(uint32_t max_blocks, uint32_t query_heads, uint32_t kv_heads,
                                  uint32_t head_dim);
    PageSoftmaxHip(int device, void *workspace, size_t bytes, uint32_t max_blocks, uint32_t query_heads,
                   uint32_t kv_heads, uint32_t head_dim);
    ~PageSoftmaxHip();
    PageSoftmaxHip(const PageSoftmaxHip &) = delete;
    PageSoftmaxHip &operator=(const PageSoftmaxHip &) = delete;

    // page_softmax_scores over every layer with rows (graph_recall.cpp:322-394).
    std::vector<double> score(const PageSummaries &, PageQueryView, const QueryScoreFrame &,
                              GqaScoreAggregation = GqaScoreAggregation::Mean);
    // PageSoftmaxCuda::score(const RawKvStore&, ...) (page_softmax_cuda.hpp:24,
    // page_softmax.cu:202-279): the binary32 means of the frame's scored
    // pages are read on the host one layer at a time, moved to the device
    // and rounded there to the fp16 operands (with recall_fp16's checks),
    // then scored as above.  A frame entry may start at any page of the
    // store; one that is not a whole stored page is a stale index extent
    // (std::invalid_argument).  Borrowed workspaces never allocate here
    // either.
    std::vector<double> score(const HostMeanSource &, PageQueryView, const QueryScoreFrame &,
                              GqaScoreAggregation = GqaScoreAggregation::Mean);
    // The same over any store with RawKvStore's reading interface
    // (kvmem/include/kvmem/raw_kv_store.hpp:105-116): config().n_layer,
    // config().n_embd_k, config().block_tokens, has_block(page) and
    // mean_k(page, layer, float *out), so an adapter holding a RawKvStore
    // passes it unchanged.
    template <class Store, class = decltype(std::declval<const Store &>().mean_k(0u, 0u, (float *)nullptr))>
    std::vector<double> score(const Store &keys, PageQueryView v, const QueryScoreFrame &frame,
                              GqaScoreAggregation aggregation = GqaScoreAggregation::Mean) {
        return score(mean_source(keys), v, frame, aggregation);
    }
    // A HostMeanSource reading a RawKvStore-like store (valid while it lives).
    template <class Store> static HostMeanSource mean_source(const Store &keys) {
        HostMeanSource src;
        src.layers = uint32_t(keys.config().n_layer);
        src.width = uint32_t(keys.config().n_embd_k);
        src.block_tokens = uint32_t(keys.config().block_tokens);
        src.has = [&keys](uint32_t page) { return bool(keys.has_block(page)); };
        src.read = [&keys](uint32_t page, uint32_t layer, float *out) { keys.mean_k(page, layer, out); };
        src.tokens = [&keys](uint32_t page, uint32_t layer) { return uint32_t(keys.mean_k_tokens(page, layer)); };
        return src;
    }
    // One layer's native Query on its producer stream, Mean
    // (page_softmax.cu:281-396).  The stream must not be capturing.
    std::vector<double> score_current_layer(const PageSummaries &, NativeCurrentLayerQuery,
                                            const QueryScoreFrame &, void *producer_stream);
    // The same from host binary32 means (page_softmax.cu:281-396): every
    // frame entry must be a whole page whose target-layer mean covers exactly
    // its count of tokens, else std::invalid_argument.
    std::vector<double> score_current_layer(const HostMeanSource &, NativeCurrentLayerQuery,
                                            const QueryScoreFrame &, void *producer_stream);
    template <class Store, class = decltype(std::declval<const Store &>().mean_k(0u, 0u, (float *)nullptr))>
    std::vector<double> score_current_layer(const Store &keys, NativeCurrentLayerQuery q,
                                            const QueryScoreFrame &frame, void *producer_stream) {
        return score_current_layer(mean_source(keys), q, frame, producer_stream);
    }
    // pick_scored_blocks (kvmem_store.cpp:418-451) on the device: mandatory
    // pages first, then by score with the tie rule; ascending ids.
    // Mandatory pages beyond the budget: std::runtime_error, as there.
    std::vector<uint32_t> pick(const std::vector<double> &scores, uint32_t budget,
                               const std::vector<uint32_t> &mandatory = {},
                               TieRule tie = TieRule::LowerFirst, bool signed_scores = false);
    // The same with the store's media ranges (pages of page_tokens tokens):
    // a page in a media range is kept only with its whole group.
    std::vector<uint32_t> pick(const std::vector<double> &scores, uint32_t budget,
                               const std::vector<uint32_t> &mandatory, TieRule tie, bool signed_scores,
                               const MediaRanges &media, uint32_t page_tokens);
    // KvMemStore::pick_topk_blocks (kvmem_store.cpp:377-379): the ungrouped
    // pick (sink, mandatory newest first and recent pages while they fit,
    // then the best scores, higher id first on ties; :578-723), then with
    // media ranges constrain_media (:453-502).  scores are the selection
    // scores, one per page.
    std::vector<uint32_t> pick_topk(const std::vector<double> &scores, uint32_t budget, uint32_t sink,
                                    uint32_t recent, const std::vector<uint32_t> &mandatory = {},
                                    const MediaRanges &media = {}, uint32_t page_tokens = 1,
                                    uint64_t total_tokens = 0);
    size_t device_bytes() const;
    kvr_context *context() const;

private:
    std::vector<uint32_t> fetch_pick(const uint32_t *sel, const uint32_t *cnt, uint32_t k, void *stream,
                                     const char *what);
    struct Impl;
    std::unique_ptr<Impl> impl_;
};

// ---- graph propagation and LRFU ------------------------------------------
// The graph types of graph_recall.hpp:47-52 (positions in tokens).
struct GraphEdge {
    uint64_t target = 0;
    double mass = 0;
};
struct GraphRow {
    uint64_t source = 0, samples = 0;
    std::vector<GraphEdge> edges;
};
struct GraphMessageSpan {
    uint64_t begin = 0, end = 0;
    bool end_known = true;
};
// What propagation reads of a GraphSnapshot (graph_recall.hpp:73-98): the
// sealed rows (any number of chunks), the block size, the accepted and
// completed prefixes and the message spans (null: none).
struct GraphView {
    uint32_t block_tokens = 64;
    uint64_t accepted_through = 0, completed_through = 0;
    std::vector<const std::vector<GraphRow> *> chunks;
    const std::vector<GraphMessageSpan> *messages = nullptr;
};

// span_coefficient (graph_recall.cpp:234-247) of every adjacent page pair
// (i, i+1), i < pages-1: sorted spans, so O((pages + spans) log spans).
std::vector<double> span_coefficients(const std::vector<GraphMessageSpan> &spans, uint32_t block_tokens,
                                      uint32_t pages, double cross);

// Graph propagation and the LRFU candidate on one device; synchronous on
// return like the reference's host functions.
class GraphRecallHip {
public:
    explicit GraphRecallHip(int device);
    ~GraphRecallHip();
    GraphRecallHip(const GraphRecallHip &) = delete;
    GraphRecallHip &operator=(const GraphRecallHip &) = delete;

    // propagate_query_scores (graph_recall.cpp:494-552) for frames whose
    // page i starts at i * block_tokens (what query_score_frame builds), up
    // to KVR_GRAPH_MAX_PAGES pages (std::length_error beyond).
    std::vector<double> propagate_query_scores(const std::vector<double> &raw, const QueryScoreFrame &,
                                               const GraphView &, double alpha = .2,
                                               double cross_message_weight = .25);
    // LrfuHistory::preview's candidate (lrfu.hpp:57-79): lambda * committed +
    // the gated scores.
    std::vector<double> lrfu_candidate(const std::vector<double> &scores, const std::vector<double> &committed,
                                       double lambda, double top_fraction);
    kvr_context *context() const;

private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
};

// LrfuHistory (lrfu.hpp:43-101): rounds, previews derived from committed
// history only, one commit per round, checkpoints sharing committed scores.
struct LrfuState {
    std::shared_ptr<const std::vector<double>> scores = std::make_shared<const std::vector<double>>();
    uint64_t round = 0;
    bool committed = false;
};
class LrfuHistoryHip {
public:
    explicit LrfuHistoryHip(GraphRecallHip &device, double lambda = 0.5, double top_fraction = 0.9);
    void begin_round();
    void preview(const std::vector<double> &scores);
    bool commit() noexcept;
    double score(size_t block) const noexcept;
    LrfuState checkpoint() const { return state_; }
    void restore(const LrfuState &state);
    void discard_candidate() noexcept { candidate_.reset(); }

private:
    GraphRecallHip *device_;
    double lambda_, fraction_;
    LrfuState state_;
    std::shared_ptr<const std::vector<double>> candidate_;
};

// ---- native payload records (memory_contract.hpp:39-68) -------------------
// One record per page holds every layer's planes at fixed offsets.  The
// types mirror the reference's; validate() enforces the rules of
// PayloadLayout::validate (kvmem/src/host/memory_contract.cpp:51-101) and
// throws MemoryError(InvalidPlan) with the reference's messages.
enum class PayloadPlaneKind { Key, Value, KeyScale, ValueScale, PackedKeyValue };
struct PayloadPlane {
    uint32_t layer = 0;
    PayloadPlaneKind kind = PayloadPlaneKind::Key;
    uint64_t offset = 0, bytes = 0, alignment = 1;
    uint64_t token_stride = 0;  // 0: opaque page encoding
    uint32_t rank = 0, head_begin = 0, head_count = 0;
};
struct PayloadLayout {
    std::string format;
    uint32_t version = 0, block_tokens = 0;
    uint64_t record_bytes = 0, alignment = 1;
    std::vector<PayloadPlane> planes;
    void validate() const;
};
// The stage-in plane of one layer's Key or Value rows (rank `rank`) in a
// pinned archive of records (page p's record at archive + p * record_bytes),
// for kvr_stage_in with page_tokens = layout.block_tokens.  The plane must
// address contiguous token rows of `format` x `width` (token_stride = the
// row size); std::invalid_argument otherwise.
kvr_plane record_plane(const PayloadLayout &layout, uint32_t layer, PayloadPlaneKind kind, const void *archive,
                       kvr_format format, uint32_t width, uint64_t tokens, kvr_gather_mode mode, void *slots,
                       uint32_t rank = 0);

// ---- stage-in entry points (llama-kvmem-stagein.h) ------------------------
// bool results with the failure on stderr, one state per execution domain
// (thread).  The product path sends packed K and V record bytes through
// enqueue_v: they are copied into a pinned 32 MiB slab (the caller's buffer
// is reusable on return) and flush moves them into their cache rows with one
// device launch that reads the pinned slab directly.
struct kvmem_gpu_state;
kvmem_gpu_state *kvmem_gpu_state_create();  // also made current on this thread
void kvmem_gpu_state_free(kvmem_gpu_state *state);
void kvmem_gpu_state_make_current(kvmem_gpu_state *state);

bool kvmem_stagein_gpu_ready(size_t n_f32, size_t n_packed = 0);
void kvmem_stagein_gpu_free();
bool kvmem_stagein_h2d_bytes(void *gpu_dst, const void *host, size_t n);
void kvmem_stagein_sync();
bool kvmem_stagein_sync_checked();
bool kvmem_stagein_enqueue_v(const void *packed, size_t nbytes, uint8_t *dst, int64_t *set_us);
// A packed raw K record (llama-kvmem-stagein.h:37-42): nt token rows of
// n_embd values in q8_0 or q4_0 (`ty`), rotated (NeoX, n_rot_rope dims of
// each n_embd_head head, positions pos0 + t, theta of n_theta = n_rot_rope/2
// host values), Walsh-Hadamard over runs of nrot (0: none), requantized into
// dst on flush.  The record is copied into the slab; the caller's buffer is
// reusable on return.
bool kvmem_stagein_enqueue_k(kvr_format ty, const void *packed, size_t nbytes, uint8_t *dst, int64_t nt,
                             int64_t n_embd, int nrot, int n_head, int n_embd_head, int n_rot_rope, int32_t pos0,
                             const float *theta, int n_theta, int64_t *copy_us, int64_t *rope_us,
                             int64_t *hadamard_us, int64_t *set_us);
bool kvmem_stagein_flush(int64_t *copy_us, int64_t *rope_us, int64_t *hadamard_us, int64_t *set_us);
bool kvmem_d2d_batched(const void *const *src, void *const *dst, const size_t *nbytes, int n);

// Stage-out (llama-kvmem-stagein.h:44-50): device records packed back to
// back into one of the two pinned slabs.  submit launches one batched copy
// that writes them over the host link (no device staging slab) and returns
// the slot; wait fences it; slot_base is the slot's host memory.  Not mixed
// with pending stage-in records (either side refuses while the other has
// records queued).
bool kvmem_stageout_enqueue(const void *gpu_src, size_t nbytes);
size_t kvmem_stageout_used();
int kvmem_stageout_submit(int64_t *copy_us);
bool kvmem_stageout_wait(int slot, int64_t *copy_us);
const uint8_t *kvmem_stageout_slot_base(int slot);
void kvmem_stageout_clear();

// Decode running mean-K (stagein.cu:270-320, 1041-1114): one binary32 sum of
// n_embd channels per layer on the device, added in token order and zeroed
// by kvmem_meank_zero.  `ty` is the K element type (F32, F16 or BF16; the
// reference passes a ggml_type); channel c = head*ne0 + dim of token t is at
// gpu_k + (tok0+t)*nb2 + head*nb1 + dim*nb0.
bool kvmem_meank_ready(uint32_t n_layer, uint32_t n_embd);
void kvmem_meank_free();
void kvmem_meank_zero(uint32_t il);
bool kvmem_meank_add(uint32_t il, kvr_format ty, const void *gpu_k, uint32_t tok0, uint32_t n_keep,
                     uint32_t n_embd, int64_t ne0, size_t nb0, size_t nb1, size_t nb2);
bool kvmem_meank_d2h(uint32_t il, float *host, uint32_t n_embd);

// ---- MemoryTransfer for recall (memory_contract.hpp:175-187) --------------
enum class TransferStatus { Pending, Complete, Failed };
struct TransferPoll {
    TransferStatus status = TransferStatus::Pending;
    std::string error;
};
enum class AbortResult { PreviousViewPreserved, SessionInvalidated };

// Restores one layer's selected pages into the slot arrays.  The pages' home
// is the pinned history, so there is nothing to spill: start_spill only
// marks the spill phase done.  start_restore enqueues kvr_stage_in on the
// transfer's stream (after `ready`, an event of the producer of the
// selection, when given); poll never blocks; publish requires a completed
// restore; abort drains before returning.
class RecallTransfer {
public:
    RecallTransfer(kvr_context *ctx, std::vector<kvr_plane> planes, uint32_t lanes, uint32_t page_tokens,
                   const uint32_t *selected, const uint32_t *count, uint32_t k,
                   kvr_copy_engine engine = KVR_ENGINE_KERNEL, void *stream = nullptr, void *ready = nullptr);
    ~RecallTransfer();
    RecallTransfer(const RecallTransfer &) = delete;
    RecallTransfer &operator=(const RecallTransfer &) = delete;
    void start_spill();
    TransferPoll poll();
    void start_restore();
    void publish();
    AbortResult abort() noexcept;
    bool published() const { return phase_ == Phase::Published; }

private:
    enum class Phase { Prepared, Spilled, Restoring, Ready, Published, Failed, Aborted };
    kvr_context *ctx_;
    std::vector<kvr_plane> planes_;
    uint32_t lanes_, page_tokens_, k_;
    const uint32_t *selected_, *count_;
    kvr_copy_engine engine_;
    void *stream_, *ready_;
    void *done_ = nullptr;  // hipEvent_t
    Phase phase_ = Phase::Prepared;
    std::string error_;
};

// Capture side of the attn-qk hook: captured K rows of each layer go into
// device running sums (kvr_summary_accumulate), and finalized pages become
// the fp16 summaries a PageSummaries points at (kvr_summary_finalize).
// The context must outlive the capture (and a RecallTransfer).
class SummaryCapture {
public:
    SummaryCapture(kvr_context *ctx, uint32_t layers, uint32_t max_pages, uint32_t page_tokens,
                   uint32_t kv_heads, uint32_t head_dim);
    ~SummaryCapture();
    SummaryCapture(const SummaryCapture &) = delete;
    SummaryCapture &operator=(const SummaryCapture &) = delete;
    // Rows [pos0, pos0+n) of layer `layer`; element (t, h, d) at
    // k + t*token_stride + h*head_stride + d*dim_stride (bytes).
    void capture(uint32_t layer, const void *k, kvr_format scalar, uint64_t pos0, uint32_t n,
                 size_t token_stride, size_t head_stride, size_t dim_stride, void *stream = nullptr);
    // fp16 summaries of the first `pages` pages of every layer.
    PageSummaries finalize(uint32_t pages, void *stream = nullptr);
    const float *means(uint32_t layer) const;

private:
    kvr_context *ctx_;
    uint32_t layers_, max_pages_, page_tokens_, kv_heads_, head_dim_;
    float *sums_ = nullptr, *means_ = nullptr;
    uint32_t *counts_ = nullptr;
    uint16_t *summaries_ = nullptr;
};

// ---- sampled attention (src/adapter/llama-kvmem-attention-cuda.h:9-16) ----
// An engine tensor as the sampler reads it: element type, element counts
// ne[0..2] and byte strides nb[1..2] (ggml's order: ne[0] the head dim,
// ne[1] rows or tokens, ne[2] heads; a mask is [tokens][rows]).
struct AttentionTensor {
    const void *data = nullptr;
    kvr_format type = KVR_FMT_F32;
    int64_t ne[3] = {0, 0, 0};
    size_t nb[3] = {0, 0, 0};
};

// llama_kvmem_attention_cuda: sampled attention page masses of one layer
// from its represented Q, native K and mask, without a token attention
// matrix.  Q and K on one device; a mask elsewhere (host memory) has its
// sampled rows staged.  Synchronous on return.
class AttentionSamplerHip {
public:
    AttentionSamplerHip();
    ~AttentionSamplerHip();
    AttentionSamplerHip(const AttentionSamplerHip &) = delete;
    AttentionSamplerHip &operator=(const AttentionSamplerHip &) = delete;
    // false when the sampler does not serve these operands (types, head
    // dim, Q and K not on one device), as the reference's score() declines;
    // else output[i][page] for sampled row rows[i].  HIP errors throw
    // std::runtime_error; a call on another device than the first throws.
    bool score(const AttentionTensor &q, const AttentionTensor &k, const AttentionTensor &mask, float scale,
               float softcap, uint32_t block, const std::vector<uint32_t> &rows,
               std::vector<std::vector<float>> &output);

private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
};

}  // namespace kvmem_hip
