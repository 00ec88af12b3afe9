// ref_driver.cpp -- extern "C" entry points over the KVMem reference host
// library, compiled from the reference's own sources into oracle/_ref.
//
// TEST INFRASTRUCTURE ONLY.  This file is this project's own glue code; it
// includes the reference's public headers at build time (the include path is
// given by oracle/Makefile) and is never part of the product library.
// It lets tests, the fixture generator and the CPU-baseline leg of the
// benchmark call the reference's real functions:
//   RawKvStore::write_layer_tokens_f16 / write_layer_mean_k / mean_k
//                                     (kvmem/src/host/raw_kv_store.cpp)
//   query_score_frame, recall_fp16, page_softmax_scores
//                                     (kvmem/src/host/graph_recall.cpp)
//   KvMemStore::pick_scored_blocks, query_fixed_blocks, pick_topk_blocks
//                                     (kvmem/src/host/kvmem_store.cpp)
//   layerwise_mean_key_scores         (kvmem/src/host/layerwise_scoring.cpp)
//   prepare_graph_accept, propagate_query_scores
//                                     (kvmem/src/host/graph_recall.cpp)
//   LrfuHistory::preview / score, and its round/commit/restore rules
//                                     (kvmem/include/kvmem/lrfu.hpp)
//   PayloadLayout::validate           (kvmem/src/host/memory_contract.cpp)
//   validate_native_layer_query       (kvmem/include/kvmem/native_layer_query.hpp)
// Exceptions never cross this boundary: each entry returns 0 on success and a
// nonzero code on a thrown exception, with the message in ref_last_error().
#include "kvmem/graph_recall.hpp"
#include "kvmem/kvmem_store.hpp"
#include "kvmem/layerwise_scoring.hpp"
#include "kvmem/layerwise_selection.hpp"
#include "kvmem/lrfu.hpp"
#include "kvmem/memory_contract.hpp"
#include "kvmem/native_layer_query.hpp"
#include "kvmem/raw_kv_store.hpp"

#include <cstring>
#include <exception>
#include <memory>
#include <numeric>
#include <string>
#include <vector>

namespace {
thread_local std::string g_error;

template <class F> int guarded(F&& body) {
    try {
        body();
        return 0;
    } catch (const std::exception& e) {
        g_error = e.what();
        return 1;
    } catch (...) {
        g_error = "unknown exception";
        return 1;
    }
}

kvmem::GqaScoreAggregation aggregation(int agg) {
    return agg == 1 ? kvmem::GqaScoreAggregation::Max : kvmem::GqaScoreAggregation::Mean;
}

// A store whose layer l holds token-major fp16 keys [tokens][width] in blocks
// of page_tokens, written the way the capture path writes fp16 K.
std::unique_ptr<kvmem::RawKvStore> store_from_f16(const uint16_t* keys, uint32_t layers,
                                                  uint64_t tokens, uint32_t width,
                                                  uint32_t page_tokens) {
    kvmem::RawKvStoreConfig cfg;
    cfg.n_layer = layers;
    cfg.n_embd_k = width;
    cfg.n_embd_v = 0;
    cfg.block_tokens = page_tokens;
    auto store = std::make_unique<kvmem::RawKvStore>(cfg);
    for (uint32_t l = 0; l < layers; ++l)
        store->write_layer_tokens_f16(0, uint32_t(tokens), l, keys + size_t(l) * tokens * width,
                                      nullptr);
    return store;
}

// A store whose layer l holds binary32 key rows, fed through the prefill
// mean-K path (write_layer_mean_k: sequential binary32 adds).
std::unique_ptr<kvmem::RawKvStore> store_from_f32(const float* keys, uint32_t layers,
                                                  uint64_t tokens, uint32_t width,
                                                  uint32_t page_tokens) {
    kvmem::RawKvStoreConfig cfg;
    cfg.n_layer = layers;
    cfg.n_embd_k = width;
    cfg.n_embd_v = 0;
    cfg.block_tokens = page_tokens;
    auto store = std::make_unique<kvmem::RawKvStore>(cfg);
    for (uint32_t l = 0; l < layers; ++l)
        store->write_layer_mean_k(0, uint32_t(tokens), l, keys + size_t(l) * tokens * width);
    return store;
}

void scores_from_store(const kvmem::RawKvStore& store, uint64_t tokens, uint32_t page_tokens,
                       const float* query, const uint32_t* layer_rows, uint32_t layers,
                       uint32_t rows, uint32_t query_heads, uint32_t kv_heads,
                       uint32_t head_dim, float scale, int agg, const uint8_t* score_mask,
                       double* out) {
    const uint32_t pages = uint32_t((tokens + page_tokens - 1) / page_tokens);
    // A budget of every page disables the sink/recent bands, so every page is
    // scored unless the caller masks it explicitly.
    auto frame = kvmem::query_score_frame(tokens, page_tokens, pages, 0, 0, {});
    if (score_mask)
        for (uint32_t j = 0; j < pages; ++j) frame.score_mask[j] = score_mask[j];
    kvmem::PageQueryView view;
    view.data = query;
    view.layer_rows = layer_rows;
    view.layers = layers;
    view.rows = rows;
    view.query_heads = query_heads;
    view.kv_heads = kv_heads;
    view.head_dim = head_dim;
    view.attention_scale = scale;
    const auto result = kvmem::page_softmax_scores(store, view, frame, aggregation(agg));
    std::memcpy(out, result.data(), sizeof(double) * result.size());
}

void copy_means(const kvmem::RawKvStore& store, uint32_t layers, uint32_t pages,
                uint32_t width, float* means) {
    if (!means) return;
    for (uint32_t l = 0; l < layers; ++l)
        for (uint32_t p = 0; p < pages; ++p)
            store.mean_k(p, l, means + (size_t(l) * pages + p) * width);
}
}  // namespace

extern "C" {

const char* ref_last_error(void) { return g_error.c_str(); }

int ref_recall_fp16(float value, float* out) {
    return guarded([&] { *out = kvmem::recall_fp16(value); });
}

int ref_query_score_frame(uint64_t accepted, uint32_t block_tokens, uint32_t budget,
                          uint32_t sink, uint32_t recent, const uint32_t* fixed,
                          uint32_t n_fixed, uint64_t* starts, uint32_t* counts,
                          uint8_t* score_mask, uint8_t* transport_mask) {
    return guarded([&] {
        std::vector<uint32_t> pins(fixed, fixed + n_fixed);
        const auto f = kvmem::query_score_frame(accepted, block_tokens, budget, sink, recent, pins);
        for (size_t i = 0; i < f.starts.size(); ++i) {
            starts[i] = f.starts[i];
            counts[i] = f.counts[i];
            score_mask[i] = f.score_mask[i];
            transport_mask[i] = f.transport_mask[i];
        }
    });
}

// Summaries (mean_k) and page-softmax scores from fp16 key history.
// keys: [layers][tokens][kv_heads*head_dim] fp16; query: [layers][rows][Hq][D].
int ref_scores_f16_keys(const uint16_t* keys, uint32_t layers, uint64_t tokens,
                        uint32_t kv_heads, uint32_t head_dim, uint32_t page_tokens,
                        const float* query, const uint32_t* layer_rows, uint32_t rows,
                        uint32_t query_heads, float scale, int agg,
                        const uint8_t* score_mask, float* means, double* scores) {
    return guarded([&] {
        const uint32_t width = kv_heads * head_dim;
        auto store = store_from_f16(keys, layers, tokens, width, page_tokens);
        copy_means(*store, layers, uint32_t((tokens + page_tokens - 1) / page_tokens), width,
                   means);
        if (scores)
            scores_from_store(*store, tokens, page_tokens, query, layer_rows, layers, rows,
                              query_heads, kv_heads, head_dim, scale, agg, score_mask, scores);
    });
}

// The same from binary32 key rows through the prefill mean-K path.
int ref_scores_f32_keys(const float* keys, uint32_t layers, uint64_t tokens,
                        uint32_t kv_heads, uint32_t head_dim, uint32_t page_tokens,
                        const float* query, const uint32_t* layer_rows, uint32_t rows,
                        uint32_t query_heads, float scale, int agg,
                        const uint8_t* score_mask, float* means, double* scores) {
    return guarded([&] {
        const uint32_t width = kv_heads * head_dim;
        auto store = store_from_f32(keys, layers, tokens, width, page_tokens);
        copy_means(*store, layers, uint32_t((tokens + page_tokens - 1) / page_tokens), width,
                   means);
        if (scores)
            scores_from_store(*store, tokens, page_tokens, query, layer_rows, layers, rows,
                              query_heads, kv_heads, head_dim, scale, agg, score_mask, scores);
    });
}

// Page-softmax scores from per-page sums that each cover `page_tokens`
// tokens (write_layer_mean_sum), i.e. mean = sum * (1/page_tokens).
int ref_scores_from_sums(const float* sums, uint32_t layers, uint32_t pages,
                         uint32_t kv_heads, uint32_t head_dim, uint32_t page_tokens,
                         const float* query, const uint32_t* layer_rows, uint32_t rows,
                         uint32_t query_heads, float scale, int agg,
                         const uint8_t* score_mask, double* scores) {
    return guarded([&] {
        const uint32_t width = kv_heads * head_dim;
        kvmem::RawKvStoreConfig cfg;
        cfg.n_layer = layers;
        cfg.n_embd_k = width;
        cfg.block_tokens = page_tokens;
        kvmem::RawKvStore store(cfg);
        for (uint32_t l = 0; l < layers; ++l)
            for (uint32_t p = 0; p < pages; ++p)
                store.write_layer_mean_sum(p * page_tokens, page_tokens, l,
                                           sums + (size_t(l) * pages + p) * width);
        scores_from_store(store, uint64_t(pages) * page_tokens, page_tokens, query, layer_rows,
                          layers, rows, query_heads, kv_heads, head_dim, scale, agg,
                          score_mask, scores);
    });
}

// Single-layer current-Q Mean scores (layerwise_mean_key_scores).
int ref_layerwise_scores_f16_keys(const uint16_t* keys, uint32_t layers, uint32_t layer,
                                  uint64_t tokens, uint32_t kv_heads, uint32_t head_dim,
                                  uint32_t page_tokens, const float* query, uint32_t rows,
                                  uint32_t query_heads, float scale, double* scores) {
    return guarded([&] {
        auto store = store_from_f16(keys, layers, tokens, kv_heads * head_dim, page_tokens);
        const uint32_t pages = uint32_t((tokens + page_tokens - 1) / page_tokens);
        auto frame = kvmem::query_score_frame(tokens, page_tokens, pages, 0, 0, {});
        kvmem::CurrentLayerQuery q;
        q.data = query;
        q.layer = layer;
        q.rows = rows;
        q.query_heads = query_heads;
        q.kv_heads = kv_heads;
        q.head_dim = head_dim;
        q.attention_scale = scale;
        const auto result = kvmem::layerwise_mean_key_scores(*store, q, frame);
        std::memcpy(scores, result.data(), sizeof(double) * result.size());
    });
}

// Half-page current-Q Mean scores: layerwise_tile_scores over transport
// pages of page_tokens with Mean-K records every mean_tokens tokens of the
// given fp16 keys, then (keep_halves) layerwise_max_page_scores.  score_mask
// is per transport page (NULL: every page).  out: one score per page.
int ref_layerwise_tile_scores_f16_keys(const uint16_t* keys, uint32_t layers, uint32_t layer, uint64_t tokens,
                                       uint32_t kv_heads, uint32_t head_dim, uint32_t mean_tokens,
                                       uint32_t page_tokens, const float* query, uint32_t rows,
                                       uint32_t query_heads, float scale, int keep_halves,
                                       const uint8_t* score_mask, double* out) {
    return guarded([&] {
        auto store = store_from_f16(keys, layers, tokens, kv_heads * head_dim, mean_tokens);
        const uint32_t pages = uint32_t((tokens + page_tokens - 1) / page_tokens);
        auto frame = kvmem::query_score_frame(tokens, page_tokens, pages, 0, 0, {});
        if (score_mask)
            for (uint32_t j = 0; j < pages; ++j) frame.score_mask[j] = score_mask[j];
        kvmem::CurrentLayerQuery q;
        q.data = query;
        q.layer = layer;
        q.rows = rows;
        q.query_heads = query_heads;
        q.kv_heads = kv_heads;
        q.head_dim = head_dim;
        q.attention_scale = scale;
        auto result = kvmem::layerwise_tile_scores(frame, page_tokens, mean_tokens, keep_halves != 0,
                                                   [&](const kvmem::QueryScoreFrame& f) {
                                                       return kvmem::layerwise_mean_key_scores(*store, q, f);
                                                   });
        if (keep_halves) result = kvmem::layerwise_max_page_scores(result);
        std::memcpy(out, result.data(), sizeof(double) * result.size());
    });
}

// KvMemStore::pick_scored_blocks over every page as a candidate.  The
// reference's only tie rule is higher page id first.
int ref_pick_scored_blocks(const double* scores, uint32_t n, const uint32_t* mandatory,
                           uint32_t n_mandatory, uint32_t budget, int signed_scores,
                           uint32_t* out, uint32_t* n_out) {
    return guarded([&] {
        kvmem::KvMemStoreConfig cfg;
        cfg.block_tokens = 1;
        cfg.select_budget = budget;
        cfg.sink_blocks = 0;
        cfg.recent_blocks = 0;
        kvmem::KvMemStore store(cfg);
        store.register_append(n);
        std::vector<uint32_t> candidates(n);
        std::iota(candidates.begin(), candidates.end(), 0u);
        const std::vector<double> values(scores, scores + n);
        const std::vector<uint32_t> pins(mandatory, mandatory + n_mandatory);
        const auto picked =
            store.pick_scored_blocks(candidates, values, pins, budget, signed_scores != 0);
        std::memcpy(out, picked.data(), sizeof(uint32_t) * picked.size());
        *n_out = uint32_t(picked.size());
    });
}

}  // extern "C"

namespace {
// A KvMemStore of ceil(total_tokens / page_tokens) pages, a selection budget
// of `budget` pages, the given sink/recent bands and media token ranges
// (ranges[2i], ranges[2i+1]).
std::unique_ptr<kvmem::KvMemStore> policy_store(uint64_t total_tokens, uint32_t page_tokens, uint32_t budget,
                                                uint32_t sink, uint32_t recent, const uint32_t* ranges,
                                                uint32_t n_ranges) {
    kvmem::KvMemStoreConfig cfg;
    cfg.block_tokens = page_tokens;
    cfg.select_budget = budget * page_tokens;
    cfg.sink_blocks = sink;
    cfg.recent_blocks = recent;
    auto store = std::make_unique<kvmem::KvMemStore>(cfg);
    store->register_append(uint32_t(total_tokens));
    std::vector<std::pair<uint32_t, uint32_t>> media;
    for (uint32_t r = 0; r < n_ranges; ++r) media.emplace_back(ranges[2 * r], ranges[2 * r + 1]);
    store->set_media_ranges(std::move(media));
    return store;
}

void copy_out(const std::vector<uint32_t>& v, uint32_t* out, uint32_t* n_out) {
    std::memcpy(out, v.data(), sizeof(uint32_t) * v.size());
    *n_out = uint32_t(v.size());
}
}  // namespace

extern "C" {

// KvMemStore::query_fixed_blocks of such a store.
int ref_query_fixed_blocks(uint64_t total_tokens, uint32_t page_tokens, uint32_t budget, uint32_t sink,
                           uint32_t recent, const uint32_t* ranges, uint32_t n_ranges, const uint32_t* mandatory,
                           uint32_t n_mandatory, uint32_t* out, uint32_t* n_out) {
    return guarded([&] {
        auto store = policy_store(total_tokens, page_tokens, budget, sink, recent, ranges, n_ranges);
        copy_out(store->query_fixed_blocks(std::vector<uint32_t>(mandatory, mandatory + n_mandatory)), out, n_out);
    });
}

// KvMemStore::pick_scored_blocks over every page of such a store (media
// groups apply).
int ref_pick_scored_grouped(const double* scores, uint64_t total_tokens, uint32_t page_tokens,
                            const uint32_t* ranges, uint32_t n_ranges, const uint32_t* mandatory,
                            uint32_t n_mandatory, uint32_t budget, int signed_scores, uint32_t* out,
                            uint32_t* n_out) {
    return guarded([&] {
        auto store = policy_store(total_tokens, page_tokens, budget, 0, 0, ranges, n_ranges);
        const uint32_t n = store->block_count();
        std::vector<uint32_t> candidates(n);
        std::iota(candidates.begin(), candidates.end(), 0u);
        copy_out(store->pick_scored_blocks(candidates, std::vector<double>(scores, scores + n),
                                           std::vector<uint32_t>(mandatory, mandatory + n_mandatory), budget,
                                           signed_scores != 0),
                 out, n_out);
    });
}

// KvMemStore::pick_topk_blocks(mandatory) of such a store whose pages carry
// the given selection scores (pick_topk_ungrouped, then constrain_media when
// media ranges exist).
int ref_pick_topk_blocks(const double* scores, uint64_t total_tokens, uint32_t page_tokens, uint32_t budget,
                         uint32_t sink, uint32_t recent, const uint32_t* ranges, uint32_t n_ranges,
                         const uint32_t* mandatory, uint32_t n_mandatory, uint32_t* out, uint32_t* n_out) {
    return guarded([&] {
        auto store = policy_store(total_tokens, page_tokens, budget, sink, recent, ranges, n_ranges);
        store->set_attn_scores(std::vector<double>(scores, scores + store->block_count()));
        copy_out(store->pick_topk_blocks(std::vector<uint32_t>(mandatory, mandatory + n_mandatory)), out, n_out);
    });
}

// propagate_query_scores over a frame of n pages of block_tokens (page i
// starts at i*block_tokens, transport mask as given, NULL: every page) and a
// snapshot holding the given page-indexed rows as sealed rows of one sample.
// n_spans == UINT32_MAX: no message spans (span_coefficient returns 1).
int ref_propagate_query_scores(const double* raw, uint32_t n, const uint8_t* mask,
                               uint32_t block_tokens, uint32_t n_rows, const uint32_t* row_source,
                               const uint32_t* row_begin, const uint32_t* edge_target,
                               const double* edge_mass, uint32_t n_spans, const uint64_t* span_begin,
                               const uint64_t* span_end, const uint8_t* span_known, double alpha,
                               double cross, double* out) {
    return guarded([&] {
        auto frame = kvmem::query_score_frame(uint64_t(n) * block_tokens, block_tokens, 1, 0, 0, {});
        for (uint32_t i = 0; i < n; ++i) frame.transport_mask[i] = mask ? mask[i] : 1;
        kvmem::GraphSnapshot graph;
        graph.block_tokens = block_tokens;
        graph.accepted_through = graph.completed_through = uint64_t(n) * block_tokens;
        std::vector<kvmem::GraphRow> rows(n_rows);
        for (uint32_t r = 0; r < n_rows; ++r) {
            rows[r].source = uint64_t(row_source[r]) * block_tokens;
            rows[r].samples = 1;
            for (uint32_t e = row_begin[r]; e < row_begin[r + 1]; ++e)
                rows[r].edges.push_back({uint64_t(edge_target[e]) * block_tokens, edge_mass[e]});
        }
        if (n_rows) graph.chunks.push_back(std::make_shared<const std::vector<kvmem::GraphRow>>(std::move(rows)));
        if (n_spans != UINT32_MAX) {
            std::vector<kvmem::GraphMessageSpan> spans(n_spans);
            for (uint32_t s = 0; s < n_spans; ++s) spans[s] = {span_begin[s], span_end[s], span_known[s] != 0};
            graph.set_messages(spans);
        }
        const std::vector<double> in(raw, raw + n);
        const auto result = kvmem::propagate_query_scores(in, frame, graph, alpha, cross);
        std::memcpy(out, result.data(), sizeof(double) * n);
    });
}

// One prepare_graph_accept over tokens [0, end) with the given sampled rows
// (row s: source position sample_pos[s], mass over token-position targets
// sample_target[sample_begin[s] .. sample_begin[s+1])), then the snapshot's
// rows that propagation reads (samples > 0, source block complete),
// flattened by page.  Capacities: max_rows rows, max_edges edges.
int ref_graph_accept(uint32_t block_tokens, uint64_t end, uint32_t n_samples, const uint64_t* sample_pos,
                     const uint32_t* sample_begin, const uint64_t* sample_target, const double* sample_mass,
                     uint32_t topk, uint32_t max_rows, uint32_t max_edges, uint32_t* n_rows,
                     uint32_t* row_source, uint32_t* row_begin, uint32_t* edge_target, double* edge_mass) {
    return guarded([&] {
        kvmem::GraphSnapshot graph;
        graph.block_tokens = block_tokens;
        std::vector<kvmem::AcceptedAttentionRow> rows(n_samples);
        for (uint32_t s = 0; s < n_samples; ++s) {
            rows[s].source_position = sample_pos[s];
            for (uint32_t e = sample_begin[s]; e < sample_begin[s + 1]; ++e)
                rows[s].mass.push_back({sample_target[e], sample_mass[e]});
        }
        graph = kvmem::prepare_graph_accept(graph, 0, end, rows, size_t(1) << 30, topk);
        uint32_t r = 0, e = 0;
        row_begin[0] = 0;
        for (const auto& chunk : graph.chunks)
            for (const auto& row : *chunk) {
                if (!row.samples || row.source + block_tokens > graph.completed_through) continue;
                if (r == max_rows || e + row.edges.size() > max_edges) throw std::length_error("graph capacity");
                row_source[r] = uint32_t(row.source / block_tokens);
                for (const auto& edge : row.edges) {
                    edge_target[e] = uint32_t(edge.target / block_tokens);
                    edge_mass[e++] = edge.mass;
                }
                row_begin[++r] = e;
            }
        *n_rows = r;
    });
}

// LrfuHistory(lambda, fraction) with committed history (n_history entries,
// none: a fresh history), one round, one preview; out[i] = score(i).
int ref_lrfu_preview(const double* history, uint32_t n_history, const double* scores, uint32_t n,
                     double lambda, double fraction, double* out) {
    return guarded([&] {
        kvmem::LrfuHistory h(lambda, fraction);
        if (n_history) {
            kvmem::LrfuState state;
            state.scores = std::make_shared<const std::vector<double>>(history, history + n_history);
            state.round = 1;
            state.committed = true;
            h.restore(state);
        }
        h.begin_round();
        h.preview(std::vector<double>(scores, scores + n));
        for (uint32_t i = 0; i < n; ++i) out[i] = h.score(i);
    });
}

// PayloadLayout::validate (kvmem/src/host/memory_contract.cpp:51-101) of a
// layout whose planes are n rows of 9 values: layer, kind, offset, bytes,
// alignment, token_stride, rank, head_begin, head_count.  Returns 0 when
// valid, 1 with the message in ref_last_error() when it throws.
int ref_payload_validate(const char* format, uint32_t version, uint32_t block_tokens, uint64_t record_bytes,
                         uint64_t alignment, const uint64_t* planes, uint32_t n) {
    return guarded([&] {
        kvmem::PayloadLayout l;
        l.format = format;
        l.version = version;
        l.block_tokens = block_tokens;
        l.record_bytes = record_bytes;
        l.alignment = alignment;
        for (uint32_t i = 0; i < n; ++i) {
            const uint64_t* r = planes + 9 * size_t(i);
            kvmem::PayloadPlane p;
            p.layer = uint32_t(r[0]);
            p.kind = kvmem::PayloadPlaneKind(r[1]);
            p.offset = r[2];
            p.bytes = r[3];
            p.alignment = r[4];
            p.token_stride = r[5];
            p.rank = uint32_t(r[6]);
            p.head_begin = uint32_t(r[7]);
            p.head_count = uint32_t(r[8]);
            l.planes.push_back(p);
        }
        l.validate();
    });
}

// validate_native_layer_query (kvmem/include/kvmem/native_layer_query.hpp:36-53)
// of a Query at address `data` (never dereferenced); scalar 0 f32, 1 f16,
// 2 bf16.
int ref_native_query_validate(uintptr_t data, size_t bytes, uint32_t rows, uint32_t query_heads,
                              uint32_t kv_heads, uint32_t head_dim, float scale, int scalar, size_t row_stride,
                              size_t head_stride, size_t dimension_stride) {
    return guarded([&] {
        kvmem::NativeCurrentLayerQuery q;
        q.data = reinterpret_cast<const void*>(data);
        q.bytes = bytes;
        q.rows = rows;
        q.query_heads = query_heads;
        q.kv_heads = kv_heads;
        q.head_dim = head_dim;
        q.attention_scale = scale;
        q.scalar = kvmem::NativeQueryScalar(scalar);
        q.row_stride = row_stride;
        q.head_stride = head_stride;
        q.dimension_stride = dimension_stride;
        kvmem::validate_native_layer_query(q);
    });
}

// LrfuHistory driven by a script of operations, to compare its state machine
// with another implementation's.  ops[i]: 0 begin_round, 1 preview of the
// next `lens[i]` values of `values`, 2 commit, 3 checkpoint (kept), 4 restore
// of the kept checkpoint.  After each op, results[i] = 0 on success, 1 when
// it threw (message dropped), 2 when commit returned false; scores[i * probe
// + b] = score(b) for b < probe.
int ref_lrfu_script(double lambda, double fraction, const int* ops, const uint32_t* lens, uint32_t n_ops,
                    const double* values, uint32_t probe, int* results, double* scores) {
    return guarded([&] {
        kvmem::LrfuHistory h(lambda, fraction);
        kvmem::LrfuState kept;
        size_t cursor = 0;
        for (uint32_t i = 0; i < n_ops; ++i) {
            int r = 0;
            try {
                switch (ops[i]) {
                case 0: h.begin_round(); break;
                case 1:
                    h.preview(std::vector<double>(values + cursor, values + cursor + lens[i]));
                    break;
                case 2: r = h.commit() ? 0 : 2; break;
                case 3: kept = h.checkpoint(); break;
                default: h.restore(kept); break;
                }
            } catch (const std::exception&) {
                r = 1;
            }
            if (ops[i] == 1) cursor += lens[i];
            results[i] = r;
            for (uint32_t b = 0; b < probe; ++b) scores[size_t(i) * probe + b] = h.score(b);
        }
    });
}

}  // extern "C"
