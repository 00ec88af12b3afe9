// kvr_internal.hpp -- kernel argument blocks and launchers shared by the
// C ABI (kvr_capi.cpp) and the kernels (kvr_kernels.hip).  Host side only
// validates; every launcher assumes its arguments were checked.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace kvr {

enum SummarySource : int { kSrcKeysF16 = 0, kSrcKeysQ8 = 1, kSrcSummary = 2 };
constexpr uint32_t kMaxMandatory = 64;  // inline mandatory pages per call
enum Scalar : uint32_t { kScalarF16 = 0, kScalarF32 = 3, kScalarBF16 = 4 };  // kvr_format values
enum Aggregation : uint32_t { kAggMean = 0, kAggMax = 1, kAggMaxLogit = 2 };

struct QueryArgs {
    const uint8_t *data;
    uint32_t scalar;  // Scalar
    uint32_t rows, qheads, kvheads, dim;
    uint64_t row_stride, head_stride, dim_stride, lane_stride;  // bytes
    double scale;
    uint32_t dense;  // (row, head, dim) packed: element i sits at i * element size
    uint32_t packed16;  // dense fp16 with 16-byte aligned lanes: loadable 8 elements at a time
};

// Page summaries of `lanes` histories, optionally fused with the logits of
// every query vector against every page.
struct SummaryArgs {
    const uint8_t *src;        // keys (token-major rows) or fp16 summaries
    uint64_t src_lane_stride;  // bytes
    uint64_t tokens;           // per lane (keys)
    uint32_t page_tokens;
    uint32_t pages;            // per lane
    uint32_t width;            // kv_heads * head_dim
    uint32_t lanes;
    float *means;              // [lanes][pages][width] or null
    uint16_t *summaries;       // [lanes][pages][width] or null
    QueryArgs q;               // fused logits only
    uint32_t q_stage;          // stage the query in LDS (rows*qheads*dim*2 bytes)
    double *logits;            // [lanes][rows*qheads][pages]
    uint32_t *status;
    uint32_t epoch;
};

struct PackQueryArgs {
    QueryArgs q;
    uint32_t lanes;
    uint16_t *out;  // [lanes][rows][qheads][dim] fp16
    uint32_t *status;
    uint32_t epoch;
};

struct MfmaLogitsArgs {
    const uint16_t *qpack;      // [lanes][rows][qheads][dim]
    const uint16_t *summaries;  // [lanes][pages][kvheads*dim]
    uint32_t lanes, pages, rows, qheads, kvheads, dim;
    double scale;
    double *logits;             // [lanes][rows*qheads][pages]
};

struct SelectArgs {
    // softmax units (k_probs): the lane's logits rows, overwritten with the
    // units' aggregation terms (short rows with few units keep the terms in
    // LDS instead); `units` per lane, counted in counters[lane]
    double *logits;            // [lanes][rows*qheads][pages]
    double *stats;             // [lanes][units][2]: long Mean rows' (max, sum), or null
    const uint8_t *mask;       // [pages] or null
    uint32_t units;
    uint32_t *counters;        // [lanes], zero between launches
    // aggregation (do_aggregate): scores[lane][p] (+)= sum of the terms
    uint32_t rows, qheads, kvheads;
    uint32_t aggregation;
    double weight;             // active_layers * heads
    int accumulate;
    int do_aggregate;
    // selection (do_select)
    double *scores;            // [lanes][pages]
    uint32_t lanes, pages, k;
    uint32_t tie_higher_first;
    int signed_scores;
    int do_select;
    uint32_t n_mandatory;      // inline fixed pages (any order)
    uint32_t mandatory[kMaxMandatory];
    const uint32_t *fixed;     // device list of fixed pages (any order, repeats allowed) or null
    uint32_t n_fixed;
    // media groups (k_select_groups only): pages of a group are kept whole
    const uint32_t *groups;    // [n_groups][2] disjoint page ranges [begin, end)
    uint32_t n_groups;
    // pages ranked before every other page (k_select_groups only)
    const uint32_t *preferred;        // [lanes][preferred_stride] or null
    const uint32_t *preferred_count;  // [lanes]
    uint32_t preferred_stride;
    // half-page scoring: the softmax columns are half pages (pages = 2 x the
    // selected pages), the score mask is per selected page (column j reads
    // mask[j >> mask_shift]); the tail folds each pair of half masses into
    // one page score (kFoldSum: left + right, kFoldMax: the larger)
    uint32_t fold;
    uint32_t mask_shift;
    uint32_t *selected;        // [lanes][k]
    uint32_t *count;           // [lanes]
    uint32_t *status;
    uint32_t epoch;
    // layer stacks: the softmax workgroups compute the logits themselves
    // from the fp16 summaries and the query (null: the logits are given)
    const uint16_t *summaries;  // [lanes][pages][kvheads*dim]
    QueryArgs q;
};

// Softmax units per 256-thread workgroup: one per wave for rows held in
// registers (up to 1024 pages), the whole workgroup for longer rows.
enum Fold : uint32_t { kFoldNone = 0, kFoldSum = 1, kFoldMax = 2 };
// Pages the selection runs over (half-page columns fold in pairs).
__host__ __device__ inline uint32_t select_pages(const SelectArgs &a) { return a.fold ? a.pages / 2 : a.pages; }

constexpr uint32_t kUnitsPerBlock = 4;
__host__ __device__ constexpr uint32_t units_per_block(uint32_t pages) { return pages <= 1024 ? kUnitsPerBlock : 1; }

// One launch of a layer stack (k_stack_group): the summaries of m layers
// and the softmax units and selections of the previous group's mp layers.
constexpr uint32_t kStackGroup = 4;
struct StackGroupArgs {
    SummaryArgs s[kStackGroup];
    SelectArgs p[kStackGroup];
    uint32_t m, mp;
    uint32_t summary_blocks;  // summary workgroups: layer_blocks per part of the group's layers
    uint32_t layer_blocks;    // workgroups covering one layer's summaries
    uint32_t layers_per_part; // consecutive layers a summary workgroup walks
    uint32_t probs_per_lane;  // softmax workgroups per lane and layer
    uint32_t q_slot;          // elements of one LDS query staging buffer (multiple of 8)
};

struct GatherPlane {
    const uint8_t *src;   // device-visible pinned (or device staging) base
    uint8_t *dst;
    uint64_t src_lane_stride, dst_lane_stride;
    uint64_t tokens;
    uint32_t src_row, dst_row;  // bytes per token row
    uint32_t width;
    uint32_t format;            // kvr_format of the source
    uint32_t mode;              // kvr_gather_mode
    // raw-K transform (mode 3): rotation and Walsh-Hadamard parameters
    const float *theta;         // [n_rot/2]
    uint32_t head_dim, n_rot, fwht;
    float fwht_scale;           // 1/sqrt(fwht) in binary32
    int64_t pos_base;           // position of history token 0
    uint64_t page_stride;       // 0: token-major source; else page p at p * page_stride
};

struct GatherArgs {
    GatherPlane plane[8];
    uint32_t n_planes;
    uint32_t lanes, k, page_tokens;
    uint32_t chunk_rows;        // token rows per workgroup
    uint32_t chunks;            // per page
    const uint32_t *selected;   // [lanes][k]; null -> slot i holds page i
    const uint32_t *count;      // [lanes]; null -> k
    uint64_t src_page_stride;   // 0: read pinned history; else staged page i at i*stride
    uint32_t workgroups;        // grid bound of the persistent gather
    uint32_t threads;           // workgroup size (64, 128 or 256)
    uint32_t lds_per_wave;      // staging bytes per wave (set by the launcher)
};

struct AccumulateArgs {
    float *sums;                // [pages][width]
    uint32_t *counts;           // [pages]
    uint32_t page_tokens, width, dim;
    const uint8_t *k;
    uint32_t scalar;
    uint64_t pos0;
    uint32_t n;
    uint64_t token_stride, head_stride, dim_stride;
    uint32_t first_page, segments;
};

struct FinalizeArgs {
    const float *sums;
    const uint32_t *counts;
    uint32_t pages, width;
    float *means;
    uint16_t *summaries;
    uint32_t *status;
    uint32_t epoch;
};

struct CopyOp {
    const uint8_t *src;
    uint8_t *dst;
    uint64_t bytes;
};

// ---- launchers (kvr_kernels.hip) ------------------------------------------
// start/stop (either may be null): events stamped with the launch's own
// start and end.
hipError_t launch_summary(int source, bool fuse, const SummaryArgs &a, hipStream_t s, hipEvent_t start = nullptr,
                          hipEvent_t stop = nullptr);
hipError_t launch_pack_query(const PackQueryArgs &a, hipStream_t s);
hipError_t launch_logits_mfma(const MfmaLogitsArgs &a, hipStream_t s);
// page softmax -> terms -> aggregation (+ selection); grid (units, lanes)
hipError_t launch_probs(const SelectArgs &a, hipStream_t s);
// selection over given scores, one workgroup per lane
hipError_t launch_select(const SelectArgs &a, hipStream_t s);
// selection with media groups and preferred pages (rows of at most
// kGroupSelectPages pages), one workgroup per lane
constexpr uint32_t kGroupSelectPages = 4096;
hipError_t launch_select_groups(const SelectArgs &a, hipStream_t s);
// pages per lane whose fixed-page bitmap the selection tails hold (LDS)
constexpr uint32_t kFixedBitmapPages = 524288;
// one stack launch: `pa`'s softmax/selection beside `sa`'s summaries with
// fused logits (sa.q and sa.logits set)
// start/stop (either may be null): events stamped with the launch's own
// start and end.
hipError_t launch_stack_group(int source, StackGroupArgs g, hipStream_t s, hipEvent_t start = nullptr,
                              hipEvent_t stop = nullptr);
hipError_t launch_gather(const GatherArgs &a, hipStream_t s);
hipError_t launch_accumulate(const AccumulateArgs &a, hipStream_t s);
hipError_t launch_finalize(const FinalizeArgs &a, hipStream_t s);
hipError_t launch_copy_ops(const CopyOp *ops, uint32_t n, hipStream_t s);
// bytes (a multiple of 16) of device-visible pinned memory read by a kernel
hipError_t launch_link_read(const void *src, void *dst, uint64_t bytes, hipStream_t s);

// Half-page masses [lanes][2 * pages] -> page scores [lanes][pages]
// (layerwise_tile_scores' sum, layerwise_max_page_scores' max), with the
// reference's validation (a negative or non-finite half, or mass on a masked
// page, raises the scores status and leaves the lane's scores unwritten).
struct FoldArgs {
    const double *halves;
    const uint8_t *mask;   // [pages] or null
    uint32_t lanes, pages, rule;
    double *scores;
    uint32_t *status;
    uint32_t epoch;
};
hipError_t launch_fold_halves(const FoldArgs &a, hipStream_t s);

// ---- static scratch of the no-allocation entry (kvr_scratch.hip) ----------
// Layout: kScratchCounters per-lane completion counters, then the logits
// (binary64) and the packed fp16 queries of one layer.
constexpr size_t kScratchBytes = size_t(16) << 20;
constexpr uint32_t kScratchCounters = 1024;
constexpr size_t kScratchCounterBytes = size_t(kScratchCounters) * sizeof(uint32_t);
// Looks up this device's copy of the array (the device must be current);
// once per device, later calls return at once.
hipError_t scratch_init(int device);
// The device address found by scratch_init, or null before it.
uint8_t *scratch_address(int device);
// n words at p set to v (a kernel, so the clear can sit inside a graph).
hipError_t launch_fill_u32(uint32_t *p, uint32_t n, uint32_t v, hipStream_t s);

enum SynthKind : int {
    kSynthNormalF16 = 0, kSynthScaledNormalF16 = 1, kSynthNormalF32 = 2,
    kSynthQ8 = 3, kSynthQ41 = 4, kSynthNormalQ8 = 5
};
struct SynthArgs {
    int kind;
    uint64_t base;
    uint64_t count;    // elements, or blocks for q8_0 / q4_1
    uint32_t width;    // scaled normal
    const float *scale;
    float lo, hi, lo2, hi2;
    void *out;
};
hipError_t launch_synth(const SynthArgs &a, hipStream_t s);

// Graph propagation and LRFU preview of per-page scores: one workgroup per
// lane, the lane's pages in LDS.
constexpr uint32_t kGraphLanes = 16;       // lanes per launch (kernarg table)
constexpr uint32_t kGraphMaxPages = 8192;  // 8 bytes of LDS per page
struct GraphLane {
    uint32_t n_rows, n_edges;
    const uint32_t *row_source, *row_begin, *edge_target;
    const double *edge_mass, *neighbor_weight;
};
struct GraphLrfuArgs {
    double *scores;         // [lanes][pages]; propagated in place
    const uint8_t *mask;    // [lanes][pages] transport nodes, or null (all)
    uint32_t pages;
    uint32_t lane0;         // first lane of this launch
    int propagate;
    double alpha;
    GraphLane graph[kGraphLanes];
    int lrfu;
    const double *history;  // [lanes][history_pages] or null
    uint32_t history_pages;
    double lambda;
    int gate;               // threshold applies (top fraction < 1)
    uint32_t rank;          // ascending rank of the threshold score
    double *candidate;      // [lanes][pages]
    uint32_t *status;
    uint32_t epoch;
};
// One launch per kGraphLanes lanes; `graphs` holds every lane's graph.
hipError_t launch_graph_lrfu(GraphLrfuArgs a, const GraphLane *graphs, uint32_t lanes, hipStream_t s);

// Sampled attention page masses (kvr_attention.hip).  Key formats are
// kvr_format values; query and mask scalars are Scalar values.
enum KeyFormat : uint32_t { kKeyF16 = 0, kKeyQ8 = 1, kKeyF32 = 3, kKeyBF16 = 4, kKeyQ4 = 5, kKeyQ5 = 6 };
constexpr uint32_t kAttnRows = 64;  // sampled rows per launch (kernarg table)
struct AttnArgs {
    const uint8_t *q;
    uint64_t q_row_stride, q_head_stride;
    const uint8_t *k;
    uint64_t k_row_stride, k_head_stride;
    const uint8_t *mask;
    uint64_t mask_row_stride;
    uint32_t q_scalar, mask_scalar, k_format;
    uint32_t dim, heads, kvheads, group;
    uint32_t tokens, page_tokens, pages;
    uint32_t page_group;  // pages per workgroup, 1..16
    float scale, softcap;
    float *lse;       // [n_rows][heads][pages]
    float *stats;     // [n_rows][heads][page groups][2]: max, sum of exp(lse - max)
    float *mass;      // [n_rows][pages], this launch's first row
    uint32_t n_rows;  // <= kAttnRows
    uint32_t rows[kAttnRows];       // query rows
    uint32_t mask_rows[kAttnRows];  // mask rows
};
// Both launches of one batch of rows: page log-sum-exps, then the
// normalized, head-averaged masses.
hipError_t launch_attention(const AttnArgs &a, hipStream_t s);

}  // namespace kvr
