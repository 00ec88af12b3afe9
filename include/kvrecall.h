/*
 * kvrecall.h -- C ABI of the MI355X (gfx950) KVMem recall hot path.
 *
 * One layer of recall is: page summaries (mean-K) -> GQA query-vs-summary
 * scoring -> page softmax + head aggregation -> top-k page selection ->
 * gather of the selected K/V pages from pinned host history into a device
 * slot array (copy, dequantize to fp16, or requantize to q8_0).
 *
 * Conventions
 *  - Plain C: pointers, sizes and enums.  No exceptions cross this boundary.
 *  - Every entry returns kvr_status; on failure kvr_last_error() holds a
 *    message for the calling thread.  Geometry is validated on the host before
 *    any launch: a rejected call launches nothing.
 *  - "dev" pointers are device memory of the context's GPU, "pinned" pointers
 *    are page-locked host memory (hipHostMalloc, or kvr_host_alloc), "host"
 *    pointers are ordinary host memory read during the call.
 *  - Streams are passed as `void*` (a hipStream_t); NULL selects the
 *    context's own streams.  Calls are asynchronous on their stream.  Device
 *    side operand errors (a query or summary value that is non-finite or
 *    rounds to fp16 infinity) make the selection of that call empty and are
 *    reported by kvr_check(); a raised error stays raised until kvr_check
 *    reports it.
 *  - Graph capture: the scoring, selection and kernel-engine gather entries
 *    allocate nothing and never wait on the host once the context's
 *    workspace is large enough, so they may be recorded into a HIP graph
 *    (hipStreamBeginCapture on the select stream; the copy stream joins
 *    through an event and must be joined back before capture ends).  Run
 *    each shape once before capture, or bind a workspace: growth during
 *    capture fails with KVR_ERR_WORKSPACE.  The DMA stage-in engine reads
 *    the selection on the host and refuses capture.
 *  - A context is used by one host thread at a time.  Its calls may use
 *    different streams: a call that uses the context's workspace or
 *    counters on another stream than the previous such call waits on the
 *    device for what that stream has queued.  Calls on captured streams are
 *    not ordered that way: the caller orders them.
 *
 * Reference citations are relative to the KVMem 0.19.0 source tree.
 */
#ifndef KVRECALL_H
#define KVRECALL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KVR_VERSION_MAJOR 0
#define KVR_VERSION_MINOR 1
/* Host mandatory lists up to this length travel inside the launch (and may
 * be graph-captured); longer ones are uploaded by the call. */
#define KVR_MAX_INLINE_MANDATORY 64
#define KVR_MAX_PLANES 8
/* Layers whose summaries share one launch in kvr_recall_stack. */
#define KVR_STACK_GROUP 4

typedef struct kvr_context kvr_context;

typedef enum kvr_status {
    KVR_OK = 0,
    KVR_ERR_INVALID = 1,     /* invalid argument or geometry                    */
    KVR_ERR_NONFINITE = 2,   /* recall operand NaN/inf (recall_fp16 rejects)    */
    KVR_ERR_RANGE = 3,       /* recall operand rounds to fp16 infinity          */
    KVR_ERR_BUDGET = 4,      /* mandatory pages (with their media groups) exceed
                              * the selection budget                           */
    KVR_ERR_WORKSPACE = 5,   /* borrowed workspace too small for the call       */
    KVR_ERR_HIP = 6,         /* HIP runtime error                               */
    KVR_ERR_SCORES = 7,      /* negative or non-finite score without signed mode*/
    KVR_ERR_UNSUPPORTED = 8, /* format/mode combination not provided            */
    KVR_ERR_GRAPH = 9        /* invalid graph mass or weight, or a propagation  *
                              * result below its signed residual                */
} kvr_status;

typedef enum kvr_format {
    KVR_FMT_F16 = 0,   /* binary16                                          */
    KVR_FMT_Q8_0 = 1,  /* blocks of 32: {fp16 d; int8 qs[32]}, 34 bytes     */
    KVR_FMT_Q4_1 = 2,  /* blocks of 32: {fp16 d; fp16 m; u8 qs[16]}, 20 bytes*/
    KVR_FMT_F32 = 3,   /* binary32 (query and capture input only)           */
    KVR_FMT_BF16 = 4,  /* bfloat16 (query and capture input only)           */
    KVR_FMT_Q4_0 = 5,  /* blocks of 32: {fp16 d; u8 qs[16]}, 18 bytes;
                          element i: ((qs[i%16] >> (i<16 ? 0 : 4)) & 15) - 8,
                          times d (attention keys, gather copy and raw-K
                          transform)                                       */
    KVR_FMT_Q5_0 = 6   /* blocks of 32: {fp16 d; u8 qh[4]; u8 qs[16]}, 22
                          bytes; the q4_0 nibble plus bit i of qh (little
                          endian) as bit 4, minus 16, times d (attention
                          keys only)                                       */
} kvr_format;

typedef enum kvr_aggregation {
    KVR_AGG_MEAN = 0,      /* GqaScoreAggregation::Mean                        */
    KVR_AGG_MAX = 1,       /* GqaScoreAggregation::Max (max of probabilities)  */
    KVR_AGG_MAX_LOGIT = 2  /* max of the group's logits, then one softmax      */
} kvr_aggregation;

typedef enum kvr_tie_rule {
    KVR_TIE_LOWER_FIRST = 0,  /* equal scores: lower page id wins              */
    KVR_TIE_HIGHER_FIRST = 1  /* equal scores: higher id wins (KvMemStore rule) */
} kvr_tie_rule;

typedef enum kvr_gather_mode {
    KVR_GATHER_COPY = 0,         /* bytes unchanged                           */
    KVR_GATHER_DEQUANT_F16 = 1,  /* decode to binary32, RNE to binary16       */
    KVR_GATHER_REQUANT_Q8_0 = 2, /* q8_0 -> binary32 -> q8_0                   */
    KVR_GATHER_ROPE_FWHT = 3     /* raw K (q8_0 or q4_0): decode, NeoX RoPE at
                                    the token's position, Walsh-Hadamard
                                    transform, requantize to the source format
                                    (plane.rope holds the parameters)         */
} kvr_gather_mode;

/* Parameters of KVR_GATHER_ROPE_FWHT (kvmem_stagein_enqueue_k,
 * src/adapter/llama-kvmem-stagein.h:37-42).  Token t of the history has
 * position pos_base + t.  In each head of head_dim values, pairs (i, i +
 * n_rot/2) for i < n_rot/2 rotate by (position * theta[i]); then each run of
 * fwht values of the row (0: none) is scaled by 1/sqrt(fwht) and
 * Walsh-Hadamard transformed. */
typedef struct kvr_rope {
    uint32_t head_dim;     /* width is a multiple of it */
    uint32_t n_rot;        /* even, at most head_dim and 512 (0: no rotation) */
    const float *theta;    /* dev, n_rot/2 values */
    uint32_t fwht;         /* 0, 64, 128, 256 or 512; divides width */
    int64_t pos_base;
} kvr_rope;

typedef enum kvr_copy_engine {
    KVR_ENGINE_AUTO = 0,    /* the faster engine for the mode                 */
    KVR_ENGINE_KERNEL = 1,  /* device-driven kernel reading pinned memory     */
    KVR_ENGINE_SDMA = 2     /* DMA copies (host reads the selection first)    */
} kvr_copy_engine;

/* Resident key history of `lanes` independent sequences, token-major rows of
 * kv_heads*head_dim channels.  Lane i starts at data + i*lane_stride bytes. */
typedef struct kvr_key_history {
    const void *data;       /* dev */
    kvr_format format;      /* KVR_FMT_F16 or KVR_FMT_Q8_0 */
    uint64_t tokens;        /* per lane */
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t page_tokens;
    uint32_t lanes;         /* 0 is read as 1 */
    size_t lane_stride;     /* bytes; 0 = tightly packed */
} kvr_key_history;

/* Query rows of one layer: element (lane, r, h, d) at
 * data + lane*lane_stride + r*row_stride + h*head_stride + d*dim_stride. */
typedef struct kvr_query {
    const void *data;       /* dev */
    kvr_format scalar;      /* KVR_FMT_F32, KVR_FMT_F16 or KVR_FMT_BF16 */
    uint32_t rows;
    uint32_t query_heads;
    uint32_t kv_heads;
    uint32_t head_dim;
    size_t row_stride, head_stride, dim_stride, lane_stride; /* bytes */
    float attention_scale;  /* 0 selects 1/sqrt(head_dim) */
} kvr_query;

/* One plane (K or V) of one layer's history for the gather.  Lane i reads
 * history + i*host_lane_stride and writes slots + i*slot_lane_stride.
 * Slot s of a lane holds the lane's s-th selected page (ascending page id)
 * at rows [s*page_tokens, s*page_tokens + valid). */
typedef struct kvr_plane {
    const void *history;    /* pinned, token-major rows */
    kvr_format format;      /* KVR_FMT_F16, KVR_FMT_Q8_0, KVR_FMT_Q4_1 or KVR_FMT_Q4_0 */
    uint32_t width;         /* channels per token row */
    uint64_t tokens;        /* per lane */
    kvr_gather_mode mode;
    void *slots;            /* dev */
    size_t host_lane_stride, slot_lane_stride; /* bytes; 0 = tightly packed */
    const kvr_rope *rope;   /* KVR_GATHER_ROPE_FWHT only (else ignored) */
    /* 0: history is token-major (page p's rows start at p * page_tokens
     * rows).  Else page p's rows start at history + p * page_stride, one
     * native payload record per page: history points at the plane's offset
     * in the first record, page_stride is the record size and the plane's
     * rows are contiguous (PayloadPlane token_stride = the row size;
     * kvmem/include/kvmem/memory_contract.hpp:43-68).  host_lane_stride
     * 0 then means pages * page_stride. */
    size_t page_stride;
} kvr_plane;

/* Half-page scoring (layerwise Mean-K on a grid of half the transport page,
 * kvmem/src/host/layerwise_selection.cpp:14-75): the summaries are half
 * pages, one softmax runs over every half, and each transport page's score
 * is its halves' masses folded. */
typedef enum kvr_half_fold {
    KVR_HALF_NONE = 0,  /* summaries are the transport pages                */
    KVR_HALF_SUM = 1,   /* left + right (layerwise_tile_scores, :60-72)     */
    KVR_HALF_MAX = 2    /* the larger half (layerwise_max_page_scores,
                           :24-30, for a Query scored in one call)          */
} kvr_half_fold;

/* Pages a device selection keeps besides its best-scored ones, all in
 * device memory so that the call can be graph-captured (the lists are read
 * when the selection runs).  Replaces the `mandatory` and media-range
 * arguments of KvMemStore::pick_scored_blocks
 * (kvmem/src/host/kvmem_store.cpp:418-451). */
typedef struct kvr_page_policy {
    const uint32_t *fixed;           /* dev: pages kept first in every lane, any
                                        order, repeats allowed, ids >= pages
                                        ignored; each brings its whole group and
                                        together they must fit k (else the lane's
                                        selection is empty and kvr_check reports
                                        KVR_ERR_BUDGET)                         */
    uint32_t n_fixed;
    const uint32_t *groups;          /* dev [n_groups][2]: disjoint ascending page
                                        ranges [begin, end) kept whole or not at
                                        all (kvr_media_page_groups); the pages
                                        are then visited in rank order and a
                                        group that no longer fits is skipped.
                                        NULL: every page alone                 */
    uint32_t n_groups;
    const uint32_t *preferred;       /* dev [lanes][preferred_stride]: pages ranked
                                        before every other page (the second pass
                                        of KvMemStore::pick_topk_blocks), or NULL */
    const uint32_t *preferred_count; /* dev [lanes]                              */
    uint32_t preferred_stride;
} kvr_page_policy;

/* One layer of recall for `lanes` sequences (kvr_recall_layer). */
typedef struct kvr_layer_recall {
    const kvr_key_history *keys;   /* resident keys to summarize, or NULL to
                                      score the resident `summaries` as given */
    uint16_t *summaries;           /* dev fp16 [lanes][pages][Hkv*D] */
    float *means;                  /* dev, optional binary32 mean-K output */
    uint32_t pages;                /* pages per lane (when keys is NULL) */
    uint32_t page_tokens;          /* (when keys is NULL) */
    uint32_t lanes;                /* (when keys is NULL; 0 is read as 1) */
    const kvr_query *query;
    const uint8_t *score_mask;     /* dev [pages] or NULL for all pages */
    kvr_aggregation aggregation;
    uint32_t k;                    /* selection budget per lane */
    kvr_tie_rule tie_rule;
    const uint32_t *mandatory;     /* host, any number of ids (up to
                                      KVR_MAX_INLINE_MANDATORY distinct ones
                                      inside the launch; more are uploaded
                                      and then refuse graph capture)        */
    uint32_t n_mandatory;
    double *scores;                /* dev [lanes][pages] */
    uint32_t *selected;            /* dev [lanes][k], ascending ids */
    uint32_t *count;               /* dev [lanes] */
    const kvr_plane *planes;       /* gather targets, may be NULL */
    uint32_t n_planes;
    kvr_copy_engine engine;
    int force_mfma;                /* -1 never, 0 by rows*group >= 16, 1 always */
    void *summary_begin;           /* optional hipEvent_t stamped with the
                                      start / end of the summary kernel (with
                                      resident summaries: recorded on the
                                      select stream just before / after the
                                      logits kernels) */
    void *summary_end;             /* (measurement only; may be NULL;
                                      refused while the stream is captured)  */
    void *select_end;              /* optional hipEvent_t recorded on the select
                                      stream once the selection is written,
                                      before any stage-in is enqueued (same
                                      rules as the summary events)           */
    const kvr_page_policy *policy; /* optional device-side fixed pages, media
                                      groups and preferred pages (besides
                                      `mandatory`); with groups or preferred
                                      pages the selection is its own launch
                                      (pages <= KVR_GROUP_SELECT_PAGES)      */
    kvr_half_fold half_fold;       /* KVR_HALF_NONE, or the key history's (or
                                      resident summaries') pages are half
                                      transport pages: the history holds whole
                                      transport pages of two summary pages;
                                      summaries and the softmax cover the
                                      halves; score_mask, mandatory, policy,
                                      scores, the selection and the gather
                                      (2 * page_tokens rows per slot) are per
                                      transport page                         */
} kvr_layer_recall;

/* ---- context ------------------------------------------------------------ */

/* Replaces PageSoftmaxCuda(int device) (kvmem/include/kvmem/page_softmax_cuda.hpp:13)
 * and kvmem_gpu_state_create (src/adapter/llama-kvmem-stagein.h:12). */
kvr_status kvr_create(int device, kvr_context **out);
/* Replaces ~PageSoftmaxCuda and kvmem_gpu_state_free (llama-kvmem-stagein.h:14):
 * drains the context's streams, then releases what it owns. */
kvr_status kvr_destroy(kvr_context *ctx);
/* Thread-local message of the last failed call (stderr text of cuda_ok,
 * llama-kvmem-stagein.cu:93-99; exception text of page_softmax.cu:15-17). */
const char *kvr_last_error(void);
const char *kvr_status_string(kvr_status status);
/* Drains `stream` (NULL: both context streams) and reports the first device
 * side operand error raised since the previous check.  Replaces
 * kvmem_stagein_sync_checked (llama-kvmem-stagein.h:34) and the poison-flag
 * readback of score_current_layer (page_softmax.cu:372-375). */
kvr_status kvr_check(kvr_context *ctx, void *stream);
/* The context's own streams (hipStream_t), for event wiring by callers. */
void *kvr_select_stream(kvr_context *ctx);
void *kvr_copy_stream(kvr_context *ctx);

typedef enum kvr_option {
    KVR_OPT_GATHER_WORKGROUPS = 1, /* grid bound of the device-driven gather (default: 16
                                      for copies, 32 when a plane decodes) */
    KVR_OPT_GATHER_CHUNK_ROWS = 2, /* token rows per gather work item (default 8, <= 64) */
    KVR_OPT_GATHER_THREADS = 3,    /* gather workgroup size: 64, 128 or 256 (default: 64
                                      for copies, 256 when a plane decodes) */
    KVR_OPT_ATTN_PAGE_GROUP = 4    /* pages per attention-sampler workgroup, 1..16
                                      (default: by the call's size) */
} kvr_option;

/* Tuning knobs of a context; value 0 restores the default.  No reference
 * counterpart (the reference's slab size and op table are compile-time
 * constants, llama-kvmem-stagein.cu:32-33). */
kvr_status kvr_set_option(kvr_context *ctx, kvr_option option, int64_t value);

/* ---- workspace ------------------------------------------------------------ */

/* Device bytes one scoring call needs for this geometry.  Replaces
 * PageSoftmaxCuda::workspace_bytes (page_softmax_cuda.hpp:15). */
size_t kvr_workspace_bytes(uint32_t lanes, uint32_t max_pages, uint32_t max_rows,
                           uint32_t query_heads, uint32_t kv_heads, uint32_t head_dim);
/* Borrow a caller-planned workspace (256-byte aligned dev memory): afterwards
 * no call on this context allocates device memory, and a call that needs more
 * fails with KVR_ERR_WORKSPACE before any launch.  Replaces the borrowed
 * workspace constructor (page_softmax_cuda.hpp:16-17, page_softmax.cu:181-192). */
kvr_status kvr_bind_workspace(kvr_context *ctx, void *workspace, size_t bytes);
/* Device bytes currently owned or borrowed.  Replaces device_bytes()
 * (page_softmax_cuda.hpp:28). */
size_t kvr_device_bytes(kvr_context *ctx);

/* ---- page summaries ---------------------------------------------------- */

/* Per page, per channel: binary32 sum of the page's key rows in token order
 * from zero, times (1.0f/valid_tokens); then the fp16 operand rounding of
 * recall_fp16.  Replaces RawKvStore::capture_mean_f16 / add_mean_f32 /
 * mean_k (kvmem/src/host/raw_kv_store.cpp:158-197, 606-625) followed by the
 * host staging loop of PageSoftmaxCuda::score (page_softmax.cu:239-248).
 * means: dev [lanes][pages][Hkv*D] or NULL; summaries: dev fp16, same shape. */
kvr_status kvr_summary_build(kvr_context *ctx, const kvr_key_history *keys, float *means,
                             uint16_t *summaries, void *stream);

/* Capture-side running sum: adds n key rows at positions pos0.. of one
 * sequence into per-page binary32 sums (a segment starting at page offset 0
 * restarts that page's sum), one channel per thread, token order.  Replaces
 * kvmem_meank_add (llama-kvmem-stagein.h:63, stagein.cu:270-320) and
 * RawKvStore::write_layer_mean_k (raw_kv_store.cpp:422-441).
 * Element (t, h, d) of k is at k + t*token_stride + h*head_stride + d*dim_stride. */
kvr_status kvr_summary_accumulate(kvr_context *ctx, float *sums, uint32_t *counts,
                                  uint32_t page_tokens, const void *k, kvr_format scalar,
                                  uint64_t pos0, uint32_t n, uint32_t kv_heads,
                                  uint32_t head_dim, size_t token_stride,
                                  size_t head_stride, size_t dim_stride, void *stream);
/* means = sums * (1.0f/counts), summaries = fp16 operand of means (pages with
 * count 0 give zeros).  Replaces RawKvStore::mean_k (raw_kv_store.cpp:606-614). */
kvr_status kvr_summary_finalize(kvr_context *ctx, const float *sums, const uint32_t *counts,
                                uint32_t pages, uint32_t width, float *means,
                                uint16_t *summaries, void *stream);

/* ---- scoring --------------------------------------------------------------- */

/* Page softmax scores of one layer: logits scale*sum_d fp16(q)*fp16(summary)
 * in binary64, softmax over the pages of score_mask, then the head
 * aggregation.  out += mass / (active_layers * heads) when `accumulate`,
 * so calling it once per active layer reproduces the multi-layer sum.
 * Replaces page_softmax_scores (kvmem/src/host/graph_recall.cpp:322-394),
 * PageSoftmaxCuda::score / score_current_layer (page_softmax.cu:202-396) and
 * layerwise_mean_key_scores (kvmem/src/host/layerwise_scoring.cpp:10-63).
 * summaries: dev fp16 [lanes][pages][Hkv*D]; scores: dev [lanes][pages]. */
kvr_status kvr_score(kvr_context *ctx, const kvr_query *q, const uint16_t *summaries,
                     uint32_t lanes, uint32_t pages, const uint8_t *score_mask,
                     kvr_aggregation aggregation, uint32_t active_layers, int accumulate,
                     double *scores, int force_mfma, void *stream);

/* ---- selection ------------------------------------------------------------- */

/* Per lane: mandatory pages first (host list, any length), then the top of
 * (score desc, id by tie rule) up to k pages; ids ascending.  Rejects (device side, empty result,
 * KVR_ERR_SCORES at kvr_check) a negative or non-finite score unless
 * signed_scores.  Replaces KvMemStore::pick_scored_blocks
 * (kvmem/src/host/kvmem_store.cpp:418-451) with every page a candidate.
 * scores: dev [lanes][pages]; selected: dev [lanes][k]; count: dev [lanes]. */
kvr_status kvr_select_topk(kvr_context *ctx, const double *scores, uint32_t lanes,
                           uint32_t pages, uint32_t k, const uint32_t *mandatory,
                           uint32_t n_mandatory, kvr_tie_rule tie_rule, int signed_scores,
                           uint32_t *selected, uint32_t *count, void *stream);

/* Half-page masses [lanes][2 * pages] (kvr_score over the half pages, with
 * `accumulate` over Query tiles) folded into page scores [lanes][pages]:
 * layerwise_tile_scores' left + right or, at the end of a tiled Query,
 * layerwise_max_page_scores (kvmem/src/host/layerwise_selection.cpp:24-75).
 * A negative or non-finite half, or mass on a page outside score_mask
 * ([pages] or NULL), raises KVR_ERR_SCORES at kvr_check and leaves that
 * lane's scores unwritten. */
kvr_status kvr_fold_half_pages(kvr_context *ctx, const double *halves, uint32_t lanes, uint32_t pages,
                               const uint8_t *score_mask, kvr_half_fold rule, double *scores, void *stream);

/* Rows of at most this many pages per lane take media groups or preferred
 * pages; rows of at most KVR_FIXED_BITMAP_PAGES take fixed pages. */
#define KVR_GROUP_SELECT_PAGES 4096
#define KVR_FIXED_BITMAP_PAGES 524288

/* kvr_select_topk with a device-side page policy (NULL: none).  Without
 * groups or preferred pages it is the same one-wave/one-workgroup top-k;
 * with them each lane's pages are put in rank order (preferred first,
 * score desc, id by tie rule) and walked, keeping each group or lone page
 * that still fits: KvMemStore::pick_scored_blocks with media ranges
 * (kvmem/src/host/kvmem_store.cpp:418-451) and the fill of constrain_media
 * (:453-502). */
kvr_status kvr_select_pages(kvr_context *ctx, const double *scores, uint32_t lanes, uint32_t pages, uint32_t k,
                            const kvr_page_policy *policy, kvr_tie_rule tie_rule, int signed_scores,
                            uint32_t *selected, uint32_t *count, void *stream);

/* ---- page policies on the host (no device work) ----------------------- */

/* Media (image) token ranges of a history, in the order the engine recorded
 * them: ranges[2i] is the first token of range i, ranges[2i+1] one past its
 * last.  A range covers pages [first / page_tokens, ceil(end / page_tokens)). */
typedef struct kvr_media {
    const uint32_t *ranges;
    uint32_t n_ranges;
    uint32_t page_tokens;
    uint64_t total_tokens;   /* tokens in the history */
} kvr_media;

typedef enum kvr_media_merge {
    KVR_MEDIA_OVERLAP = 0,   /* ranges that share a page join, transitively
                                (scored_media_group, kvmem_store.cpp:18-32)  */
    KVR_MEDIA_IN_ORDER = 1   /* ranges starting at or past total_tokens or
                                empty are dropped; a range starting before
                                the previous group's end extends it, in list
                                order (constrain_media, kvmem_store.cpp:453-468) */
} kvr_media_merge;

/* The page groups of `media` over `pages` pages: disjoint ascending
 * [begin, end) pairs written to groups (room for n_ranges pairs).  The
 * device list of kvr_page_policy.groups. */
kvr_status kvr_media_page_groups(const kvr_media *media, uint32_t pages, kvr_media_merge merge, uint32_t *groups,
                                 uint32_t *n_groups);

/* The fixed pages of a Query pick, ascending: every page when budget is 0
 * or at least pages; else the sink pages, the page where the last media
 * range starts (when it starts before total_tokens) and the mandatory pages,
 * each with its whole OVERLAP group and required to fit (KVR_ERR_BUDGET; a
 * mandatory id >= pages: KVR_ERR_INVALID), then the newest `recent` pages
 * newest first while their groups fit.  media may be NULL.  out: room for
 * `pages` ids.  Replaces KvMemStore::query_fixed_blocks
 * (kvmem/src/host/kvmem_store.cpp:381-408); the result is the fixed list of
 * the device pick with the OVERLAP groups, tie rule higher-first. */
kvr_status kvr_query_fixed_pages(uint32_t pages, uint32_t budget, uint32_t sink, uint32_t recent,
                                 const kvr_media *media, const uint32_t *mandatory, uint32_t n_mandatory,
                                 uint32_t *out, uint32_t *n_out);

/* The kept part of the ungrouped top-k pick, ascending: every page when
 * budget is 0 or at least pages; else, while the budget has room, the sink
 * pages, the mandatory pages from the last listed to the first (ids >= pages
 * ignored) and the newest `recent` pages newest first.  The device pick then
 * fills the budget by score, higher id first on ties.  Replaces the fixed
 * part of KvMemStore::pick_topk_ungrouped (kvmem_store.cpp:578-644). */
kvr_status kvr_topk_fixed_pages(uint32_t pages, uint32_t budget, uint32_t sink, uint32_t recent,
                                const uint32_t *mandatory, uint32_t n_mandatory, uint32_t *out, uint32_t *n_out);

/* The kept part of constrain_media's pass (kvmem_store.cpp:453-490), for
 * histories with media ranges, pages > budget and budget > 0 (else the
 * ungrouped pick stands): the sink pages and the last IN_ORDER group are
 * required (KVR_ERR_BUDGET), then the mandatory pages newest first, each
 * with its group when it fits.  The device pick then takes the ungrouped
 * pick's pages as preferred pages and the IN_ORDER groups, tie rule
 * higher-first: KvMemStore::pick_topk_blocks (kvmem_store.cpp:377-379). */
kvr_status kvr_media_fixed_pages(uint32_t pages, uint32_t budget, uint32_t sink, const kvr_media *media,
                                 const uint32_t *mandatory, uint32_t n_mandatory, uint32_t *out, uint32_t *n_out);

/* ---- stage-in ------------------------------------------------------------ */

/* Gather each lane's selected pages of every plane from pinned history into
 * its slot array.  Reads `selected`/`count` on the device (KERNEL engine) or
 * after waiting for them (SDMA engine).  Replaces write_block_to_gpu
 * (src/adapter/llama-memory-kvmem.cpp:4450-4526) with kvmem_stagein_enqueue_v /
 * kvmem_stagein_flush (src/adapter/llama-kvmem-stagein.h:41-50,
 * stagein.cu:673-794, 861-881) and the dequant/quant kernels
 * (stagein.cu:133-199). */
kvr_status kvr_stage_in(kvr_context *ctx, const kvr_plane *planes, uint32_t n_planes,
                        uint32_t lanes, uint32_t page_tokens, const uint32_t *selected,
                        const uint32_t *count, uint32_t k, kvr_copy_engine engine,
                        void *stream);

/* ---- one layer, end to end -------------------------------------------- */

/* Summaries (or resident summaries) -> scores -> selection on select_stream,
 * then the gather on copy_stream after an event; nothing waits on the host.
 * Replaces score_retrieval + apply_native_selection's stage-in
 * (src/adapter/llama-memory-kvmem.cpp:4604-4653, 5011-5126). */
kvr_status kvr_recall_layer(kvr_context *ctx, const kvr_layer_recall *desc,
                            void *select_stream, void *copy_stream);

/* kvr_recall_layer that allocates nothing, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No reference counterpart.  The
 * scoring logits, packed queries and per-lane counters live in a static
 * device array of KVR_NOALLOC_SCRATCH_BYTES per GPU (held until the process
 * ends; its first KVR_NOALLOC_MAX_LANES * 4 bytes are the counters) instead
 * of the context's workspace; a call whose lanes*rows*query_heads*pages*8
 * bytes of logits, lanes*rows*query_heads*16 of softmax statistics (+
 * lanes*rows*query_heads*head_dim*2 of packed queries on the matrix-core
 * path), each rounded up to 256, do not fit fails with KVR_ERR_WORKSPACE
 * before any launch.  The gather uses the kernel engine
 * (KVR_ENGINE_SDMA with planes: KVR_ERR_UNSUPPORTED).  The context must have
 * been created beforehand (kvr_create allocates; this call does not).  Every
 * call on one GPU shares its array: calls that overlap in time on one GPU,
 * from any context or stream, race and give undefined results. */
#define KVR_NOALLOC_SCRATCH_BYTES (16u << 20)
#define KVR_NOALLOC_MAX_LANES 1024
kvr_status kvr_recall_layer_noalloc(kvr_context *ctx, const kvr_layer_recall *desc, void *select_stream,
                                    void *copy_stream);

/* n layers of recall in order, with results identical to n kvr_recall_layer
 * calls.  When every layer takes the fused vector scoring path with one
 * geometry, the layers go in groups of up to KVR_STACK_GROUP consecutive
 * layers with one summary source, one launch per group: group g's summaries
 * run beside group g-1's softmax units and selections (the context then
 * keeps 2*KVR_STACK_GROUP logits buffers: a borrowed workspace needs
 * 2*KVR_STACK_GROUP times kvr_workspace_bytes of one layer).  Each layer's selection, select_end event
 * and stage-in therefore follow the next group's launch, and a layer's
 * summary events bracket its group's launch: the first layer of a group
 * that has summary events gets them stamped with the launch's own start and
 * end (no markers between kernels), any other layer's are recorded just
 * before and after it.  Otherwise the layers run one after another.  Replaces one select_layerwise_history call per attention
 * layer (kvmem/src/host/layerwise_selection.cpp:185-199), each followed by
 * that layer's stage-in. */
kvr_status kvr_recall_stack(kvr_context *ctx, const kvr_layer_recall *layers, uint32_t n,
                            void *select_stream, void *copy_stream);

/* ---- sampled attention (attention-feedback observer) --------------------- */

/* One layer's sampled attention: for each sampled query row, the softmax of
 * every query head over all key tokens, summed per page of page_tokens
 * tokens and averaged over the heads.  Query element (r, h, d) at
 * q + r*q_row_stride + h*q_head_stride + d*size; the key row of token t and
 * kv-head g at k + t*k_row_stride + g*k_head_stride (head_dim values, in
 * blocks of 32 for the quantized formats); additive mask element (r, t) at
 * mask + r*mask_row_stride + t*size.  Logit = scale*dot, then
 * softcap*tanh(logit/softcap) when softcap > 0, plus the mask; a token with
 * a non-finite mask value is left out. */
typedef struct kvr_attention_sample {
    const void *q;             /* dev */
    kvr_format q_format;       /* KVR_FMT_F32, KVR_FMT_F16 or KVR_FMT_BF16 */
    size_t q_row_stride, q_head_stride;     /* bytes */
    const void *k;             /* dev */
    kvr_format k_format;       /* F16, BF16, F32 (16-byte aligned rows) or
                                  Q8_0, Q4_0, Q5_0 (2-byte aligned rows)  */
    size_t k_row_stride, k_head_stride;     /* bytes */
    const void *mask;          /* dev */
    kvr_format mask_format;    /* KVR_FMT_F32, KVR_FMT_F16 or KVR_FMT_BF16 */
    size_t mask_row_stride;    /* bytes */
    uint32_t head_dim;         /* multiple of 32, at most 256 */
    uint32_t query_heads, kv_heads;
    uint32_t tokens, page_tokens;
    float scale, softcap;
    const uint32_t *rows;      /* host: the sampled query (and mask) rows */
    uint32_t n_rows;
    const uint32_t *mask_rows; /* host, optional: mask row of each sample when
                                  it differs from rows[i] (a mask staged row
                                  by row); NULL: rows[i]                      */
} kvr_attention_sample;

/* Workspace of kvr_attention_page_mass for n_rows sampled rows: up to
 * KVR_ATTENTION_ROWS rows go in one launch, fewer when their page
 * log-sum-exp tables (12 bytes per row, head and page) would pass 32 MiB. */
#define KVR_ATTENTION_ROWS 64
size_t kvr_attention_workspace_bytes(uint32_t n_rows, uint32_t query_heads, uint32_t pages);

/* mass: dev float [n_rows][ceil(tokens/page_tokens)], row i for rows[i].
 * A query head whose every token is masked gives NaN for its row, as in the
 * reference.  Unsupported formats or head_dim: KVR_ERR_UNSUPPORTED (the
 * reference's score() returns false).  Replaces
 * llama_kvmem_attention_cuda::score (src/adapter/llama-kvmem-attention-cuda.h:9-16,
 * .cu:148-193: page_lse, normalize, average at :59-126); asynchronous on
 * `stream` (NULL: the context's select stream). */
kvr_status kvr_attention_page_mass(kvr_context *ctx, const kvr_attention_sample *sample, float *mass,
                                   void *stream);

/* ---- graph propagation and LRFU (between scoring and selection) ---------- */

/* Pages per lane that kvr_propagate_scores / kvr_lrfu_preview take: one
 * workgroup per lane holds the lane's pages in LDS (8 bytes each). */
#define KVR_GRAPH_MAX_PAGES 8192

/* One lane's accepted attention graph, flattened by page: row r moves
 * evidence from page row_source[r] to pages edge_target[row_begin[r] ..
 * row_begin[r+1]) in proportion to edge_mass (the sealed row's mass over its
 * samples).  Only rows with samples and a completed source block belong here
 * (the reference skips the others).  neighbor_weight[i] is the message-span
 * coefficient between pages i and i+1 (1 inside one message, the cross
 * weight across a boundary); NULL means 1 everywhere.  All pointers are
 * device memory; rows may be empty (n_rows 0, pointers NULL). */
typedef struct kvr_page_graph {
    uint32_t n_rows;
    uint32_t n_edges;                /* row_begin[n_rows]                     */
    const uint32_t *row_source;      /* [n_rows] page ids                     */
    const uint32_t *row_begin;       /* [n_rows + 1], nondecreasing           */
    const uint32_t *edge_target;     /* [n_edges] page ids                    */
    const double *edge_mass;         /* [n_edges] finite, >= 0                */
    const double *neighbor_weight;   /* [pages - 1] in [0, 1], or NULL        */
} kvr_page_graph;

/* One hop of positive Query evidence over the graph, in place:
 *   scores = min(raw, 0) + G(max(raw, 0))
 * with every page of transport_mask a node (NULL: every page).  Each node
 * gives alpha/4 of its share to each adjacent node (times the span
 * coefficient) and alpha/2 over its graph row; pages outside the mask
 * neither give nor receive.  alpha 0, at most one node or no positive
 * evidence leave the scores untouched.  Transfers are summed as integers in
 * units of at most 2^-61 of the evidence total, so every run gives the same
 * bits; results match the reference to ~1e-15 of that total.  A non-finite score
 * raises KVR_ERR_SCORES, an invalid mass, weight or row range or a result
 * below its residual KVR_ERR_GRAPH at kvr_check; the scores are then left as
 * they were.  graphs: host array of `lanes` entries (NULL: no graph rows).
 * Replaces propagate_query_scores (kvmem/src/host/graph_recall.cpp:494-552;
 * span_coefficient :234-247) for the frames query_score_frame builds (page i
 * starts at token i * block_tokens).  scores, transport_mask: dev
 * [lanes][pages]. */
kvr_status kvr_propagate_scores(kvr_context *ctx, double *scores, uint32_t lanes, uint32_t pages,
                                const uint8_t *transport_mask, const kvr_page_graph *graphs,
                                double alpha, void *stream);

/* LRFU preview: candidate[i] = lambda * history[i] + gate(scores[i]), where
 * gate keeps a score at or above the top_fraction threshold (the score of
 * ascending rank min(n-1, floor((1 - top_fraction) * n))) and clips the rest
 * to min(score, 0); top_fraction 1 keeps every score.  history pages past
 * history_pages count as 0 (history may be NULL when history_pages is 0).
 * Binary64 with separate roundings, bit-identical to the reference.  A
 * non-finite score raises KVR_ERR_SCORES at kvr_check (candidate unwritten).
 * The caller keeps the candidate and makes it the next history on commit.
 * Replaces LrfuHistory::preview / score (kvmem/include/kvmem/lrfu.hpp:57-90).
 * scores, candidate: dev [lanes][pages] (candidate may be scores);
 * history: dev [lanes][history_pages]. */
kvr_status kvr_lrfu_preview(kvr_context *ctx, const double *scores, uint32_t lanes, uint32_t pages,
                            const double *history, uint32_t history_pages, double lambda,
                            double top_fraction, double *candidate, void *stream);

/* kvr_propagate_scores then kvr_lrfu_preview of the propagated scores, in
 * one launch: scores end propagated, candidate holds the LRFU candidate
 * (the sequence RecallPolicy::query runs,
 * backends/radiance/adapter/recall_policy.hpp:104-117).  Errors as the two
 * calls; a lane whose propagation fails writes neither output (errors are
 * per lane here and in both calls: other lanes complete). */
kvr_status kvr_propagate_lrfu(kvr_context *ctx, double *scores, uint32_t lanes, uint32_t pages,
                              const uint8_t *transport_mask, const kvr_page_graph *graphs, double alpha,
                              const double *history, uint32_t history_pages, double lambda,
                              double top_fraction, double *candidate, void *stream);

/* ---- device copies ------------------------------------------------------- */

/* One launch of n byte copies (16-byte path when aligned).  Replaces
 * kvmem_d2d_batched (llama-kvmem-stagein.h:56, stagein.cu:236-261, 1006-1039).
 * src/dst/nbytes are host arrays of n entries, uploaded by the call through
 * one of four pinned tables (so a call refuses graph capture; a table is
 * reused once the copy launch that read it has run, on any stream). */
kvr_status kvr_d2d_batched(kvr_context *ctx, const void *const *src, void *const *dst,
                           const size_t *nbytes, uint32_t n, void *stream);

/* ---- memory and measurement helpers ------------------------------------ */

/* Page-locked, device-mapped host memory (hipHostMalloc).  Replaces the slab
 * pins of kvmem_stagein_gpu_ready (stagein.cu:392-405). */
kvr_status kvr_host_alloc(size_t bytes, void **out);
kvr_status kvr_host_free(void *ptr);
/* Best-of-`reps` hipMemcpyAsync bandwidth of one `bytes` pinned->device copy,
 * GB/s (10^9 B/s).  Measurement helper with no reference counterpart. */
kvr_status kvr_h2d_peak_gbps(kvr_context *ctx, size_t bytes, int reps, double *gbps);
/* Best-of-`reps` rate of a kernel reading `bytes` (a multiple of 16) of
 * device-mapped pinned memory (the way the gather reads the history) and
 * writing it to device memory, GB/s.  Measurement helper with no reference
 * counterpart. */
kvr_status kvr_h2d_read_peak_gbps(kvr_context *ctx, size_t bytes, int reps, double *gbps);

/* ---- seeded synthetic inputs (device fill) ----------------------------- */
/* Bit-identical to the generator of the test oracle; no reference counterpart.
 * normal: sum of 12 uniform 24-bit fractions minus 6, rounded once. */
kvr_status kvr_synth_normal_f16(kvr_context *ctx, uint64_t seed, uint64_t stream_id,
                                uint64_t count, uint16_t *out, void *stream);
kvr_status kvr_synth_scaled_normal_f16(kvr_context *ctx, uint64_t seed, uint64_t stream_id,
                                       uint64_t rows, uint32_t width, const float *scale,
                                       uint16_t *out, void *stream);
kvr_status kvr_synth_normal_f32(kvr_context *ctx, uint64_t seed, uint64_t stream_id,
                                uint64_t count, float *out, void *stream);
kvr_status kvr_synth_q8_0(kvr_context *ctx, uint64_t seed, uint64_t stream_id,
                          uint64_t blocks, float d_lo, float d_hi, uint8_t *out, void *stream);
kvr_status kvr_synth_q4_1(kvr_context *ctx, uint64_t seed, uint64_t stream_id,
                          uint64_t blocks, float d_lo, float d_hi, float m_lo, float m_hi,
                          uint8_t *out, void *stream);
kvr_status kvr_synth_normal_q8_0(kvr_context *ctx, uint64_t seed, uint64_t stream_id,
                                 uint64_t blocks, uint8_t *out, void *stream);

#ifdef __cplusplus
}
#endif
#endif
