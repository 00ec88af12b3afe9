// kvr_capi.cpp -- the extern "C" boundary (include/kvrecall.h).
//
// Host side: argument validation (nothing launches on a rejected call),
// context streams/events, workspace planning, and the composition of one
// layer's launches.  All compute is in kvr_kernels.hip.
#include "kvrecall.h"

#include "kvr_device.hpp"
#include "kvr_internal.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

struct kvr_context {
    int device = 0;
    hipStream_t sel = nullptr, copy = nullptr;
    hipEvent_t ev_sel = nullptr;   // select work done -> copy stream may read the selection
    uint32_t *status = nullptr;    // dev [kStatusWords]
    uint32_t *counters = nullptr;  // dev [counters_cap], zero between launches
    uint32_t counters_cap = 0;
    uint32_t epoch = 0;
    uint8_t *ws = nullptr;
    size_t ws_bytes = 0;
    bool ws_borrowed = false;
    // batched device copies: a ring of op tables, each reused only after the
    // copy launch that read it has run (its event)
    static constexpr int kOpSlots = 4;
    struct OpSlot {
        kvr::CopyOp *dev = nullptr, *pin = nullptr;
        uint32_t cap = 0;
        hipEvent_t done = nullptr;
    } ops[kOpSlots];
    uint32_t ops_next = 0;
    // host fixed-page lists longer than the inline capacity: one upload per
    // call, reused once the previous call's readers have run (fixed_ev)
    uint32_t *fixed_dev = nullptr, *fixed_pin = nullptr;
    size_t fixed_cap = 0;
    hipEvent_t fixed_ev = nullptr;
    // the stream of the last call that used the workspace or the counters
    hipStream_t ws_stream = nullptr;
    hipEvent_t ws_ev = nullptr;
    // SDMA stage-in: span copies fan out over kDmaStreams streams (each can
    // drive its own DMA engine) and join back into the copy stream.
    hipStream_t dma[4] = {};
    hipEvent_t dma_fork = nullptr, dma_join[4] = {};
    hipStream_t readback = nullptr;  // selection readback, ordered only on the select event
    uint32_t *sel_pin = nullptr;
    size_t sel_pin_cap = 0;
    uint8_t *staging = nullptr;
    size_t staging_bytes = 0;
    // tuning
    uint32_t gather_wgs = 0;  // 0: by mode (kDefaultGatherWgs / kDefaultDecodeGatherWgs)
    uint32_t attn_page_group = 0;  // 0: by the call's size
    uint32_t chunk_rows = 8;
    bool chunk_rows_set = false;  // chosen by the caller (else by the planes)
    uint32_t gather_threads = 0;  // 0: by mode
};

namespace {

thread_local std::string g_error;

kvr_status fail(kvr_status s, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
    return s;
}

}  // namespace

namespace kvr {
kvr_status set_error(kvr_status s, const char *message) {
    g_error = message;
    return s;
}
}  // namespace kvr

namespace {

kvr_status hip_fail(hipError_t e, const char *what) {
    return fail(KVR_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

#define KVR_HIP(expr)                                              \
    do {                                                           \
        const hipError_t e_ = (expr);                              \
        if (e_ != hipSuccess) return hip_fail(e_, #expr);          \
    } while (0)

struct DeviceGuard {
    int previous = -1;
    explicit DeviceGuard(int device) {
        if (hipGetDevice(&previous) != hipSuccess) previous = -1;
        if (previous != device) (void)hipSetDevice(device);
    }
    ~DeviceGuard() {
        int now = -1;
        if (previous >= 0 && hipGetDevice(&now) == hipSuccess && now != previous) (void)hipSetDevice(previous);
    }
};

size_t align256(size_t b) { return (b + 255) & ~size_t(255); }
constexpr size_t kGatherLds = 65536;  // dynamic LDS bound of one gather workgroup
constexpr int kDmaStreams = 4;
bool aligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }
bool pow2(uint32_t v) { return v && !(v & (v - 1)); }

size_t row_bytes(kvr_format f, uint32_t width) {
    switch (f) {
    case KVR_FMT_F16: return size_t(width) * 2;
    case KVR_FMT_Q8_0: return width % 32 ? 0 : size_t(width) / 32 * 34;
    case KVR_FMT_Q4_1: return width % 32 ? 0 : size_t(width) / 32 * 20;
    case KVR_FMT_Q4_0: return width % 32 ? 0 : size_t(width) / 32 * 18;
    default: return 0;
    }
}

size_t scalar_bytes(kvr_format f) {
    return f == KVR_FMT_F32 ? 4 : (f == KVR_FMT_F16 || f == KVR_FMT_BF16) ? 2 : 0;
}

hipStream_t stream_or(void *s, hipStream_t fallback) {
    return s ? static_cast<hipStream_t>(s) : fallback;
}

// True while `s` records into a graph: such calls may not allocate or wait.
bool capturing(hipStream_t s) {
    hipStreamCaptureStatus c = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(s, &c) == hipSuccess && c != hipStreamCaptureStatusNone;
}

double logit_scale(float attention_scale, uint32_t dim) {
    return attention_scale > 0 ? double(attention_scale) : 1 / std::sqrt(double(dim));
}

uint32_t page_count(uint64_t tokens, uint32_t page_tokens) {
    return uint32_t((tokens + page_tokens - 1) / page_tokens);
}

kvr_status check_ctx(kvr_context *ctx) {
    if (!ctx) return fail(KVR_ERR_INVALID, "null context");
    return KVR_OK;
}

// Query geometry.  Element strides must address disjoint elements of the
// declared scalar (native_layer_query.hpp:36-57 qualifies the same layouts).
kvr_status check_query(const kvr_query *q, uint32_t lanes) {
    if (!q || !q->data) return fail(KVR_ERR_INVALID, "missing query");
    const size_t el = scalar_bytes(q->scalar);
    if (!el) return fail(KVR_ERR_INVALID, "query scalar must be f32, f16 or bf16");
    if (!q->rows || !q->query_heads || !q->kv_heads || !q->head_dim || q->query_heads % q->kv_heads)
        return fail(KVR_ERR_INVALID, "invalid query geometry (rows %u, heads %u/%u, dim %u)", q->rows,
                    q->query_heads, q->kv_heads, q->head_dim);
    if (!std::isfinite(q->attention_scale) || q->attention_scale < 0)
        return fail(KVR_ERR_INVALID, "attention scale must be finite and nonnegative");
    if (!aligned(q->data, el) || q->row_stride % el || q->head_stride % el || q->dim_stride % el ||
        q->lane_stride % el || !q->dim_stride || (q->query_heads > 1 && !q->head_stride) ||
        (q->rows > 1 && !q->row_stride) || (lanes > 1 && !q->lane_stride))
        return fail(KVR_ERR_INVALID, "query strides must be nonzero multiples of the scalar size");
    return KVR_OK;
}

kvr::QueryArgs query_args(const kvr_query *q) {
    kvr::QueryArgs a{};
    a.data = static_cast<const uint8_t *>(q->data);
    a.scalar = uint32_t(q->scalar);
    a.rows = q->rows;
    a.qheads = q->query_heads;
    a.kvheads = q->kv_heads;
    a.dim = q->head_dim;
    a.row_stride = q->row_stride;
    a.head_stride = q->head_stride;
    a.dim_stride = q->dim_stride;
    a.lane_stride = q->lane_stride;
    a.scale = logit_scale(q->attention_scale, q->head_dim);
    const uint64_t esz = a.scalar == kvr::kScalarF32 ? 4 : 2;
    a.dense = a.dim_stride == esz && a.head_stride == esz * a.dim && a.row_stride == esz * a.dim * a.qheads;
    a.packed16 = a.dense && a.scalar == kvr::kScalarF16 && reinterpret_cast<uintptr_t>(a.data) % 16 == 0 &&
                 a.lane_stride % 16 == 0 && (uint64_t(a.rows) * a.qheads * a.dim) % 8 == 0;
    return a;
}

bool valu_dim_ok(uint32_t dim) { return dim % 8 == 0 && pow2(dim / 8) && dim / 8 <= 64; }

// Fused scoring stages the fp16 query rows in LDS when they fit 32 KiB.
uint32_t stage_query(const kvr::QueryArgs &q) {
    return uint64_t(q.rows) * q.qheads * q.dim * 2 <= 32768 ? 1u : 0u;
}

kvr_status ensure_workspace(kvr_context *ctx, size_t bytes, hipStream_t s) {
    if (bytes <= ctx->ws_bytes) return KVR_OK;
    if (ctx->ws_borrowed)
        return fail(KVR_ERR_WORKSPACE, "call needs %zu workspace bytes, borrowed workspace has %zu", bytes,
                    ctx->ws_bytes);
    if (capturing(s))
        return fail(KVR_ERR_WORKSPACE, "call needs %zu workspace bytes (have %zu) while its stream is captured; "
                                       "run it once before capture or bind a workspace", bytes, ctx->ws_bytes);
    KVR_HIP(hipStreamSynchronize(ctx->sel));
    KVR_HIP(hipStreamSynchronize(ctx->copy));
    if (ctx->ws) KVR_HIP(hipFree(ctx->ws));
    ctx->ws = nullptr;
    ctx->ws_bytes = 0;
    KVR_HIP(hipMalloc(&ctx->ws, bytes));
    ctx->ws_bytes = bytes;
    return KVR_OK;
}

constexpr uint32_t kInitialCounters = 64;

// Per-lane completion counters of the softmax launch (zero between launches).
kvr_status ensure_counters(kvr_context *ctx, uint32_t lanes, hipStream_t s) {
    if (lanes <= ctx->counters_cap) return KVR_OK;
    if (capturing(s))
        return fail(KVR_ERR_WORKSPACE, "%u lanes need new counters while the stream is captured; "
                                       "run the shape once before capture", lanes);
    KVR_HIP(hipStreamSynchronize(ctx->sel));
    KVR_HIP(hipStreamSynchronize(ctx->copy));
    if (ctx->counters) KVR_HIP(hipFree(ctx->counters));
    ctx->counters = nullptr;
    ctx->counters_cap = 0;
    const uint32_t cap = std::max<uint32_t>(lanes, kInitialCounters);
    KVR_HIP(hipMalloc(&ctx->counters, cap * sizeof(uint32_t)));
    KVR_HIP(hipMemset(ctx->counters, 0, cap * sizeof(uint32_t)));
    KVR_HIP(hipDeviceSynchronize());
    ctx->counters_cap = cap;
    return KVR_OK;
}

// the logits, then two statistics per softmax row (long Mean rows)
size_t logits_only_bytes(uint32_t lanes, uint32_t pages, uint32_t rows, uint32_t qheads) {
    return align256(size_t(lanes) * rows * qheads * pages * sizeof(double));
}
size_t logits_bytes(uint32_t lanes, uint32_t pages, uint32_t rows, uint32_t qheads) {
    return logits_only_bytes(lanes, pages, rows, qheads) + align256(size_t(lanes) * rows * qheads * 2 * sizeof(double));
}
size_t qpack_bytes(uint32_t lanes, uint32_t rows, uint32_t qheads, uint32_t dim) {
    return align256(size_t(lanes) * rows * qheads * dim * sizeof(uint16_t));
}

static_assert(kvr::kMaxMandatory == KVR_MAX_INLINE_MANDATORY, "inline mandatory capacity");
static_assert(kvr::kStackGroup == KVR_STACK_GROUP, "layers per stack launch");
static_assert(kvr::kScratchBytes == KVR_NOALLOC_SCRATCH_BYTES, "static scratch size");
static_assert(kvr::kScratchCounters == KVR_NOALLOC_MAX_LANES, "static scratch counters");

// A call's host mandatory pages: distinct, ascending.  Up to
// KVR_MAX_INLINE_MANDATORY travel in the launch's arguments; a longer list
// is uploaded (stage_fixed) and the launch reads it from `dev`.
struct Mandatory {
    uint32_t n = 0;
    uint32_t ids[KVR_MAX_INLINE_MANDATORY];
    std::vector<uint32_t> more;
    const uint32_t *dev = nullptr;
};

kvr_status check_mandatory(const uint32_t *ids, uint32_t n, uint32_t pages, uint32_t k, Mandatory &m) {
    if (n && !ids) return fail(KVR_ERR_INVALID, "missing mandatory list");
    std::vector<uint32_t> v(ids, ids + n);
    for (uint32_t id : v)
        if (id >= pages) return fail(KVR_ERR_INVALID, "mandatory page %u is outside %u pages", id, pages);
    std::sort(v.begin(), v.end());
    v.erase(std::unique(v.begin(), v.end()), v.end());
    if (v.size() > k)
        return fail(KVR_ERR_BUDGET, "%zu mandatory pages exceed the selection budget %u", v.size(), k);
    if (v.size() > KVR_MAX_INLINE_MANDATORY && pages > kvr::kFixedBitmapPages)
        return fail(KVR_ERR_UNSUPPORTED, "more than %d mandatory pages need at most %u pages per lane",
                    KVR_MAX_INLINE_MANDATORY, kvr::kFixedBitmapPages);
    m.n = uint32_t(v.size());
    m.more.clear();
    m.dev = nullptr;
    if (v.size() <= KVR_MAX_INLINE_MANDATORY) std::copy(v.begin(), v.end(), m.ids);
    else m.more = std::move(v);
    return KVR_OK;
}

// Uploads the long mandatory lists of one call in one copy on `s`.  The
// pinned and device buffers are reused only after the previous call that
// uploaded has run its readers (fixed_ev, recorded by fixed_done).  A
// captured stream cannot take the upload: such callers pass a device list
// (kvr_page_policy.fixed).
kvr_status stage_fixed(kvr_context *ctx, Mandatory *const *lists, uint32_t n, hipStream_t s, bool &staged) {
    staged = false;
    size_t total = 0;
    for (uint32_t i = 0; i < n; ++i) total += lists[i]->more.size();
    if (!total) return KVR_OK;
    if (capturing(s))
        return fail(KVR_ERR_INVALID, "more than %d host mandatory pages are uploaded by the call and cannot be "
                                     "captured; pass them as a device list (kvr_page_policy.fixed)",
                    KVR_MAX_INLINE_MANDATORY);
    KVR_HIP(hipEventSynchronize(ctx->fixed_ev));
    if (total > ctx->fixed_cap) {
        if (ctx->fixed_dev) KVR_HIP(hipFree(ctx->fixed_dev));
        if (ctx->fixed_pin) KVR_HIP(hipHostFree(ctx->fixed_pin));
        ctx->fixed_dev = ctx->fixed_pin = nullptr;
        ctx->fixed_cap = 0;
        KVR_HIP(hipMalloc(&ctx->fixed_dev, total * sizeof(uint32_t)));
        KVR_HIP(hipHostMalloc(reinterpret_cast<void **>(&ctx->fixed_pin), total * sizeof(uint32_t),
                              hipHostMallocDefault));
        ctx->fixed_cap = total;
    }
    size_t at = 0;
    for (uint32_t i = 0; i < n; ++i) {
        Mandatory &m = *lists[i];
        if (m.more.empty()) continue;
        std::copy(m.more.begin(), m.more.end(), ctx->fixed_pin + at);
        m.dev = ctx->fixed_dev + at;
        at += m.more.size();
    }
    KVR_HIP(hipMemcpyAsync(ctx->fixed_dev, ctx->fixed_pin, total * sizeof(uint32_t), hipMemcpyHostToDevice, s));
    staged = true;
    return KVR_OK;
}

// After the last launch that reads the uploaded lists.
kvr_status fixed_done(kvr_context *ctx, bool staged, hipStream_t s) {
    if (staged) KVR_HIP(hipEventRecord(ctx->fixed_ev, s));
    return KVR_OK;
}

void put_mandatory(const Mandatory &m, kvr::SelectArgs &sa) {
    sa.n_mandatory = 0;
    sa.fixed = nullptr;
    sa.n_fixed = 0;
    if (m.more.empty()) {
        sa.n_mandatory = m.n;
        std::copy(m.ids, m.ids + m.n, sa.mandatory);
    } else {
        sa.fixed = m.dev;
        sa.n_fixed = m.n;
    }
}

// Calls that use the context's workspace or counters are ordered on the
// device: a call on another stream than the previous such call first waits
// for what that stream has queued (an event recorded now), so two streams
// never share the buffers at once.  Captured streams are left to the
// caller's own ordering.
kvr_status ws_order(kvr_context *ctx, hipStream_t s) {
    const hipStream_t prev = ctx->ws_stream;
    ctx->ws_stream = s;
    if (!prev || prev == s || capturing(s) || capturing(prev)) return KVR_OK;
    KVR_HIP(hipEventRecord(ctx->ws_ev, prev));
    KVR_HIP(hipStreamWaitEvent(s, ctx->ws_ev, 0));
    return KVR_OK;
}

// A device-side page policy, checked on the host (its lists are read on the
// device when the selection runs).
struct Policy {
    const kvr_page_policy *p = nullptr;
    bool grouped = false;  // media groups or preferred pages: k_select_groups
};

kvr_status check_policy(const kvr_page_policy *p, uint32_t lanes, uint32_t pages, uint32_t k, Policy &out) {
    out = Policy{};
    if (!p) return KVR_OK;
    if ((p->n_fixed && !p->fixed) || (p->n_groups && !p->groups))
        return fail(KVR_ERR_INVALID, "page policy lists missing");
    if (p->preferred && (!p->preferred_count || !p->preferred_stride))
        return fail(KVR_ERR_INVALID, "preferred pages need their counts and a nonzero stride");
    if (p->n_groups > pages) return fail(KVR_ERR_INVALID, "%u media groups for %u pages", p->n_groups, pages);
    out.p = p;
    out.grouped = p->n_groups || p->preferred;
    if (out.grouped && pages > kvr::kGroupSelectPages)
        return fail(KVR_ERR_UNSUPPORTED, "media groups and preferred pages need at most %u pages per lane (got %u)",
                    kvr::kGroupSelectPages, pages);
    if (p->n_fixed && pages > kvr::kFixedBitmapPages)
        return fail(KVR_ERR_UNSUPPORTED, "fixed pages need at most %u pages per lane", kvr::kFixedBitmapPages);
    (void)lanes;
    (void)k;
    return KVR_OK;
}

// A selection with the policy's lists.  The host mandatory pages (m) and the
// policy's fixed list are both read (a device list replaces the inline
// one only when the host list is empty).
kvr_status put_policy(const Policy &pol, const Mandatory &m, kvr::SelectArgs &sa) {
    put_mandatory(m, sa);
    if (!pol.p) return KVR_OK;
    const kvr_page_policy &p = *pol.p;
    if (p.n_fixed) {
        if (sa.fixed) return fail(KVR_ERR_INVALID, "a host mandatory list longer than %d and a device fixed list "
                                                   "cannot be combined", KVR_MAX_INLINE_MANDATORY);
        sa.fixed = p.fixed;
        sa.n_fixed = p.n_fixed;
    }
    sa.groups = p.groups;
    sa.n_groups = p.n_groups;
    sa.preferred = p.preferred;
    sa.preferred_count = p.preferred_count;
    sa.preferred_stride = p.preferred_stride;
    return KVR_OK;
}

struct ScorePlan {
    kvr::QueryArgs q;
    uint32_t lanes, pages, rows, qheads, kvheads, dim;
    bool mfma;
    double *logits;
    uint16_t *qpack;
    uint32_t *counters;  // per-lane completion counters of the softmax launch
    uint32_t fold;       // kvr::Fold: the columns are half pages folded in pairs
};

// Where a call's logits, packed queries and counters live: the context's
// workspace (grown on demand) unless `fixed` names the static scratch.
struct FixedScratch {
    uint8_t *base;      // device address of the scratch array
    size_t bytes;       // its size
};

kvr_status plan_score(kvr_context *ctx, const kvr_query *q, uint32_t lanes, uint32_t pages,
                      int force_mfma, hipStream_t stream, ScorePlan &p, const FixedScratch *fixed = nullptr) {
    if (kvr_status s = check_query(q, lanes)) return s;
    if (!pages) return fail(KVR_ERR_INVALID, "no pages to score");
    p.fold = kvr::kFoldNone;
    p.q = query_args(q);
    p.lanes = lanes;
    p.pages = pages;
    p.rows = q->rows;
    p.qheads = q->query_heads;
    p.kvheads = q->kv_heads;
    p.dim = q->head_dim;
    const uint32_t group = q->query_heads / q->kv_heads;
    p.mfma = force_mfma > 0 || (force_mfma == 0 && uint64_t(q->rows) * group >= 16);
    if (p.mfma && q->head_dim % 4)
        return fail(KVR_ERR_INVALID, "matrix-core scoring needs head_dim %% 4 == 0");
    if (!p.mfma && !valu_dim_ok(q->head_dim))
        return fail(KVR_ERR_INVALID, "head_dim %u: vector scoring needs 8*2^i <= 512", q->head_dim);
    const size_t lb = logits_bytes(lanes, pages, q->rows, q->query_heads);
    const size_t qb = p.mfma ? qpack_bytes(lanes, q->rows, q->query_heads, q->head_dim) : 0;
    if (fixed) {
        // counters first, then logits and packed queries; nothing grows
        if (lanes > kvr::kScratchCounters || kvr::kScratchCounterBytes + lb + qb > fixed->bytes)
            return fail(KVR_ERR_WORKSPACE, "call needs %u counters and %zu bytes of logits and queries; the static "
                                           "scratch holds %u counters and %zu bytes", lanes, lb + qb,
                        kvr::kScratchCounters, fixed->bytes - kvr::kScratchCounterBytes);
        p.counters = reinterpret_cast<uint32_t *>(fixed->base);
        p.logits = reinterpret_cast<double *>(fixed->base + kvr::kScratchCounterBytes);
        p.qpack = reinterpret_cast<uint16_t *>(fixed->base + kvr::kScratchCounterBytes + lb);
        return KVR_OK;
    }
    if (kvr_status s = ensure_workspace(ctx, lb + qb, stream)) return s;
    p.logits = reinterpret_cast<double *>(ctx->ws);
    p.qpack = reinterpret_cast<uint16_t *>(ctx->ws + lb);
    p.counters = nullptr;  // the context's, sized at launch
    return KVR_OK;
}

// logits -> softmax -> aggregation (+ selection).
kvr::SelectArgs make_select_args(kvr_context *ctx, const ScorePlan &p, const uint8_t *mask, kvr_aggregation agg,
                                 uint32_t active_layers, int accumulate, double *scores, bool do_select, uint32_t k,
                                 kvr_tie_rule tie, const Mandatory &mand, uint32_t *selected, uint32_t *count) {
    kvr::SelectArgs sa{};
    sa.logits = p.logits;
    sa.stats = reinterpret_cast<double *>(reinterpret_cast<uint8_t *>(p.logits) +
                                          logits_only_bytes(p.lanes, p.pages, p.rows, p.qheads));
    sa.mask = mask;
    sa.units = p.rows * (agg == KVR_AGG_MEAN ? p.qheads : p.kvheads);
    sa.counters = p.counters ? p.counters : ctx->counters;
    sa.fold = p.fold;
    sa.mask_shift = p.fold ? 1 : 0;
    sa.rows = p.rows;
    sa.qheads = p.qheads;
    sa.kvheads = p.kvheads;
    sa.aggregation = uint32_t(agg);
    sa.weight = double(active_layers) * (agg == KVR_AGG_MEAN ? p.qheads : p.kvheads);
    sa.accumulate = accumulate;
    sa.do_aggregate = 1;
    sa.scores = scores;
    sa.lanes = p.lanes;
    sa.pages = p.pages;
    sa.k = k;
    sa.tie_higher_first = tie == KVR_TIE_HIGHER_FIRST;
    sa.signed_scores = 0;
    sa.do_select = do_select;
    put_mandatory(mand, sa);
    sa.selected = selected;
    sa.count = count;
    sa.status = ctx->status;
    sa.epoch = ctx->epoch;
    return sa;
}

kvr_status enqueue_probs_and_select(kvr_context *ctx, const ScorePlan &p, const uint8_t *mask,
                                    kvr_aggregation agg, uint32_t active_layers, int accumulate,
                                    double *scores, bool do_select, uint32_t k, kvr_tie_rule tie,
                                    const Mandatory &mand, uint32_t *selected, uint32_t *count,
                                    hipStream_t s, const Policy *pol = nullptr) {
    if (p.lanes > 65535) return fail(KVR_ERR_INVALID, "at most 65535 lanes per call");
    if (!p.counters)
        if (kvr_status st = ensure_counters(ctx, p.lanes, s)) return st;
    kvr::SelectArgs sa = make_select_args(ctx, p, mask, agg, active_layers, accumulate, scores, do_select, k, tie,
                                          mand, selected, count);
    if (pol)
        if (kvr_status st = put_policy(*pol, mand, sa)) return st;
    if (do_select && pol && pol->grouped) {
        // media groups / preferred pages: the selection is its own launch,
        // over the (folded) page scores
        sa.do_select = 0;
        KVR_HIP(kvr::launch_probs(sa, s));
        sa.do_select = 1;
        sa.pages = kvr::select_pages(sa);
        sa.fold = kvr::kFoldNone;
        sa.mask_shift = 0;
        KVR_HIP(kvr::launch_select_groups(sa, s));
        return KVR_OK;
    }
    KVR_HIP(kvr::launch_probs(sa, s));
    return KVR_OK;
}

// Resident fp16 summaries as the source of the fused logits (no mean-K).
kvr::SummaryArgs resident_args(kvr_context *ctx, const ScorePlan &p, const uint16_t *summaries) {
    kvr::SummaryArgs a{};
    a.src = reinterpret_cast<const uint8_t *>(summaries);
    a.src_lane_stride = uint64_t(p.pages) * p.kvheads * p.dim * 2;
    a.pages = p.pages;
    a.width = p.kvheads * p.dim;
    a.lanes = p.lanes;
    a.q = p.q;
    a.q_stage = stage_query(p.q);
    a.logits = p.logits;
    a.status = ctx->status;
    a.epoch = ctx->epoch;
    return a;
}

kvr_status enqueue_logits(kvr_context *ctx, const ScorePlan &p, const uint16_t *summaries,
                          hipStream_t s) {
    if (p.mfma) {
        kvr::PackQueryArgs pq{};
        pq.q = p.q;
        pq.lanes = p.lanes;
        pq.out = p.qpack;
        pq.status = ctx->status;
        pq.epoch = ctx->epoch;
        KVR_HIP(kvr::launch_pack_query(pq, s));
        kvr::MfmaLogitsArgs ma{};
        ma.qpack = p.qpack;
        ma.summaries = summaries;
        ma.lanes = p.lanes;
        ma.pages = p.pages;
        ma.rows = p.rows;
        ma.qheads = p.qheads;
        ma.kvheads = p.kvheads;
        ma.dim = p.dim;
        ma.scale = p.q.scale;
        ma.logits = p.logits;
        KVR_HIP(kvr::launch_logits_mfma(ma, s));
    } else {
        KVR_HIP(kvr::launch_summary(kvr::kSrcSummary, true, resident_args(ctx, p, summaries), s));
    }
    return KVR_OK;
}

kvr_status check_keys(const kvr_key_history *k, uint32_t &pages, size_t &lane_stride) {
    if (!k || !k->data) return fail(KVR_ERR_INVALID, "missing key history");
    if (k->format != KVR_FMT_F16 && k->format != KVR_FMT_Q8_0)
        return fail(KVR_ERR_UNSUPPORTED, "key history must be f16 or q8_0");
    if (!k->tokens || !k->kv_heads || !k->head_dim || !k->page_tokens)
        return fail(KVR_ERR_INVALID, "empty key history geometry");
    const uint32_t width = k->kv_heads * k->head_dim;
    if (width % 8) return fail(KVR_ERR_INVALID, "kv_heads*head_dim must be a multiple of 8");
    if (k->format == KVR_FMT_Q8_0 && width % 64)
        return fail(KVR_ERR_INVALID, "q8_0 keys need kv_heads*head_dim %% 64 == 0");
    const uint64_t p = (k->tokens + k->page_tokens - 1) / k->page_tokens;
    if (p > 0xffffffffull) return fail(KVR_ERR_INVALID, "too many pages");
    pages = uint32_t(p);
    const size_t rb = row_bytes(k->format, width);
    const uint32_t lanes = k->lanes ? k->lanes : 1;
    lane_stride = k->lane_stride ? k->lane_stride : size_t(k->tokens) * rb;
    if (lanes > 1 && lane_stride < size_t(k->tokens) * rb)
        return fail(KVR_ERR_INVALID, "key lane stride overlaps");
    const size_t need = k->format == KVR_FMT_F16 ? 16 : 4;
    if (!aligned(k->data, need) || lane_stride % need)
        return fail(KVR_ERR_INVALID, "key history must be %zu-byte aligned", need);
    return KVR_OK;
}

kvr_status check_summary_out(const float *means, const uint16_t *summaries) {
    if ((means && !aligned(means, 16)) || (summaries && !aligned(summaries, 16)))
        return fail(KVR_ERR_INVALID, "summary outputs must be 16-byte aligned");
    return KVR_OK;
}

kvr::SummaryArgs summary_args(kvr_context *ctx, const kvr_key_history *k, uint32_t pages,
                              size_t lane_stride, float *means, uint16_t *summaries) {
    kvr::SummaryArgs a{};
    a.src = static_cast<const uint8_t *>(k->data);
    a.src_lane_stride = lane_stride;
    a.tokens = k->tokens;
    a.page_tokens = k->page_tokens;
    a.pages = pages;
    a.width = k->kv_heads * k->head_dim;
    a.lanes = k->lanes ? k->lanes : 1;
    a.means = means;
    a.summaries = summaries;
    a.status = ctx->status;
    a.epoch = ctx->epoch;
    return a;
}

// ---- stage-in -------------------------------------------------------------

struct PlanePlan {
    kvr::GatherPlane g;
    const uint8_t *host;   // pinned host pointer (SDMA engine)
    size_t host_row;
};

kvr_status check_planes(const kvr_plane *planes, uint32_t n, uint32_t lanes, uint32_t page_tokens,
                        uint32_t k, uint32_t chunk_rows, PlanePlan *out) {
    if (n > KVR_MAX_PLANES) return fail(KVR_ERR_INVALID, "at most %d planes", KVR_MAX_PLANES);
    if (n && !planes) return fail(KVR_ERR_INVALID, "missing planes");
    for (uint32_t i = 0; i < n; ++i) {
        const kvr_plane &p = planes[i];
        if (!p.history || !p.slots || !p.width || !p.tokens)
            return fail(KVR_ERR_INVALID, "plane %u: missing history, slots or geometry", i);
        const size_t srow = row_bytes(p.format, p.width);
        if (!srow) return fail(KVR_ERR_UNSUPPORTED, "plane %u: history format must be f16, q8_0, q4_1 or q4_0 "
                                                    "(width %% 32 == 0 for blocks)", i);
        const bool raw_k = p.mode == KVR_GATHER_ROPE_FWHT;
        size_t drow = 0;
        if (p.mode == KVR_GATHER_COPY) drow = srow;
        else if (p.mode == KVR_GATHER_DEQUANT_F16 && p.format != KVR_FMT_Q4_0) drow = size_t(p.width) * 2;
        else if (p.mode == KVR_GATHER_REQUANT_Q8_0 && p.format == KVR_FMT_Q8_0) drow = srow;
        else if (raw_k && (p.format == KVR_FMT_Q8_0 || p.format == KVR_FMT_Q4_0)) drow = srow;
        if (!drow) return fail(KVR_ERR_UNSUPPORTED, "plane %u: gather mode not provided for this format", i);
        if (raw_k) {
            // kvmem_stagein_enqueue_k / rope_neox / fwht_ok (stagein.cu:477-479, 534-541, 817-831)
            const kvr_rope *r = p.rope;
            if (!r || !r->head_dim || p.width % r->head_dim || r->n_rot % 2 || r->n_rot > r->head_dim ||
                r->n_rot > 512 || (r->n_rot && !r->theta))
                return fail(KVR_ERR_INVALID, "plane %u: raw-K transform needs head_dim dividing the width, an even "
                                             "n_rot <= min(head_dim, 512) and its theta", i);
            if (r->fwht && ((r->fwht != 64 && r->fwht != 128 && r->fwht != 256 && r->fwht != 512) ||
                            p.width % r->fwht))
                return fail(KVR_ERR_INVALID, "plane %u: Walsh-Hadamard size must be 64, 128, 256 or 512 and "
                                             "divide the width", i);
            if (4 * (srow + 16 + size_t(p.width) * 4) > kGatherLds)
                return fail(KVR_ERR_INVALID, "plane %u: rows too wide for the raw-K transform", i);
        }
        if (p.mode == KVR_GATHER_DEQUANT_F16 && p.format != KVR_FMT_F16 && (p.width % 32 || !aligned(p.slots, 16)))
            return fail(KVR_ERR_INVALID, "plane %u: dequantized slots must be 16-byte aligned", i);
        (void)chunk_rows;
        if (p.format != KVR_FMT_F16 && p.mode != KVR_GATHER_COPY && 4 * (srow + 16) > kGatherLds)
            return fail(KVR_ERR_INVALID, "plane %u: rows too wide for the staged decoder", i);
        hipPointerAttribute_t attr{};
        if (hipPointerGetAttributes(&attr, p.history) != hipSuccess || attr.type != hipMemoryTypeHost ||
            !attr.devicePointer) {
            (void)hipGetLastError();
            return fail(KVR_ERR_INVALID, "plane %u: history is not pinned, device-mapped host memory", i);
        }
        const size_t lane_pages = size_t((p.tokens + page_tokens - 1) / page_tokens);
        if (p.page_stride && p.page_stride < size_t(page_tokens) * srow)
            return fail(KVR_ERR_INVALID, "plane %u: a page's rows overlap the next record (page_stride)", i);
        const size_t src_bytes = p.page_stride ? lane_pages * p.page_stride : size_t(p.tokens) * srow;
        const size_t hls = p.host_lane_stride ? p.host_lane_stride : src_bytes;
        const size_t sls = p.slot_lane_stride ? p.slot_lane_stride : size_t(k) * page_tokens * drow;
        if (lanes > 1 && (hls < src_bytes || sls < size_t(k) * page_tokens * drow))
            return fail(KVR_ERR_INVALID, "plane %u: lane strides overlap", i);
        PlanePlan &pp = out[i];
        pp.g = kvr::GatherPlane{};
        pp.g.src = static_cast<const uint8_t *>(attr.devicePointer);
        pp.g.dst = static_cast<uint8_t *>(p.slots);
        pp.g.src_lane_stride = hls;
        pp.g.dst_lane_stride = sls;
        pp.g.page_stride = p.page_stride;
        pp.g.tokens = p.tokens;
        pp.g.src_row = uint32_t(srow);
        pp.g.dst_row = uint32_t(drow);
        pp.g.width = p.width;
        pp.g.format = uint32_t(p.format);
        pp.g.mode = uint32_t(p.mode);
        if (raw_k) {
            pp.g.theta = p.rope->theta;
            pp.g.head_dim = p.rope->head_dim;
            pp.g.n_rot = p.rope->n_rot;
            pp.g.fwht = p.rope->fwht;
            pp.g.fwht_scale = p.rope->fwht ? 1.0f / std::sqrt(float(p.rope->fwht)) : 1.0f;
            pp.g.pos_base = p.rope->pos_base;
        }
        pp.host = static_cast<const uint8_t *>(p.history);
        pp.host_row = srow;
    }
    return KVR_OK;
}

// Copies fill the host link with one wave on each of 16 CUs (so they take
// little from the summary kernel beside them); decoding planes need more
// waves to hide their ALU work behind the link.
constexpr uint32_t kDefaultGatherWgs = 16, kDefaultGatherThreads = 64;               // copies
constexpr uint32_t kDefaultDecodeGatherWgs = 32, kDefaultDecodeGatherThreads = 256;  // decoding planes
constexpr uint32_t kDefaultChunkRows = 8;
// The raw-K transform is a chain of dependent LDS phases per row: one row
// per work item and a grid of 1024 workgroups keep many waves per SIMD to
// hide them (8 rows per item and 32 workgroups left one wave per SIMD).
constexpr uint32_t kRawKChunkRows = 1, kRawKGatherWgs = 1024;
bool has_raw_k(const PlanePlan *pp, uint32_t n) {
    for (uint32_t i = 0; i < n; ++i)
        if (pp[i].g.mode == KVR_GATHER_ROPE_FWHT) return true;
    return false;
}

// Rows per gather work item: the context's setting, bounded by the page and
// by the LDS a staged decode needs (source rows + requantized rows).
// Rows per gather item: the option, bounded so that every wave's LDS slice
// of a decoding plane fits the workgroup's LDS.
uint32_t gather_chunk_rows(uint32_t chunk_rows, uint32_t threads, const PlanePlan *pp, uint32_t n,
                           uint32_t page_tokens) {
    uint32_t cr = std::min(chunk_rows, page_tokens);
    const size_t waves = threads / 64;
    for (uint32_t i = 0; i < n; ++i) {
        if (pp[i].g.mode == KVR_GATHER_COPY || pp[i].g.format == KVR_FMT_F16) continue;
        // the raw-K transform also keeps one binary32 row per wave
        const size_t fixed = pp[i].g.mode == KVR_GATHER_ROPE_FWHT ? size_t(pp[i].g.width) * 4 : 0;
        cr = std::min<uint32_t>(cr, uint32_t((kGatherLds / waves - fixed) / (size_t(pp[i].g.src_row) + 16)));
    }
    return std::max<uint32_t>(cr, 1);
}

kvr_status enqueue_gather_kernel(kvr_context *ctx, const PlanePlan *pp, uint32_t n, uint32_t lanes,
                                 uint32_t page_tokens, const uint32_t *selected, const uint32_t *count,
                                 uint32_t k, hipStream_t s) {
    if (!n) return KVR_OK;
    kvr::GatherArgs ga{};
    for (uint32_t i = 0; i < n; ++i) ga.plane[i] = pp[i].g;
    ga.n_planes = n;
    ga.lanes = lanes;
    ga.k = k;
    ga.page_tokens = page_tokens;
    const bool raw_k = has_raw_k(pp, n);
    ga.chunk_rows = gather_chunk_rows(ctx->chunk_rows_set || !raw_k ? ctx->chunk_rows : kRawKChunkRows, 256, pp, n,
                                      page_tokens);
    ga.chunks = (page_tokens + ga.chunk_rows - 1) / ga.chunk_rows;
    ga.selected = selected;
    ga.count = count;
    bool decode = false;
    for (uint32_t i = 0; i < n; ++i)
        decode = decode || (pp[i].g.mode != KVR_GATHER_COPY && pp[i].g.format != KVR_FMT_F16);
    ga.workgroups = ctx->gather_wgs ? ctx->gather_wgs
                    : raw_k         ? kRawKGatherWgs
                    : decode        ? kDefaultDecodeGatherWgs
                                    : kDefaultGatherWgs;
    ga.threads = ctx->gather_threads ? ctx->gather_threads : decode ? kDefaultDecodeGatherThreads
                                                                     : kDefaultGatherThreads;
    KVR_HIP(kvr::launch_gather(ga, s));
    return KVR_OK;
}

// DMA engine: wait for the selection, then hipMemcpyAsync per run of
// consecutive selected pages (contiguous in the history and in the slots),
// spread round-robin over kDmaStreams streams that join back into `s`.
// Copy modes land in the slots; decoding modes land in a device staging area
// that the gather kernel then decodes HBM -> HBM.  No CU reads host memory.
// `sel_ready`, when given, is the event after which the selection is valid:
// the readback then waits on it alone (not on earlier copies queued on s).
kvr_status enqueue_gather_sdma(kvr_context *ctx, PlanePlan *pp, uint32_t n, uint32_t lanes,
                               uint32_t page_tokens, const uint32_t *selected, const uint32_t *count,
                               uint32_t k, hipStream_t s, hipEvent_t sel_ready = nullptr) {
    if (!n) return KVR_OK;
    if (capturing(s))
        return fail(KVR_ERR_INVALID, "the DMA stage-in engine reads the selection on the host and cannot be "
                                     "captured; use the kernel engine inside graphs");
    const size_t words = size_t(lanes) * (k + 1);
    if (ctx->sel_pin_cap < words) {
        if (ctx->sel_pin) KVR_HIP(hipHostFree(ctx->sel_pin));
        ctx->sel_pin = nullptr;
        ctx->sel_pin_cap = 0;
        KVR_HIP(hipHostMalloc(reinterpret_cast<void **>(&ctx->sel_pin), words * 4, hipHostMallocDefault));
        ctx->sel_pin_cap = words;
    }
    const hipStream_t rb = sel_ready ? ctx->readback : s;
    if (sel_ready) KVR_HIP(hipStreamWaitEvent(rb, sel_ready, 0));
    KVR_HIP(hipMemcpyAsync(ctx->sel_pin, selected, size_t(lanes) * k * 4, hipMemcpyDeviceToHost, rb));
    KVR_HIP(hipMemcpyAsync(ctx->sel_pin + size_t(lanes) * k, count, size_t(lanes) * 4, hipMemcpyDeviceToHost, rb));
    KVR_HIP(hipStreamSynchronize(rb));
    size_t staged = 0;
    for (uint32_t i = 0; i < n; ++i)
        if (pp[i].g.mode != KVR_GATHER_COPY && pp[i].g.format != KVR_FMT_F16)
            staged += size_t(lanes) * k * page_tokens * pp[i].host_row;
    if (staged > ctx->staging_bytes) {
        if (ctx->ws_borrowed) return fail(KVR_ERR_WORKSPACE, "DMA staging needs %zu bytes", staged);
        if (ctx->staging) KVR_HIP(hipFree(ctx->staging));
        ctx->staging = nullptr;
        ctx->staging_bytes = 0;
        KVR_HIP(hipMalloc(&ctx->staging, staged));
        ctx->staging_bytes = staged;
    }
    KVR_HIP(hipEventRecord(ctx->dma_fork, s));
    for (int d = 0; d < kDmaStreams; ++d) KVR_HIP(hipStreamWaitEvent(ctx->dma[d], ctx->dma_fork, 0));
    uint32_t rr = 0;
    size_t at = 0;
    for (uint32_t i = 0; i < n; ++i) {
        PlanePlan &p = pp[i];
        const bool decode = p.g.mode != KVR_GATHER_COPY && p.g.format != KVR_FMT_F16;
        const size_t span = size_t(page_tokens) * p.host_row;
        for (uint32_t lane = 0; lane < lanes; ++lane) {
            const uint32_t cnt = std::min(ctx->sel_pin[size_t(lanes) * k + lane], k);
            const uint32_t *ids = ctx->sel_pin + size_t(lane) * k;
            for (uint32_t slot = 0; slot < cnt;) {
                const uint32_t page = ids[slot];
                const uint64_t first = uint64_t(page) * page_tokens;
                if (first >= p.g.tokens) { ++slot; continue; }
                // extend over consecutive pages that are full (token-major
                // sources only: records put other planes between pages)
                uint32_t run = 1;
                while (!p.g.page_stride && slot + run < cnt && ids[slot + run] == page + run &&
                       uint64_t(page + run) * page_tokens < p.g.tokens &&
                       uint64_t(page + run) * page_tokens <= p.g.tokens - page_tokens)
                    ++run;
                const uint64_t rows = std::min<uint64_t>(uint64_t(run) * page_tokens, p.g.tokens - first);
                const uint8_t *src = p.host + lane * p.g.src_lane_stride +
                                     (p.g.page_stride ? uint64_t(page) * p.g.page_stride : first * p.host_row);
                uint8_t *dst = decode ? ctx->staging + at + (size_t(lane) * k + slot) * span
                                      : p.g.dst + lane * p.g.dst_lane_stride + size_t(slot) * page_tokens * p.g.dst_row;
                KVR_HIP(hipMemcpyAsync(dst, src, rows * p.host_row, hipMemcpyHostToDevice,
                                       ctx->dma[rr++ % kDmaStreams]));
                slot += run;
            }
        }
        if (decode) at += size_t(lanes) * k * span;
    }
    for (int d = 0; d < kDmaStreams; ++d) {
        KVR_HIP(hipEventRecord(ctx->dma_join[d], ctx->dma[d]));
        KVR_HIP(hipStreamWaitEvent(s, ctx->dma_join[d], 0));
    }
    at = 0;
    for (uint32_t i = 0; i < n; ++i) {
        PlanePlan &p = pp[i];
        if (p.g.mode == KVR_GATHER_COPY || p.g.format == KVR_FMT_F16) continue;
        const size_t span = size_t(page_tokens) * p.host_row;
        kvr::GatherArgs ga{};
        ga.plane[0] = p.g;
        ga.plane[0].src = ctx->staging + at;
        ga.plane[0].src_lane_stride = size_t(k) * span;
        ga.n_planes = 1;
        ga.lanes = lanes;
        ga.k = k;
        ga.page_tokens = page_tokens;
        const bool raw_k = p.g.mode == KVR_GATHER_ROPE_FWHT;
        ga.chunk_rows = gather_chunk_rows(ctx->chunk_rows_set || !raw_k ? ctx->chunk_rows : kRawKChunkRows, 256, &p,
                                          1, page_tokens);
        ga.chunks = (page_tokens + ga.chunk_rows - 1) / ga.chunk_rows;
        ga.workgroups = 1024;  // HBM -> HBM: use the whole GPU
        ga.threads = 256;
        ga.selected = selected;  // page ids bound each slot's valid rows
        ga.count = count;
        ga.src_page_stride = span;
        KVR_HIP(kvr::launch_gather(ga, s));
        at += size_t(lanes) * k * span;
    }
    return KVR_OK;
}

}  // namespace

// ===========================================================================
extern "C" {

const char *kvr_last_error(void) { return g_error.c_str(); }

const char *kvr_status_string(kvr_status s) {
    switch (s) {
    case KVR_OK: return "ok";
    case KVR_ERR_INVALID: return "invalid argument";
    case KVR_ERR_NONFINITE: return "nonfinite recall operand";
    case KVR_ERR_RANGE: return "recall operand exceeds fp16 range";
    case KVR_ERR_BUDGET: return "mandatory pages exceed the budget";
    case KVR_ERR_WORKSPACE: return "workspace too small";
    case KVR_ERR_HIP: return "HIP runtime error";
    case KVR_ERR_SCORES: return "invalid score";
    case KVR_ERR_UNSUPPORTED: return "unsupported format or mode";
    case KVR_ERR_GRAPH: return "invalid graph mass, weight or row, or propagation result";
    }
    return "unknown status";
}

kvr_status kvr_create(int device, kvr_context **out) {
    if (!out) return fail(KVR_ERR_INVALID, "null output");
    *out = nullptr;
    int n = 0;
    KVR_HIP(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) return fail(KVR_ERR_INVALID, "device %d of %d", device, n);
    DeviceGuard guard(device);
    auto *ctx = new kvr_context;
    ctx->device = device;
    hipError_t e = hipStreamCreateWithFlags(&ctx->sel, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&ctx->copy, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&ctx->ev_sel, hipEventDisableTiming);
    for (int i = 0; i < kvr_context::kOpSlots && e == hipSuccess; ++i)
        e = hipEventCreateWithFlags(&ctx->ops[i].done, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&ctx->fixed_ev, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&ctx->ws_ev, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&ctx->dma_fork, hipEventDisableTiming);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&ctx->readback, hipStreamNonBlocking);
    for (int i = 0; i < kDmaStreams && e == hipSuccess; ++i) {
        e = hipStreamCreateWithFlags(&ctx->dma[i], hipStreamNonBlocking);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&ctx->dma_join[i], hipEventDisableTiming);
    }
    if (e == hipSuccess) e = hipMalloc(&ctx->status, kvr::kStatusWords * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMemset(ctx->status, 0, kvr::kStatusWords * sizeof(uint32_t));
    // select counters for up to 64 lanes, so calls on a borrowed workspace
    // never allocate
    if (e == hipSuccess) e = hipMalloc(&ctx->counters, kInitialCounters * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMemset(ctx->counters, 0, kInitialCounters * sizeof(uint32_t));
    if (e == hipSuccess) ctx->counters_cap = kInitialCounters;
    // this device's address of the no-allocation entry's static scratch
    if (e == hipSuccess) e = kvr::scratch_init(device);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        kvr_destroy(ctx);
        return hip_fail(e, "context creation");
    }
    *out = ctx;
    return KVR_OK;
}

kvr_status kvr_destroy(kvr_context *ctx) {
    if (!ctx) return KVR_OK;
    DeviceGuard guard(ctx->device);
    if (ctx->sel) (void)hipStreamSynchronize(ctx->sel);
    if (ctx->copy) (void)hipStreamSynchronize(ctx->copy);
    if (ctx->ws && !ctx->ws_borrowed) (void)hipFree(ctx->ws);
    if (ctx->staging) (void)hipFree(ctx->staging);
    if (ctx->status) (void)hipFree(ctx->status);
    if (ctx->counters) (void)hipFree(ctx->counters);
    for (kvr_context::OpSlot &o : ctx->ops) {
        if (o.done) (void)hipEventSynchronize(o.done);
        if (o.dev) (void)hipFree(o.dev);
        if (o.pin) (void)hipHostFree(o.pin);
        if (o.done) (void)hipEventDestroy(o.done);
    }
    if (ctx->fixed_ev) (void)hipEventSynchronize(ctx->fixed_ev);
    if (ctx->fixed_dev) (void)hipFree(ctx->fixed_dev);
    if (ctx->fixed_pin) (void)hipHostFree(ctx->fixed_pin);
    if (ctx->fixed_ev) (void)hipEventDestroy(ctx->fixed_ev);
    if (ctx->ws_ev) (void)hipEventDestroy(ctx->ws_ev);
    if (ctx->sel_pin) (void)hipHostFree(ctx->sel_pin);
    if (ctx->ev_sel) (void)hipEventDestroy(ctx->ev_sel);
    for (int i = 0; i < kDmaStreams; ++i) {
        if (ctx->dma[i]) (void)hipStreamSynchronize(ctx->dma[i]);
        if (ctx->dma[i]) (void)hipStreamDestroy(ctx->dma[i]);
        if (ctx->dma_join[i]) (void)hipEventDestroy(ctx->dma_join[i]);
    }
    if (ctx->dma_fork) (void)hipEventDestroy(ctx->dma_fork);
    if (ctx->readback) (void)hipStreamSynchronize(ctx->readback);
    if (ctx->readback) (void)hipStreamDestroy(ctx->readback);
    if (ctx->sel) (void)hipStreamDestroy(ctx->sel);
    if (ctx->copy) (void)hipStreamDestroy(ctx->copy);
    delete ctx;
    return KVR_OK;
}

kvr_status kvr_set_option(kvr_context *ctx, kvr_option option, int64_t value) {
    if (kvr_status s = check_ctx(ctx)) return s;
    switch (option) {
    case KVR_OPT_GATHER_WORKGROUPS:
        if (value < 0 || value > 65536) return fail(KVR_ERR_INVALID, "gather workgroups must be in [0, 65536]");
        ctx->gather_wgs = uint32_t(value);
        return KVR_OK;
    case KVR_OPT_GATHER_CHUNK_ROWS:
        if (value < 0 || value > 64) return fail(KVR_ERR_INVALID, "gather chunk rows must be in [0, 64]");
        ctx->chunk_rows = value ? uint32_t(value) : kDefaultChunkRows;
        ctx->chunk_rows_set = value != 0;
        return KVR_OK;
    case KVR_OPT_GATHER_THREADS:
        if (value != 0 && value != 64 && value != 128 && value != 256)
            return fail(KVR_ERR_INVALID, "gather workgroup size must be 64, 128 or 256");
        ctx->gather_threads = uint32_t(value);
        return KVR_OK;
    case KVR_OPT_ATTN_PAGE_GROUP:
        if (value < 0 || value > 16) return fail(KVR_ERR_INVALID, "attention page group must be in [0, 16]");
        ctx->attn_page_group = uint32_t(value);
        return KVR_OK;
    }
    return fail(KVR_ERR_INVALID, "unknown option %d", int(option));
}

void *kvr_select_stream(kvr_context *ctx) { return ctx ? ctx->sel : nullptr; }
void *kvr_copy_stream(kvr_context *ctx) { return ctx ? ctx->copy : nullptr; }

kvr_status kvr_check(kvr_context *ctx, void *stream) {
    if (kvr_status s = check_ctx(ctx)) return s;
    DeviceGuard guard(ctx->device);
    if (stream) {
        KVR_HIP(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
    } else {
        KVR_HIP(hipStreamSynchronize(ctx->sel));
        KVR_HIP(hipStreamSynchronize(ctx->copy));
    }
    uint32_t st[kvr::kStatusWords] = {};
    KVR_HIP(hipMemcpy(st, ctx->status, sizeof st, hipMemcpyDeviceToHost));
    // A raised word holds the number of the call that raised it (graph
    // replays repeat the number their capture gave them); reporting clears it.
    if (!st[kvr::kStatusNonfinite] && !st[kvr::kStatusRange] && !st[kvr::kStatusScores] &&
        !st[kvr::kStatusGraph] && !st[kvr::kStatusBudget])
        return KVR_OK;
    KVR_HIP(hipMemset(ctx->status, 0, sizeof st));
    KVR_HIP(hipDeviceSynchronize());
    if (st[kvr::kStatusNonfinite])
        return fail(KVR_ERR_NONFINITE, "nonfinite recall operand (call %u)", st[kvr::kStatusNonfinite]);
    if (st[kvr::kStatusRange])
        return fail(KVR_ERR_RANGE, "recall operand rounds to fp16 infinity (call %u)", st[kvr::kStatusRange]);
    if (st[kvr::kStatusScores])
        return fail(KVR_ERR_SCORES, "negative or nonfinite score (call %u)", st[kvr::kStatusScores]);
    if (st[kvr::kStatusBudget])
        return fail(KVR_ERR_BUDGET, "fixed pages (with their whole media groups) exceed the selection budget (call %u)",
                    st[kvr::kStatusBudget]);
    return fail(KVR_ERR_GRAPH, "invalid graph mass, weight or row, or propagation result below its residual (call %u)",
                st[kvr::kStatusGraph]);
}

size_t kvr_workspace_bytes(uint32_t lanes, uint32_t max_pages, uint32_t max_rows, uint32_t query_heads,
                           uint32_t kv_heads, uint32_t head_dim) {
    (void)kv_heads;
    lanes = lanes ? lanes : 1;
    return logits_bytes(lanes, max_pages, max_rows, query_heads) +
           qpack_bytes(lanes, max_rows, query_heads, head_dim);
}

kvr_status kvr_bind_workspace(kvr_context *ctx, void *workspace, size_t bytes) {
    if (kvr_status s = check_ctx(ctx)) return s;
    if (!workspace || !aligned(workspace, 256) || !bytes)
        return fail(KVR_ERR_INVALID, "borrowed workspace is missing or not 256-byte aligned");
    DeviceGuard guard(ctx->device);
    KVR_HIP(hipStreamSynchronize(ctx->sel));
    KVR_HIP(hipStreamSynchronize(ctx->copy));
    if (ctx->ws && !ctx->ws_borrowed) KVR_HIP(hipFree(ctx->ws));
    ctx->ws = static_cast<uint8_t *>(workspace);
    ctx->ws_bytes = bytes;
    ctx->ws_borrowed = true;
    return KVR_OK;
}

size_t kvr_device_bytes(kvr_context *ctx) {
    if (!ctx) return 0;
    size_t ops = 0;
    for (const kvr_context::OpSlot &o : ctx->ops) ops += o.cap * sizeof(kvr::CopyOp);
    return ctx->ws_bytes + ctx->staging_bytes + kvr::kStatusWords * 4 + ops + ctx->fixed_cap * sizeof(uint32_t);
}

kvr_status kvr_summary_build(kvr_context *ctx, const kvr_key_history *keys, float *means,
                             uint16_t *summaries, void *stream) {
    if (kvr_status s = check_ctx(ctx)) return s;
    uint32_t pages;
    size_t ls;
    if (kvr_status s = check_keys(keys, pages, ls)) return s;
    if (kvr_status s = check_summary_out(means, summaries)) return s;
    if (!means && !summaries) return fail(KVR_ERR_INVALID, "no summary output");
    DeviceGuard guard(ctx->device);
    ++ctx->epoch;
    const auto a = summary_args(ctx, keys, pages, ls, means, summaries);
    KVR_HIP(kvr::launch_summary(keys->format == KVR_FMT_F16 ? kvr::kSrcKeysF16 : kvr::kSrcKeysQ8, false, a,
                                stream_or(stream, ctx->sel)));
    return KVR_OK;
}


kvr_status kvr_summary_accumulate(kvr_context *ctx, float *sums, uint32_t *counts, uint32_t page_tokens,
                                  const void *k, kvr_format scalar, uint64_t pos0, uint32_t n,
                                  uint32_t kv_heads, uint32_t head_dim, size_t token_stride,
                                  size_t head_stride, size_t dim_stride, void *stream) {
    if (kvr_status s = check_ctx(ctx)) return s;
    const size_t el = scalar_bytes(scalar);
    if (!sums || !counts || !k || !page_tokens || !kv_heads || !head_dim || !el)
        return fail(KVR_ERR_INVALID, "invalid capture geometry or scalar");
    if (!n) return KVR_OK;
    if (!aligned(k, el) || token_stride % el || head_stride % el || dim_stride % el || !dim_stride ||
        (n > 1 && !token_stride) || (kv_heads > 1 && !head_stride))
        return fail(KVR_ERR_INVALID, "capture strides must be nonzero multiples of the scalar size");
    DeviceGuard guard(ctx->device);
    kvr::AccumulateArgs a{};
    a.sums = sums;
    a.counts = counts;
    a.page_tokens = page_tokens;
    a.width = kv_heads * head_dim;
    a.dim = head_dim;
    a.k = static_cast<const uint8_t *>(k);
    a.scalar = uint32_t(scalar);
    a.pos0 = pos0;
    a.n = n;
    a.token_stride = token_stride;
    a.head_stride = head_stride;
    a.dim_stride = dim_stride;
    a.first_page = uint32_t(pos0 / page_tokens);
    a.segments = uint32_t((pos0 + n - 1) / page_tokens) - a.first_page + 1;
    KVR_HIP(kvr::launch_accumulate(a, stream_or(stream, ctx->sel)));
    return KVR_OK;
}

kvr_status kvr_summary_finalize(kvr_context *ctx, const float *sums, const uint32_t *counts, uint32_t pages,
                                uint32_t width, float *means, uint16_t *summaries, void *stream) {
    if (kvr_status s = check_ctx(ctx)) return s;
    if (!sums || !counts || !pages || !width || (!means && !summaries))
        return fail(KVR_ERR_INVALID, "invalid summary finalize arguments");
    DeviceGuard guard(ctx->device);
    ++ctx->epoch;
    kvr::FinalizeArgs a{};
    a.sums = sums;
    a.counts = counts;
    a.pages = pages;
    a.width = width;
    a.means = means;
    a.summaries = summaries;
    a.status = ctx->status;
    a.epoch = ctx->epoch;
    KVR_HIP(kvr::launch_finalize(a, stream_or(stream, ctx->sel)));
    return KVR_OK;
}

kvr_status kvr_score(kvr_context *ctx, const kvr_query *q, const uint16_t *summaries, uint32_t lanes,
                     uint32_t pages, const uint8_t *score_mask, kvr_aggregation aggregation,
                     uint32_t active_layers, int accumulate, double *scores, int force_mfma, void *stream) {
    if (kvr_status s = check_ctx(ctx)) return s;
    lanes = lanes ? lanes : 1;
    if (!summaries || !scores || !aligned(summaries, 16))
        return fail(KVR_ERR_INVALID, "summaries (16-byte aligned) and scores are required");
    if (aggregation > KVR_AGG_MAX_LOGIT) return fail(KVR_ERR_INVALID, "unknown aggregation");
    if (!active_layers) return fail(KVR_ERR_INVALID, "active_layers must be >= 1");
    DeviceGuard guard(ctx->device);
    const hipStream_t s = stream_or(stream, ctx->sel);
    ScorePlan p;
    if (kvr_status st = plan_score(ctx, q, lanes, pages, force_mfma, s, p)) return st;
    if (kvr_status st = ws_order(ctx, s)) return st;
    ++ctx->epoch;
    if (kvr_status st = enqueue_logits(ctx, p, summaries, s)) return st;
    Mandatory none;
    return enqueue_probs_and_select(ctx, p, score_mask, aggregation, active_layers, accumulate, scores, false, 1,
                                    KVR_TIE_LOWER_FIRST, none, nullptr, nullptr, s);
}

namespace {
kvr_status select_common(kvr_context *ctx, const double *scores, uint32_t lanes, uint32_t pages, uint32_t k,
                         const uint32_t *mandatory, uint32_t n_mandatory, const kvr_page_policy *policy,
                         kvr_tie_rule tie_rule, int signed_scores, uint32_t *selected, uint32_t *count,
                         void *stream) {
    if (kvr_status s = check_ctx(ctx)) return s;
    lanes = lanes ? lanes : 1;
    if (!scores || !selected || !count || !pages)
        return fail(KVR_ERR_INVALID, "scores, selected, count and pages are required");
    if (!k) return fail(KVR_ERR_INVALID, "invalid scored selection frame (budget 0)");
    if (tie_rule > KVR_TIE_HIGHER_FIRST) return fail(KVR_ERR_INVALID, "unknown tie rule");
    if (lanes > 65535) return fail(KVR_ERR_INVALID, "at most 65535 lanes per call");
    Mandatory m;
    if (kvr_status s = check_mandatory(mandatory, n_mandatory, pages, k, m)) return s;
    Policy pol;
    if (kvr_status s = check_policy(policy, lanes, pages, k, pol)) return s;
    DeviceGuard guard(ctx->device);
    const hipStream_t st = stream_or(stream, ctx->sel);
    Mandatory *lists[1] = {&m};
    bool staged = false;
    if (kvr_status s = stage_fixed(ctx, lists, 1, st, staged)) return s;
    ++ctx->epoch;
    kvr::SelectArgs sa{};
    sa.scores = const_cast<double *>(scores);
    sa.lanes = lanes;
    sa.pages = pages;
    sa.k = k;
    sa.tie_higher_first = tie_rule == KVR_TIE_HIGHER_FIRST;
    sa.signed_scores = signed_scores != 0;
    sa.do_select = 1;
    if (kvr_status s = put_policy(pol, m, sa)) return s;
    sa.selected = selected;
    sa.count = count;
    sa.status = ctx->status;
    sa.epoch = ctx->epoch;
    KVR_HIP(pol.grouped ? kvr::launch_select_groups(sa, st) : kvr::launch_select(sa, st));
    return fixed_done(ctx, staged, st);
}
}  // namespace

kvr_status kvr_fold_half_pages(kvr_context *ctx, const double *halves, uint32_t lanes, uint32_t pages,
                               const uint8_t *score_mask, kvr_half_fold rule, double *scores, void *stream) {
    if (kvr_status s = check_ctx(ctx)) return s;
    lanes = lanes ? lanes : 1;
    if (!halves || !scores || !pages) return fail(KVR_ERR_INVALID, "halves, scores and pages are required");
    if (rule != KVR_HALF_SUM && rule != KVR_HALF_MAX) return fail(KVR_ERR_INVALID, "unknown half-page fold");
    if (lanes > 65535) return fail(KVR_ERR_INVALID, "at most 65535 lanes per call");
    DeviceGuard guard(ctx->device);
    ++ctx->epoch;
    kvr::FoldArgs a{};
    a.halves = halves;
    a.mask = score_mask;
    a.lanes = lanes;
    a.pages = pages;
    a.rule = rule == KVR_HALF_SUM ? kvr::kFoldSum : kvr::kFoldMax;
    a.scores = scores;
    a.status = ctx->status;
    a.epoch = ctx->epoch;
    KVR_HIP(kvr::launch_fold_halves(a, stream_or(stream, ctx->sel)));
    return KVR_OK;
}

kvr_status kvr_select_topk(kvr_context *ctx, const double *scores, uint32_t lanes, uint32_t pages, uint32_t k,
                           const uint32_t *mandatory, uint32_t n_mandatory, kvr_tie_rule tie_rule,
                           int signed_scores, uint32_t *selected, uint32_t *count, void *stream) {
    return select_common(ctx, scores, lanes, pages, k, mandatory, n_mandatory, nullptr, tie_rule, signed_scores,
                         selected, count, stream);
}

kvr_status kvr_select_pages(kvr_context *ctx, const double *scores, uint32_t lanes, uint32_t pages, uint32_t k,
                            const kvr_page_policy *policy, kvr_tie_rule tie_rule, int signed_scores,
                            uint32_t *selected, uint32_t *count, void *stream) {
    return select_common(ctx, scores, lanes, pages, k, nullptr, 0, policy, tie_rule, signed_scores, selected, count,
                         stream);
}

namespace {
kvr_status check_graph_frame(kvr_context *ctx, const double *scores, uint32_t pages) {
    if (kvr_status s = check_ctx(ctx)) return s;
    if (!scores || !pages) return fail(KVR_ERR_INVALID, "scores and pages are required");
    if (pages > kvr::kGraphMaxPages)
        return fail(KVR_ERR_UNSUPPORTED, "%u pages per lane exceed KVR_GRAPH_MAX_PAGES (%u)", pages,
                    kvr::kGraphMaxPages);
    return KVR_OK;
}
}  // namespace

namespace {
kvr_status graph_lanes(const kvr_page_graph *graphs, uint32_t lanes, std::vector<kvr::GraphLane> &g) {
    g.assign(lanes, kvr::GraphLane{});
    for (uint32_t l = 0; graphs && l < lanes; ++l) {
        const kvr_page_graph &x = graphs[l];
        if (x.n_rows && (!x.row_source || !x.row_begin))
            return fail(KVR_ERR_INVALID, "graph rows need row_source and row_begin (lane %u)", l);
        if (x.n_edges && (!x.edge_target || !x.edge_mass))
            return fail(KVR_ERR_INVALID, "graph edges need edge_target and edge_mass (lane %u)", l);
        g[l] = {x.n_rows, x.n_edges, x.row_source, x.row_begin, x.edge_target, x.edge_mass, x.neighbor_weight};
    }
    return KVR_OK;
}

kvr_status lrfu_args(const double *history, uint32_t history_pages, double lambda, double top_fraction,
                     double *candidate, uint32_t pages, kvr::GraphLrfuArgs &a) {
    if (!candidate) return fail(KVR_ERR_INVALID, "candidate is required");
    if (history_pages && !history) return fail(KVR_ERR_INVALID, "history_pages without history");
    if (!(lambda >= 0.0 && lambda <= 1.0) || !(top_fraction > 0.0 && top_fraction <= 1.0))
        return fail(KVR_ERR_INVALID, "invalid LRFU decay or hit fraction");
    a.lrfu = 1;
    a.history = history_pages ? history : nullptr;
    a.history_pages = history_pages;
    a.lambda = lambda;
    a.gate = top_fraction < 1.0;
    if (a.gate) {
        // the reference's rank: min(n - 1, size_t((1 - fraction) * n)) in binary64
        const double r = (1.0 - top_fraction) * double(pages);
        a.rank = std::min<uint32_t>(pages - 1, uint32_t(r));
    }
    a.candidate = candidate;
    return KVR_OK;
}

kvr_status launch_rescore(kvr_context *ctx, kvr::GraphLrfuArgs &a, const std::vector<kvr::GraphLane> &g,
                          uint32_t lanes, void *stream) {
    DeviceGuard guard(ctx->device);
    ++ctx->epoch;
    a.status = ctx->status;
    a.epoch = ctx->epoch;
    KVR_HIP(kvr::launch_graph_lrfu(a, g.data(), lanes, stream_or(stream, ctx->sel)));
    return KVR_OK;
}
}  // namespace

kvr_status kvr_propagate_scores(kvr_context *ctx, double *scores, uint32_t lanes, uint32_t pages,
                                const uint8_t *transport_mask, const kvr_page_graph *graphs, double alpha,
                                void *stream) {
    if (kvr_status s = check_graph_frame(ctx, scores, pages)) return s;
    lanes = lanes ? lanes : 1;
    if (!(alpha >= 0.0 && alpha <= 1.0)) return fail(KVR_ERR_INVALID, "invalid attention decay (alpha)");
    std::vector<kvr::GraphLane> g;
    if (kvr_status s = graph_lanes(graphs, lanes, g)) return s;
    kvr::GraphLrfuArgs a{};
    a.scores = scores;
    a.mask = transport_mask;
    a.pages = pages;
    a.propagate = 1;
    a.alpha = alpha;
    return launch_rescore(ctx, a, g, lanes, stream);
}

kvr_status kvr_lrfu_preview(kvr_context *ctx, const double *scores, uint32_t lanes, uint32_t pages,
                            const double *history, uint32_t history_pages, double lambda, double top_fraction,
                            double *candidate, void *stream) {
    if (kvr_status s = check_graph_frame(ctx, scores, pages)) return s;
    lanes = lanes ? lanes : 1;
    kvr::GraphLrfuArgs a{};
    a.scores = const_cast<double *>(scores);
    a.pages = pages;
    if (kvr_status s = lrfu_args(history, history_pages, lambda, top_fraction, candidate, pages, a)) return s;
    return launch_rescore(ctx, a, std::vector<kvr::GraphLane>(lanes), lanes, stream);
}

kvr_status kvr_propagate_lrfu(kvr_context *ctx, double *scores, uint32_t lanes, uint32_t pages,
                              const uint8_t *transport_mask, const kvr_page_graph *graphs, double alpha,
                              const double *history, uint32_t history_pages, double lambda, double top_fraction,
                              double *candidate, void *stream) {
    if (kvr_status s = check_graph_frame(ctx, scores, pages)) return s;
    lanes = lanes ? lanes : 1;
    if (!(alpha >= 0.0 && alpha <= 1.0)) return fail(KVR_ERR_INVALID, "invalid attention decay (alpha)");
    std::vector<kvr::GraphLane> g;
    if (kvr_status s = graph_lanes(graphs, lanes, g)) return s;
    kvr::GraphLrfuArgs a{};
    a.scores = scores;
    a.mask = transport_mask;
    a.pages = pages;
    a.propagate = 1;
    a.alpha = alpha;
    if (kvr_status s = lrfu_args(history, history_pages, lambda, top_fraction, candidate, pages, a)) return s;
    return launch_rescore(ctx, a, g, lanes, stream);
}

kvr_status kvr_stage_in(kvr_context *ctx, const kvr_plane *planes, uint32_t n_planes, uint32_t lanes,
                        uint32_t page_tokens, const uint32_t *selected, const uint32_t *count, uint32_t k,
                        kvr_copy_engine engine, void *stream) {
    if (kvr_status s = check_ctx(ctx)) return s;
    lanes = lanes ? lanes : 1;
    if (!selected || !count || !k || !page_tokens)
        return fail(KVR_ERR_INVALID, "selection, count, k and page_tokens are required");
    if (engine > KVR_ENGINE_SDMA) return fail(KVR_ERR_INVALID, "unknown copy engine");
    DeviceGuard guard(ctx->device);
    PlanePlan pp[KVR_MAX_PLANES];
    if (kvr_status s = check_planes(planes, n_planes, lanes, page_tokens, k, ctx->chunk_rows, pp)) return s;
    const hipStream_t s = stream_or(stream, ctx->copy);
    if (engine == KVR_ENGINE_SDMA) return enqueue_gather_sdma(ctx, pp, n_planes, lanes, page_tokens, selected, count, k, s);
    return enqueue_gather_kernel(ctx, pp, n_planes, lanes, page_tokens, selected, count, k, s);
}

namespace {

// One validated layer of recall: everything checked, nothing enqueued.
struct LayerPlan {
    const kvr_layer_recall *d = nullptr;
    // pages: summaries (softmax columns); page_tokens: tokens per selected
    // page (twice the summary grid with half pages); sel_pages: pages selected
    uint32_t pages = 0, page_tokens = 0, lanes = 1, sel_pages = 0;
    size_t key_ls = 0;
    Mandatory m;
    Policy pol;
    PlanePlan pp[KVR_MAX_PLANES];
    ScorePlan p;
    int src = kvr::kSrcSummary;
};

kvr_status plan_layer(kvr_context *ctx, const kvr_layer_recall *d, hipStream_t ss, hipStream_t cs, LayerPlan &L,
                      const FixedScratch *fixed = nullptr) {
    if (!d || !d->query || !d->summaries || !d->scores || !d->selected || !d->count)
        return fail(KVR_ERR_INVALID, "recall descriptor lacks query, summaries, scores or selection outputs");
    if (d->aggregation > KVR_AGG_MAX_LOGIT) return fail(KVR_ERR_INVALID, "unknown aggregation");
    if (d->tie_rule > KVR_TIE_HIGHER_FIRST) return fail(KVR_ERR_INVALID, "unknown tie rule");
    if (d->engine > KVR_ENGINE_SDMA) return fail(KVR_ERR_INVALID, "unknown copy engine");
    if (!d->k) return fail(KVR_ERR_INVALID, "invalid scored selection frame (budget 0)");
    L.d = d;
    L.pages = d->pages;
    L.page_tokens = d->page_tokens;
    if (d->keys) {
        if (kvr_status s = check_keys(d->keys, L.pages, L.key_ls)) return s;
        L.page_tokens = d->keys->page_tokens;
        L.lanes = d->keys->lanes ? d->keys->lanes : 1;
        L.src = d->keys->format == KVR_FMT_F16 ? kvr::kSrcKeysF16 : kvr::kSrcKeysQ8;
        if (d->keys->kv_heads != d->query->kv_heads || d->keys->head_dim != d->query->head_dim)
            return fail(KVR_ERR_INVALID, "key history and query disagree on kv heads or head_dim");
    } else {
        if (!L.pages || !L.page_tokens) return fail(KVR_ERR_INVALID, "resident summaries need pages and page_tokens");
        L.lanes = d->lanes ? d->lanes : 1;
    }
    if (kvr_status s = check_summary_out(d->means, d->summaries)) return s;
    if (d->half_fold > KVR_HALF_MAX) return fail(KVR_ERR_INVALID, "unknown half-page fold");
    L.sel_pages = L.pages;
    if (d->half_fold) {
        // layerwise_tile_scores (layerwise_selection.cpp:35-55): two Mean-K
        // records per sealed transport page
        const uint64_t tokens = d->keys ? d->keys->tokens : uint64_t(L.pages) * L.page_tokens;
        if (L.pages % 2 || tokens != uint64_t(L.pages) * L.page_tokens)
            return fail(KVR_ERR_INVALID, "half-page scores require whole transport pages of two summary pages");
        L.sel_pages = L.pages / 2;
        L.page_tokens *= 2;
    }
    if (kvr_status s = check_mandatory(d->mandatory, d->n_mandatory, L.sel_pages, d->k, L.m)) return s;
    if (kvr_status s = check_policy(d->policy, L.lanes, L.sel_pages, d->k, L.pol)) return s;
    if (!L.m.more.empty() && L.pol.p && L.pol.p->n_fixed)
        return fail(KVR_ERR_INVALID, "a host mandatory list longer than %d and a device fixed list cannot be combined",
                    KVR_MAX_INLINE_MANDATORY);
    if (kvr_status s = check_planes(d->planes, d->n_planes, L.lanes, L.page_tokens, d->k, ctx->chunk_rows, L.pp))
        return s;
    if ((d->summary_begin || d->summary_end || d->select_end) && capturing(ss))
        return fail(KVR_ERR_INVALID, "summary timing events are not recorded inside a captured graph");
    if (d->n_planes && d->engine == KVR_ENGINE_SDMA && (capturing(ss) || capturing(cs)))
        return fail(KVR_ERR_INVALID, "the DMA stage-in engine reads the selection on the host and cannot be "
                                     "captured; use the kernel engine inside graphs");
    if (kvr_status s = plan_score(ctx, d->query, L.lanes, L.pages, d->force_mfma, ss, L.p, fixed)) return s;
    L.p.fold = d->half_fold == KVR_HALF_SUM ? kvr::kFoldSum : d->half_fold == KVR_HALF_MAX ? kvr::kFoldMax
                                                                                        : kvr::kFoldNone;
    if (d->keys && !L.p.mfma && !valu_dim_ok(d->keys->head_dim))
        return fail(KVR_ERR_INVALID, "head_dim %u unsupported by fused scoring", d->keys->head_dim);
    return KVR_OK;
}

// The layer's selection is written on ss: its timing event, then its
// stage-in on cs after an event.
kvr_status enqueue_stage(kvr_context *ctx, LayerPlan &L, hipStream_t ss, hipStream_t cs) {
    const kvr_layer_recall *d = L.d;
    if (d->select_end) KVR_HIP(hipEventRecord(static_cast<hipEvent_t>(d->select_end), ss));
    if (!d->n_planes) return KVR_OK;
    KVR_HIP(hipEventRecord(ctx->ev_sel, ss));
    if (cs != ss) KVR_HIP(hipStreamWaitEvent(cs, ctx->ev_sel, 0));
    if (d->engine == KVR_ENGINE_SDMA)
        return enqueue_gather_sdma(ctx, L.pp, d->n_planes, L.lanes, L.page_tokens, d->selected, d->count, d->k, cs,
                                   ctx->ev_sel);
    return enqueue_gather_kernel(ctx, L.pp, d->n_planes, L.lanes, L.page_tokens, d->selected, d->count, d->k, cs);
}

kvr_status enqueue_layer(kvr_context *ctx, LayerPlan &L, hipStream_t ss, hipStream_t cs) {
    const kvr_layer_recall *d = L.d;
    ScorePlan &p = L.p;
    ++ctx->epoch;
    if (d->keys) {
        auto a = summary_args(ctx, d->keys, L.pages, L.key_ls, d->means, d->summaries);
        // the summary events are stamped with the kernel's own start and end
        const hipEvent_t b = static_cast<hipEvent_t>(d->summary_begin), e = static_cast<hipEvent_t>(d->summary_end);
        if (p.mfma) {
            KVR_HIP(kvr::launch_summary(L.src, false, a, ss, b, e));
        } else {
            a.q = p.q;
            a.q_stage = stage_query(p.q);
            a.logits = p.logits;
            KVR_HIP(kvr::launch_summary(L.src, true, a, ss, b, e));
        }
        if (p.mfma)
            if (kvr_status st = enqueue_logits(ctx, p, d->summaries, ss)) return st;
    } else {
        // resident summaries: the events bracket the logits launch
        if (d->summary_begin) KVR_HIP(hipEventRecord(static_cast<hipEvent_t>(d->summary_begin), ss));
        if (kvr_status st = enqueue_logits(ctx, p, d->summaries, ss)) return st;
        if (d->summary_end) KVR_HIP(hipEventRecord(static_cast<hipEvent_t>(d->summary_end), ss));
    }
    if (kvr_status st = enqueue_probs_and_select(ctx, p, d->score_mask, d->aggregation, 1, 0, d->scores, true, d->k,
                                                 d->tie_rule, L.m, d->selected, d->count, ss, &L.pol))
        return st;
    return enqueue_stage(ctx, L, ss, cs);
}

}  // namespace

kvr_status kvr_recall_layer(kvr_context *ctx, const kvr_layer_recall *d, void *select_stream, void *copy_stream) {
    if (kvr_status s = check_ctx(ctx)) return s;
    DeviceGuard guard(ctx->device);
    const hipStream_t ss = stream_or(select_stream, ctx->sel);
    const hipStream_t cs = stream_or(copy_stream, ctx->copy);
    LayerPlan L;
    if (kvr_status s = plan_layer(ctx, d, ss, cs, L)) return s;
    Mandatory *lists[1] = {&L.m};
    bool staged = false;
    if (kvr_status s = stage_fixed(ctx, lists, 1, ss, staged)) return s;
    if (kvr_status s = ws_order(ctx, ss)) return s;
    if (kvr_status s = enqueue_layer(ctx, L, ss, cs)) return s;
    return fixed_done(ctx, staged, ss);
}

kvr_status kvr_recall_layer_noalloc(kvr_context *ctx, const kvr_layer_recall *d, void *select_stream,
                                    void *copy_stream) {
    if (kvr_status s = check_ctx(ctx)) return s;
    if (d && d->engine == KVR_ENGINE_SDMA && d->n_planes)
        return fail(KVR_ERR_UNSUPPORTED, "the DMA stage-in engine allocates its staging; the no-allocation entry "
                                         "gathers with the kernel engine");
    DeviceGuard guard(ctx->device);
    const FixedScratch fixed{kvr::scratch_address(ctx->device), kvr::kScratchBytes};
    if (!fixed.base) return fail(KVR_ERR_HIP, "static scratch of device %d was not set up", ctx->device);
    const hipStream_t ss = stream_or(select_stream, ctx->sel);
    const hipStream_t cs = stream_or(copy_stream, ctx->copy);
    LayerPlan L;
    if (kvr_status s = plan_layer(ctx, d, ss, cs, L, &fixed)) return s;
    if (!L.m.more.empty())
        return fail(KVR_ERR_UNSUPPORTED, "more than %d host mandatory pages need an upload buffer; the no-allocation "
                                         "entry takes them as a device list (kvr_page_policy.fixed)",
                    KVR_MAX_INLINE_MANDATORY);
    // the counters must start at zero; a previous call on this GPU leaves them
    // so, but a clear by a kernel keeps the call safe after any abort
    KVR_HIP(kvr::launch_fill_u32(L.p.counters, L.lanes, 0u, ss));
    return enqueue_layer(ctx, L, ss, cs);
}

namespace {
kvr_status enqueue_stack(kvr_context *ctx, std::vector<LayerPlan> &plans, hipStream_t ss, hipStream_t cs);
}  // namespace

kvr_status kvr_recall_stack(kvr_context *ctx, const kvr_layer_recall *layers, uint32_t n, void *select_stream,
                            void *copy_stream) {
    if (kvr_status s = check_ctx(ctx)) return s;
    if (!n) return KVR_OK;
    if (!layers) return fail(KVR_ERR_INVALID, "missing layer descriptors");
    DeviceGuard guard(ctx->device);
    const hipStream_t ss = stream_or(select_stream, ctx->sel);
    const hipStream_t cs = stream_or(copy_stream, ctx->copy);
    std::vector<LayerPlan> plans(n);
    for (uint32_t l = 0; l < n; ++l)
        if (kvr_status s = plan_layer(ctx, &layers[l], ss, cs, plans[l])) return s;
    std::vector<Mandatory *> lists(n);
    for (uint32_t l = 0; l < n; ++l) lists[l] = &plans[l].m;
    bool staged = false;
    if (kvr_status s = stage_fixed(ctx, lists.data(), n, ss, staged)) return s;
    if (kvr_status s = ws_order(ctx, ss)) return s;
    if (kvr_status s = enqueue_stack(ctx, plans, ss, cs)) return s;
    return fixed_done(ctx, staged, ss);
}

namespace {
kvr_status enqueue_stack(kvr_context *ctx, std::vector<LayerPlan> &plans, hipStream_t ss, hipStream_t cs) {
    const uint32_t n = uint32_t(plans.size());
    // Layer l's softmax/selection rides in layer l+1's summary launch when
    // every layer takes the fused (vector) scoring path with one geometry.
    const ScorePlan &p0 = plans[0].p;
    bool fuse = n > 1;
    for (const LayerPlan &L : plans)
        fuse = fuse && !L.p.mfma && !L.pol.grouped && L.p.fold == p0.fold && L.p.lanes == p0.lanes &&
               L.p.pages == p0.pages &&
               L.p.rows == p0.rows && L.p.qheads == p0.qheads && L.p.kvheads == p0.kvheads && L.p.dim == p0.dim;
    if (!fuse) {
        for (LayerPlan &L : plans)
            if (kvr_status s = enqueue_layer(ctx, L, ss, cs)) return s;
        return KVR_OK;
    }
    if (p0.lanes > 65535) return fail(KVR_ERR_INVALID, "at most 65535 lanes per call");
    // Layers go in groups of up to kStackGroup consecutive layers with one
    // summary source; group k's summaries run in one launch beside group
    // k-1's softmax workgroups.  Key-history layers get their logits from
    // those softmax workgroups (computed from the stored summaries), resident
    // summaries from their own summary workgroups.  Two groups are in flight
    // at a time, so 2 * kStackGroup logits buffers and counter sets rotate by
    // layer.
    constexpr uint32_t G = kvr::kStackGroup;
    const size_t lb = logits_bytes(p0.lanes, p0.pages, p0.rows, p0.qheads);
    if (kvr_status s = ensure_workspace(ctx, 2 * G * lb, ss)) return s;
    if (kvr_status s = ensure_counters(ctx, 2 * G * p0.lanes, ss)) return s;
    std::vector<uint32_t> first;  // first layer of each group
    for (uint32_t l = 0; l < n; ++l)
        if (first.empty() || l - first.back() == G || plans[l].src != plans[first.back()].src) first.push_back(l);
    const uint32_t groups = uint32_t(first.size());
    first.push_back(n);
    kvr::StackGroupArgs g{};
    // enough softmax workgroups per lane for the most units an aggregation
    // has (rows * q-heads); workgroups past a layer's units only count in
    const uint32_t upb = kvr::units_per_block(p0.pages);
    g.probs_per_lane = (p0.rows * p0.qheads + upb - 1) / upb;
    g.q_slot = (p0.rows * p0.qheads * p0.dim + 7) / 8 * 8;
    int prev_src = plans[0].src;
    for (uint32_t k = 0; k <= groups; ++k) {
        g.mp = g.m;  // g.p holds that group's selections from the previous pass
        g.m = k < groups ? first[k + 1] - first[k] : 0;
        kvr::SelectArgs cur[G];
        for (uint32_t i = 0; i < g.m; ++i) {
            const uint32_t l = first[k] + i;
            LayerPlan &L = plans[l];
            const kvr_layer_recall *d = L.d;
            ++ctx->epoch;
            L.p.logits = reinterpret_cast<double *>(ctx->ws + (l % (2 * G)) * lb);
            const bool resident = L.src == kvr::kSrcSummary;
            kvr::SummaryArgs a = resident ? resident_args(ctx, L.p, d->summaries)
                                          : summary_args(ctx, d->keys, L.pages, L.key_ls, d->means, d->summaries);
            a.q = L.p.q;
            a.q_stage = stage_query(L.p.q);
            a.logits = L.p.logits;
            g.s[i] = a;
            cur[i] = make_select_args(ctx, L.p, d->score_mask, d->aggregation, 1, 0, d->scores, true, d->k,
                                      d->tie_rule, L.m, d->selected, d->count);
            if (kvr_status st = put_policy(L.pol, L.m, cur[i])) return st;
            cur[i].counters = ctx->counters + (l % (2 * G)) * p0.lanes;
            if (!resident) {
                cur[i].summaries = d->summaries;
                cur[i].q = L.p.q;
            }
        }
        // The first of the group's layers with summary events gets them
        // stamped by the launch itself (its start and end, no stream
        // markers); any other layer's events bracket the launch as markers.
        uint32_t timed = g.m;
        for (uint32_t i = 0; i < g.m && timed == g.m; ++i) {
            const kvr_layer_recall *d = plans[first[k] + i].d;
            if (d->summary_begin || d->summary_end) timed = i;
        }
        for (uint32_t i = 0; i < g.m; ++i) {
            const kvr_layer_recall *d = plans[first[k] + i].d;
            if (i != timed && d->summary_begin) KVR_HIP(hipEventRecord(static_cast<hipEvent_t>(d->summary_begin), ss));
        }
        const int src = g.m ? plans[first[k]].src : prev_src;
        const kvr_layer_recall *td = timed < g.m ? plans[first[k] + timed].d : nullptr;
        KVR_HIP(kvr::launch_stack_group(src, g, ss, td ? static_cast<hipEvent_t>(td->summary_begin) : nullptr,
                                        td ? static_cast<hipEvent_t>(td->summary_end) : nullptr));
        for (uint32_t i = 0; i < g.m; ++i) {
            const kvr_layer_recall *d = plans[first[k] + i].d;
            if (i != timed && d->summary_end) KVR_HIP(hipEventRecord(static_cast<hipEvent_t>(d->summary_end), ss));
        }
        if (k > 0)
            for (uint32_t l = first[k - 1]; l < first[k]; ++l)
                if (kvr_status s = enqueue_stage(ctx, plans[l], ss, cs)) return s;
        for (uint32_t i = 0; i < g.m; ++i) g.p[i] = cur[i];
        prev_src = src;
    }
    return KVR_OK;
}
}  // namespace

// ---- sampled attention ------------------------------------------------------

namespace {

constexpr size_t kAttnBudget = size_t(32) << 20;  // page log-sum-exp bytes per launch

// Per sampled row of a launch: the page log-sum-exps and, at most one per
// page, the page groups' (max, sum) pairs.
uint32_t attention_rows_per_launch(uint32_t n_rows, uint32_t heads, uint32_t pages) {
    const size_t per_row = std::max<size_t>(1, size_t(heads) * pages * 3 * sizeof(float));
    const size_t fit = std::max<size_t>(1, kAttnBudget / per_row);
    return uint32_t(std::min<size_t>({size_t(n_rows), fit, size_t(kvr::kAttnRows)}));
}

bool attention_key_format(kvr_format f) {
    return f == KVR_FMT_F16 || f == KVR_FMT_BF16 || f == KVR_FMT_F32 || f == KVR_FMT_Q8_0 || f == KVR_FMT_Q4_0 ||
           f == KVR_FMT_Q5_0;
}

size_t attention_key_row_bytes(kvr_format f, uint32_t dim) {
    switch (f) {
    case KVR_FMT_F16:
    case KVR_FMT_BF16: return size_t(dim) * 2;
    case KVR_FMT_F32: return size_t(dim) * 4;
    case KVR_FMT_Q8_0: return size_t(dim) / 32 * 34;
    case KVR_FMT_Q4_0: return size_t(dim) / 32 * 18;
    case KVR_FMT_Q5_0: return size_t(dim) / 32 * 22;
    default: return 0;
    }
}

}  // namespace

size_t kvr_attention_workspace_bytes(uint32_t n_rows, uint32_t query_heads, uint32_t pages) {
    if (!n_rows || !query_heads || !pages) return 0;
    const uint32_t rows = attention_rows_per_launch(n_rows, query_heads, pages);
    return align256(size_t(rows) * query_heads * pages * 3 * sizeof(float));
}

kvr_status kvr_attention_page_mass(kvr_context *ctx, const kvr_attention_sample *a, float *mass, void *stream) {
    if (kvr_status s = check_ctx(ctx)) return s;
    if (!a) return fail(KVR_ERR_INVALID, "missing attention sample");
    // What the reference's score() declines (returns false for).
    const size_t qel = scalar_bytes(a->q_format), mel = scalar_bytes(a->mask_format);
    if (!qel || !mel || !attention_key_format(a->k_format))
        return fail(KVR_ERR_UNSUPPORTED, "attention needs f32/f16/bf16 query and mask, f16/bf16/f32/q8_0/q4_0/q5_0 keys");
    if (!a->head_dim || a->head_dim % 32 || a->head_dim > 256)
        return fail(KVR_ERR_UNSUPPORTED, "attention head_dim %u: needs a multiple of 32, at most 256", a->head_dim);
    if (!a->q || !a->k || !a->mask || !mass) return fail(KVR_ERR_INVALID, "missing attention operand");
    if (!a->n_rows || !a->rows) return fail(KVR_ERR_INVALID, "no sampled rows");
    if (!a->query_heads || !a->kv_heads || a->query_heads % a->kv_heads || a->query_heads > 4096)
        return fail(KVR_ERR_INVALID, "query heads %u: need a multiple of kv heads %u, at most 4096", a->query_heads,
                    a->kv_heads);
    if (!a->tokens || !a->page_tokens) return fail(KVR_ERR_INVALID, "attention needs tokens and page_tokens");
    if (!std::isfinite(a->scale) || !std::isfinite(a->softcap) || a->softcap < 0)
        return fail(KVR_ERR_INVALID, "attention scale and softcap must be finite, softcap nonnegative");
    if (!aligned(a->q, qel) || a->q_row_stride % qel || a->q_head_stride % qel || !aligned(a->mask, mel) ||
        a->mask_row_stride % mel)
        return fail(KVR_ERR_INVALID, "query and mask strides must be multiples of their scalar size");
    const bool quant = a->k_format == KVR_FMT_Q8_0 || a->k_format == KVR_FMT_Q4_0 || a->k_format == KVR_FMT_Q5_0;
    const size_t kal = quant ? 2 : 16;
    if (!aligned(a->k, kal) || a->k_row_stride % kal || a->k_head_stride % kal)
        return fail(KVR_ERR_INVALID, "key rows and heads must start on %zu-byte boundaries", kal);
    if (a->k_row_stride >= (size_t(1) << 27))
        return fail(KVR_ERR_UNSUPPORTED, "key rows of %zu bytes: at most 128 MiB", size_t(a->k_row_stride));
    const size_t krow = attention_key_row_bytes(a->k_format, a->head_dim);
    if ((a->kv_heads > 1 && a->k_head_stride < krow) ||
        (a->tokens > 1 && a->k_row_stride < size_t(a->kv_heads - 1) * a->k_head_stride + krow))
        return fail(KVR_ERR_INVALID, "key strides overlap rows of %zu bytes", krow);
    const uint32_t pages = page_count(a->tokens, a->page_tokens);
    if (uint64_t(pages) * a->kv_heads > 0x7fffffffu) return fail(KVR_ERR_INVALID, "too many attention pages");
    if (uint64_t(pages) * a->query_heads * 2 * sizeof(float) > 0xffffffffull)
        return fail(KVR_ERR_UNSUPPORTED, "attention tables of one row (%u heads x %u pages) pass 4 GiB",
                    a->query_heads, pages);
    const uint32_t group = a->query_heads / a->kv_heads;
    const uint32_t chunk = attention_rows_per_launch(a->n_rows, a->query_heads, pages);
    DeviceGuard guard(ctx->device);
    const hipStream_t s = stream_or(stream, ctx->sel);
    if (kvr_status st = ensure_workspace(ctx, kvr_attention_workspace_bytes(a->n_rows, a->query_heads, pages), s))
        return st;
    kvr::AttnArgs g{};
    g.q = static_cast<const uint8_t *>(a->q);
    g.q_row_stride = a->q_row_stride;
    g.q_head_stride = a->q_head_stride;
    g.k = static_cast<const uint8_t *>(a->k);
    g.k_row_stride = a->k_row_stride;
    g.k_head_stride = a->k_head_stride;
    g.mask = static_cast<const uint8_t *>(a->mask);
    g.mask_row_stride = a->mask_row_stride;
    g.q_scalar = uint32_t(a->q_format);
    g.mask_scalar = uint32_t(a->mask_format);
    g.k_format = uint32_t(a->k_format);
    g.dim = a->head_dim;
    g.heads = a->query_heads;
    g.kvheads = a->kv_heads;
    g.group = group;
    g.tokens = a->tokens;
    g.page_tokens = a->page_tokens;
    g.pages = pages;
    // pages per workgroup, at most 16: about 256 workgroups per pair tile
    // for fp16 keys, 512 for q8_0 keys staged on the fp16 matrix cores,
    // 1024 for keys decoded to binary32 (measured at 131072 tokens: the
    // fp16 form streams longest at one wave per SIMD, the staged q8_0 form
    // at two)
    const uint32_t target = a->k_format == KVR_FMT_F16                              ? 256
                            : a->k_format == KVR_FMT_Q8_0 && a->head_dim % 128 == 0 ? 512
                                                                                     : 1024;
    g.page_group = ctx->attn_page_group ? ctx->attn_page_group
                                        : uint32_t(std::min<uint64_t>(16, std::max<uint64_t>(1, uint64_t(pages) * a->kv_heads / target)));
    g.scale = a->scale;
    g.softcap = a->softcap;
    g.lse = reinterpret_cast<float *>(ctx->ws);
    g.stats = g.lse + size_t(chunk) * a->query_heads * pages;
    if (kvr_status st = ws_order(ctx, s)) return st;
    for (uint32_t first = 0; first < a->n_rows; first += chunk) {
        g.n_rows = std::min(chunk, a->n_rows - first);
        std::copy(a->rows + first, a->rows + first + g.n_rows, g.rows);
        const uint32_t *mr = a->mask_rows ? a->mask_rows : a->rows;
        std::copy(mr + first, mr + first + g.n_rows, g.mask_rows);
        g.mass = mass + size_t(first) * pages;
        KVR_HIP(kvr::launch_attention(g, s));
    }
    return KVR_OK;
}

kvr_status kvr_d2d_batched(kvr_context *ctx, const void *const *src, void *const *dst, const size_t *nbytes,
                           uint32_t n, void *stream) {
    if (kvr_status s = check_ctx(ctx)) return s;
    if (!n) return KVR_OK;
    if (!src || !dst || !nbytes) return fail(KVR_ERR_INVALID, "missing copy tables");
    DeviceGuard guard(ctx->device);
    const hipStream_t s = stream_or(stream, ctx->sel);
    if (capturing(s))
        return fail(KVR_ERR_INVALID, "batched copies upload their op table through pinned memory and cannot be "
                                     "captured");
    // the slot's previous copy launch (on whatever stream) must have read
    // its table before the table is rewritten
    kvr_context::OpSlot &slot = ctx->ops[ctx->ops_next];
    ctx->ops_next = (ctx->ops_next + 1) % kvr_context::kOpSlots;
    KVR_HIP(hipEventSynchronize(slot.done));
    if (slot.cap < n) {
        if (slot.dev) KVR_HIP(hipFree(slot.dev));
        if (slot.pin) KVR_HIP(hipHostFree(slot.pin));
        slot.dev = slot.pin = nullptr;
        slot.cap = 0;
        KVR_HIP(hipMalloc(&slot.dev, sizeof(kvr::CopyOp) * n));
        KVR_HIP(hipHostMalloc(reinterpret_cast<void **>(&slot.pin), sizeof(kvr::CopyOp) * n, hipHostMallocDefault));
        slot.cap = n;
    }
    for (uint32_t i = 0; i < n; ++i)
        slot.pin[i] = kvr::CopyOp{static_cast<const uint8_t *>(src[i]), static_cast<uint8_t *>(dst[i]), nbytes[i]};
    KVR_HIP(hipMemcpyAsync(slot.dev, slot.pin, sizeof(kvr::CopyOp) * n, hipMemcpyHostToDevice, s));
    KVR_HIP(kvr::launch_copy_ops(slot.dev, n, s));
    KVR_HIP(hipEventRecord(slot.done, s));
    return KVR_OK;
}

kvr_status kvr_host_alloc(size_t bytes, void **out) {
    if (!out || !bytes) return fail(KVR_ERR_INVALID, "invalid pinned allocation");
    *out = nullptr;
    KVR_HIP(hipHostMalloc(out, bytes, hipHostMallocDefault));
    return KVR_OK;
}

kvr_status kvr_host_free(void *ptr) {
    if (ptr) KVR_HIP(hipHostFree(ptr));
    return KVR_OK;
}

kvr_status kvr_h2d_peak_gbps(kvr_context *ctx, size_t bytes, int reps, double *gbps) {
    if (kvr_status s = check_ctx(ctx)) return s;
    if (!bytes || reps < 1 || !gbps) return fail(KVR_ERR_INVALID, "invalid bandwidth probe");
    DeviceGuard guard(ctx->device);
    void *host = nullptr, *dev = nullptr;
    hipEvent_t a = nullptr, b = nullptr;
    kvr_status st = KVR_OK;
    hipError_t e = hipHostMalloc(&host, bytes, hipHostMallocDefault);
    if (e == hipSuccess) e = hipMalloc(&dev, bytes);
    if (e == hipSuccess) e = hipEventCreate(&a);
    if (e == hipSuccess) e = hipEventCreate(&b);
    if (e == hipSuccess) e = hipMemset(dev, 0, bytes);
    if (e == hipSuccess) std::memset(host, 1, bytes);
    float best = 0;
    for (int i = 0; e == hipSuccess && i <= reps; ++i) {
        e = hipEventRecord(a, ctx->copy);
        if (e == hipSuccess) e = hipMemcpyAsync(dev, host, bytes, hipMemcpyHostToDevice, ctx->copy);
        if (e == hipSuccess) e = hipEventRecord(b, ctx->copy);
        if (e == hipSuccess) e = hipEventSynchronize(b);
        float ms = 0;
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, a, b);
        if (e == hipSuccess && i > 0 && (best == 0 || ms < best)) best = ms;  // first copy warms up
    }
    if (e != hipSuccess) st = hip_fail(e, "H2D bandwidth probe");
    else *gbps = double(bytes) / (double(best) * 1e-3) / 1e9;
    if (a) (void)hipEventDestroy(a);
    if (b) (void)hipEventDestroy(b);
    if (dev) (void)hipFree(dev);
    if (host) (void)hipHostFree(host);
    return st;
}

kvr_status kvr_h2d_read_peak_gbps(kvr_context *ctx, size_t bytes, int reps, double *gbps) {
    if (kvr_status s = check_ctx(ctx)) return s;
    if (!bytes || bytes % 16 || reps < 1 || !gbps) return fail(KVR_ERR_INVALID, "invalid bandwidth probe");
    DeviceGuard guard(ctx->device);
    void *host = nullptr, *mapped = nullptr, *dev = nullptr;
    hipEvent_t a = nullptr, b = nullptr;
    kvr_status st = KVR_OK;
    hipError_t e = hipHostMalloc(&host, bytes, hipHostMallocDefault);
    if (e == hipSuccess) e = hipHostGetDevicePointer(&mapped, host, 0);
    if (e == hipSuccess) e = hipMalloc(&dev, bytes);
    if (e == hipSuccess) e = hipEventCreate(&a);
    if (e == hipSuccess) e = hipEventCreate(&b);
    if (e == hipSuccess) std::memset(host, 1, bytes);
    float best = 0;
    for (int i = 0; e == hipSuccess && i <= reps; ++i) {
        e = hipEventRecord(a, ctx->copy);
        if (e == hipSuccess) e = kvr::launch_link_read(mapped, dev, bytes, ctx->copy);
        if (e == hipSuccess) e = hipEventRecord(b, ctx->copy);
        if (e == hipSuccess) e = hipEventSynchronize(b);
        float ms = 0;
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, a, b);
        if (e == hipSuccess && i > 0 && (best == 0 || ms < best)) best = ms;  // first read warms up
    }
    if (e != hipSuccess) st = hip_fail(e, "H2D kernel read probe");
    else *gbps = double(bytes) / (double(best) * 1e-3) / 1e9;
    if (a) (void)hipEventDestroy(a);
    if (b) (void)hipEventDestroy(b);
    if (dev) (void)hipFree(dev);
    if (host) (void)hipHostFree(host);
    return st;
}

// ---- synthetic inputs -----------------------------------------------------
namespace {
kvr_status synth(kvr_context *ctx, kvr::SynthArgs a, uint64_t seed, uint64_t sid, void *stream) {
    if (kvr_status s = check_ctx(ctx)) return s;
    if (!a.out) return fail(KVR_ERR_INVALID, "null synthetic output");
    if (!a.count) return KVR_OK;
    DeviceGuard guard(ctx->device);
    a.base = kvr::synth_base(seed, sid);
    KVR_HIP(kvr::launch_synth(a, stream_or(stream, ctx->sel)));
    return KVR_OK;
}
}  // namespace

kvr_status kvr_synth_normal_f16(kvr_context *ctx, uint64_t seed, uint64_t sid, uint64_t count, uint16_t *out,
                                void *stream) {
    kvr::SynthArgs a{};
    a.kind = kvr::kSynthNormalF16;
    a.count = count;
    a.out = out;
    return synth(ctx, a, seed, sid, stream);
}

kvr_status kvr_synth_scaled_normal_f16(kvr_context *ctx, uint64_t seed, uint64_t sid, uint64_t rows,
                                       uint32_t width, const float *scale, uint16_t *out, void *stream) {
    if (!scale || !width) return fail(KVR_ERR_INVALID, "scaled normal needs a channel scale");
    kvr::SynthArgs a{};
    a.kind = kvr::kSynthScaledNormalF16;
    a.count = rows * width;
    a.width = width;
    a.scale = scale;
    a.out = out;
    return synth(ctx, a, seed, sid, stream);
}

kvr_status kvr_synth_normal_f32(kvr_context *ctx, uint64_t seed, uint64_t sid, uint64_t count, float *out,
                                void *stream) {
    kvr::SynthArgs a{};
    a.kind = kvr::kSynthNormalF32;
    a.count = count;
    a.out = out;
    return synth(ctx, a, seed, sid, stream);
}

kvr_status kvr_synth_q8_0(kvr_context *ctx, uint64_t seed, uint64_t sid, uint64_t blocks, float d_lo, float d_hi,
                          uint8_t *out, void *stream) {
    kvr::SynthArgs a{};
    a.kind = kvr::kSynthQ8;
    a.count = blocks;
    a.lo = d_lo;
    a.hi = d_hi;
    a.out = out;
    return synth(ctx, a, seed, sid, stream);
}

kvr_status kvr_synth_q4_1(kvr_context *ctx, uint64_t seed, uint64_t sid, uint64_t blocks, float d_lo, float d_hi,
                          float m_lo, float m_hi, uint8_t *out, void *stream) {
    kvr::SynthArgs a{};
    a.kind = kvr::kSynthQ41;
    a.count = blocks;
    a.lo = d_lo;
    a.hi = d_hi;
    a.lo2 = m_lo;
    a.hi2 = m_hi;
    a.out = out;
    return synth(ctx, a, seed, sid, stream);
}

kvr_status kvr_synth_normal_q8_0(kvr_context *ctx, uint64_t seed, uint64_t sid, uint64_t blocks, uint8_t *out,
                                 void *stream) {
    kvr::SynthArgs a{};
    a.kind = kvr::kSynthNormalQ8;
    a.count = blocks;
    a.out = out;
    return synth(ctx, a, seed, sid, stream);
}

}  // extern "C"
