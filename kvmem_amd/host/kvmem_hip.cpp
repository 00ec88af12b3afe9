// kvmem_hip.cpp -- C++ host layer over the recall C ABI (include/kvrecall.h).
// Everything on the device goes through kvr_* calls; this file only
// validates, stages host operands, owns buffers and translates statuses into
// the exception and bool conventions of KVMem's own interfaces.
#include "kvmem_hip/kvmem_hip.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <limits>
#include <stdexcept>

namespace kvmem_hip {
namespace {

[[noreturn]] void throw_status(kvr_status s, const char *what) {
    std::string msg = std::string(what) + ": " + kvr_last_error();
    switch (s) {
    case KVR_ERR_WORKSPACE: throw std::length_error(msg);
    case KVR_ERR_HIP:
    case KVR_ERR_BUDGET: throw std::runtime_error(msg);  // the reference's required-keep failure
    default: throw std::invalid_argument(msg);
    }
}
void ok(kvr_status s, const char *what) {
    if (s != KVR_OK) throw_status(s, what);
}
void hip_ok(hipError_t e, const char *what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}
void require(bool cond, const char *msg) {
    if (!cond) throw std::invalid_argument(msg);
}
size_t align256(size_t b) {
    if (b > std::numeric_limits<size_t>::max() - 255) throw std::length_error("workspace size overflow");
    return (b + 255) / 256 * 256;
}

struct DeviceBinding {
    int previous = 0;
    explicit DeviceBinding(int device) {
        hip_ok(hipGetDevice(&previous), "hipGetDevice");
        hip_ok(hipSetDevice(device), "hipSetDevice");
    }
    ~DeviceBinding() { (void)hipSetDevice(previous); }
};

// Drains a stream on scope exit unless disarmed: a throwing call leaves no
// work in flight over buffers it owns.
struct StreamDrain {
    hipStream_t stream;
    bool armed = true;
    ~StreamDrain() {
        if (armed) (void)hipStreamSynchronize(stream);
    }
};

bool capturing(hipStream_t s) {
    hipStreamCaptureStatus c = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(s, &c) == hipSuccess && c != hipStreamCaptureStatusNone;
}

kvr_format query_format(NativeQueryScalar s) {
    switch (s) {
    case NativeQueryScalar::Float32: return KVR_FMT_F32;
    case NativeQueryScalar::Float16: return KVR_FMT_F16;
    case NativeQueryScalar::BFloat16: return KVR_FMT_BF16;
    }
    throw std::invalid_argument("unknown native Query scalar");
}
size_t query_scalar_bytes(NativeQueryScalar s) { return s == NativeQueryScalar::Float32 ? 4 : 2; }

kvr_aggregation to_kvr(GqaScoreAggregation a) {
    switch (a) {
    case GqaScoreAggregation::Mean: return KVR_AGG_MEAN;
    case GqaScoreAggregation::Max: return KVR_AGG_MAX;
    case GqaScoreAggregation::MaxLogit: return KVR_AGG_MAX_LOGIT;
    }
    throw std::invalid_argument("invalid page softmax GQA aggregation");
}

constexpr uint32_t kRowsPerLaunch = 64;           // query rows scored per kvr_score call
constexpr size_t kLogitsBudget = size_t(64) << 20;  // binary64 logits per call

}  // namespace

// ---------------------------------------------------------------------------
QueryScoreFrame query_score_frame(uint64_t accepted, uint32_t block_tokens, uint32_t budget, uint32_t sink,
                                  uint32_t recent, const std::vector<uint32_t> &fixed) {
    require(block_tokens && budget, "invalid Query score budget or block size");
    const uint64_t pages = (accepted + block_tokens - 1) / block_tokens;
    require(pages <= std::numeric_limits<uint32_t>::max(), "Query index exceeds logical page capacity");
    const size_t n = size_t(pages);
    QueryScoreFrame f;
    f.accepted_through = accepted;
    f.starts.resize(n);
    f.counts.resize(n);
    for (size_t i = 0; i < n; ++i) {
        f.starts[i] = uint64_t(i) * block_tokens;
        f.counts[i] = uint32_t(std::min<uint64_t>(block_tokens, accepted - f.starts[i]));
    }
    const bool over = pages > budget;
    f.score_mask.assign(n, 1);
    f.transport_mask.assign(n, over ? 1 : 0);
    if (over && uint64_t(sink) + recent < pages) {
        std::fill(f.score_mask.begin(), f.score_mask.begin() + std::min<size_t>(sink, n), uint8_t(0));
        std::fill(f.score_mask.end() - std::min<size_t>(recent, n), f.score_mask.end(), uint8_t(0));
    }
    for (uint32_t id : fixed) {
        require(id < pages, "fixed Query block is outside the accepted index");
        f.transport_mask[id] = 0;
    }
    return f;
}

// Rules (native_layer_query.hpp:36-58):
//  G: data, every count and the GQA group are present, the scale is finite
//     and >= 0, and data is aligned to the scalar;
//  S: every stride is a positive multiple of the scalar, and an axis with
//     more than one element starts past everything the axes nested inside
//     it reach (the axes with smaller (stride, count), ties by position), so
//     no two elements share bytes, in any axis order; the reach stays
//     within size_t;
//  E: the reach of all three axes fits in `bytes`.
void validate_native_layer_query(const NativeCurrentLayerQuery &q) {
    const bool shaped = q.data && q.rows && q.query_heads && q.kv_heads && q.head_dim &&
                        q.query_heads % q.kv_heads == 0;
    const bool scaled = std::isfinite(q.attention_scale) && q.attention_scale >= 0;
    const size_t el = query_scalar_bytes(q.scalar);
    if (!shaped || !scaled || reinterpret_cast<uintptr_t>(q.data) % el != 0)
        throw std::invalid_argument("invalid native current-layer Query geometry");

    using wide = unsigned __int128;
    const size_t stride[3] = {q.row_stride, q.head_stride, q.dimension_stride};
    const uint32_t count[3] = {q.rows, q.query_heads, q.head_dim};
    auto inside = [&](int a, int b) {  // axis a is nested inside axis b
        if (stride[a] != stride[b]) return stride[a] < stride[b];
        return count[a] != count[b] ? count[a] < count[b] : a < b;
    };
    const wide limit = std::numeric_limits<size_t>::max();
    wide total = el;
    for (int a = 0; a < 3; ++a) {
        wide reach = el;  // bytes spanned by the axes nested inside a
        for (int b = 0; b < 3; ++b)
            if (b != a && inside(b, a)) reach += wide(stride[b]) * (count[b] - 1);
        const wide step = wide(stride[a]) * (count[a] > 1 ? count[a] - 1 : 1);
        if (stride[a] == 0 || stride[a] % el != 0 || (count[a] > 1 && stride[a] < reach) || step > limit - reach)
            throw std::invalid_argument("overlapping or overflowing native Query strides");
        total += wide(stride[a]) * (count[a] - 1);
    }
    if (total > q.bytes) throw std::invalid_argument("native Query exceeds its declared byte extent");
}

// ---------------------------------------------------------------------------
struct PageSoftmaxHip::Impl {
    int device = 0;
    kvr_context *ctx = nullptr;
    bool borrowed = false;
    uint32_t max_blocks = 0, qheads = 0, kvheads = 0, dim = 0;
    // device buffers: owned (grown on demand) or carved from the workspace
    float *q = nullptr;
    size_t q_cap = 0;  // floats
    uint8_t *mask = nullptr;
    double *scores = nullptr;
    uint32_t *sel = nullptr, *cnt = nullptr;
    // page-policy lists of media-aware picks: fixed pages [pages], groups
    // [pages][2], the grouped pass's selection [pages] and count
    uint32_t *fixed = nullptr, *groups = nullptr, *sel2 = nullptr, *cnt2 = nullptr;
    size_t page_cap = 0;
    // staging of host page means: binary32 [pages][width], counts of one,
    // fp16 operands
    float *msum = nullptr;
    uint32_t *mcount = nullptr;
    uint16_t *m16 = nullptr;
    size_t mean_cap = 0;  // elements
    uint32_t mean_pages = 0;
    std::vector<void *> owned;

    void score_layer(const uint16_t *summaries, const float *base, const PageQueryView &v, uint32_t layer,
                     uint32_t pages, uint32_t batch, kvr_aggregation agg, uint32_t active, bool &accumulate,
                     hipStream_t s);
    uint32_t check_view(const PageQueryView &v, uint32_t layers);
    hipStream_t current_layer_stream(const NativeCurrentLayerQuery &q, uint32_t pages, void *producer_stream);
    std::vector<double> current_layer(const uint16_t *summaries, const NativeCurrentLayerQuery &q,
                                      const QueryScoreFrame &frame, hipStream_t s);

    static size_t mean_bytes(uint32_t pages, uint32_t width) {
        return align256(size_t(pages) * width * 4) + align256(size_t(pages) * 4) + align256(size_t(pages) * width * 2);
    }
    void carve_means(uint8_t *b, uint32_t pages, uint32_t width) {
        msum = reinterpret_cast<float *>(b);
        b += align256(size_t(pages) * width * 4);
        mcount = reinterpret_cast<uint32_t *>(b);
        b += align256(size_t(pages) * 4);
        m16 = reinterpret_cast<uint16_t *>(b);
        mean_cap = size_t(pages) * width;
        mean_pages = pages;
    }
    // Means staging for `pages` x `width`; the counts are all one.
    void reserve_means(uint32_t pages, uint32_t width) {
        const size_t need = size_t(pages) * width;
        if (borrowed) {
            if (need > mean_cap || pages > mean_pages)
                throw std::length_error("page softmax exceeds its planned device workspace");
        } else if (need > mean_cap || pages > mean_pages) {
            hip_ok(hipStreamSynchronize(stream()), "hipStreamSynchronize");
            void *p = nullptr;
            hip_ok(hipMalloc(&p, mean_bytes(pages, width)), "hipMalloc page means");
            owned.push_back(p);
            carve_means(static_cast<uint8_t *>(p), pages, width);
            ones_pages = 0;
        }
        if (ones_pages < pages) {
            const std::vector<uint32_t> ones(pages, 1u);
            hip_ok(hipMemcpyAsync(mcount, ones.data(), size_t(pages) * 4, hipMemcpyHostToDevice, stream()),
                   "counts H2D");
            hip_ok(hipStreamSynchronize(stream()), "hipStreamSynchronize");
            ones_pages = pages;
        }
    }
    uint32_t ones_pages = 0;

    ~Impl() {
        if (ctx) {
            (void)hipSetDevice(device);
            (void)kvr_check(ctx, nullptr);
        }
        for (void *p : owned) (void)hipFree(p);
        if (ctx) (void)kvr_destroy(ctx);
    }

    hipStream_t stream() const { return static_cast<hipStream_t>(kvr_select_stream(ctx)); }

    void reserve(uint32_t rows, uint32_t pages) {
        const size_t qf = size_t(rows) * qheads * dim;
        if (borrowed) {
            if (qf > q_cap || pages > page_cap)
                throw std::length_error("page softmax exceeds its planned device workspace");
            return;
        }
        hip_ok(hipStreamSynchronize(stream()), "hipStreamSynchronize");
        if (qf > q_cap) {
            void *p = nullptr;
            hip_ok(hipMalloc(&p, qf * sizeof(float)), "hipMalloc query");
            owned.push_back(p);
            q = static_cast<float *>(p);
            q_cap = qf;
        }
        if (pages > page_cap) {
            void *p = nullptr;
            hip_ok(hipMalloc(&p, page_bytes(pages)), "hipMalloc scores");
            owned.push_back(p);
            carve_pages(static_cast<uint8_t *>(p), pages);
        }
    }

    // Per-page buffers: mask, scores, selection and count, then the policy
    // lists.
    static size_t page_bytes(uint32_t pages) {
        return align256(pages) + align256(size_t(pages) * 8) + 2 * align256(size_t(pages) * 4) + 256 +
               align256(size_t(pages) * 8) + align256(size_t(pages) * 4) + 256;
    }
    void carve_pages(uint8_t *b, uint32_t pages) {
        mask = b;
        b += align256(pages);
        scores = reinterpret_cast<double *>(b);
        b += align256(size_t(pages) * 8);
        sel = reinterpret_cast<uint32_t *>(b);
        b += align256(size_t(pages) * 4);
        fixed = reinterpret_cast<uint32_t *>(b);
        b += align256(size_t(pages) * 4);
        cnt = reinterpret_cast<uint32_t *>(b);
        cnt2 = cnt + 1;
        b += 256;
        groups = reinterpret_cast<uint32_t *>(b);
        b += align256(size_t(pages) * 8);
        sel2 = reinterpret_cast<uint32_t *>(b);
        page_cap = pages;
    }

    static size_t carve_bytes(uint32_t max_blocks, uint32_t qheads, uint32_t kvheads, uint32_t dim) {
        return align256(size_t(kRowsPerLaunch) * qheads * dim * sizeof(float)) + page_bytes(max_blocks) +
               mean_bytes(max_blocks, kvheads * dim);
    }

    // Rows of one kvr_score call within the logits budget of the workspace.
    uint32_t rows_per_call(uint32_t pages) const {
        const size_t row_bytes = size_t(pages) * qheads * sizeof(double);
        if (row_bytes > kLogitsBudget) throw std::length_error("page softmax needs a larger per-row logits budget");
        return uint32_t(std::max<size_t>(1, std::min<size_t>(kRowsPerLaunch, kLogitsBudget / row_bytes)));
    }

    void check_frame(const PageSummaries &s, const QueryScoreFrame &f) const {
        const size_t n = f.starts.size();
        require(n && f.counts.size() == n && f.score_mask.size() == n && f.transport_mask.size() == n,
                "page softmax frame geometry mismatch");
        require(n <= s.pages && s.page_tokens && s.kv_heads == kvheads && s.head_dim == dim,
                "page softmax summaries do not cover the frame");
        for (size_t b = 0; b < n; ++b)
            require(f.counts[b] && f.starts[b] == uint64_t(b) * s.page_tokens && f.starts[b] <= f.accepted_through &&
                        f.counts[b] <= f.accepted_through - f.starts[b],
                    "invalid accepted Query extent");
    }

    std::vector<double> fetch(uint32_t pages, hipStream_t s) {
        std::vector<double> out(pages);
        hip_ok(hipMemcpyAsync(out.data(), scores, size_t(pages) * 8, hipMemcpyDeviceToHost, s), "scores D2H");
        hip_ok(hipStreamSynchronize(s), "hipStreamSynchronize");
        ok(kvr_check(ctx, s), "page softmax");
        return out;
    }
};

PageSoftmaxHip::PageSoftmaxHip(int device) : impl_(new Impl) {
    impl_->device = device;
    DeviceBinding bind(device);
    ok(kvr_create(device, &impl_->ctx), "page softmax context");
}

size_t PageSoftmaxHip::workspace_bytes(uint32_t max_blocks, uint32_t qheads, uint32_t kvheads, uint32_t dim) {
    require(max_blocks && qheads && kvheads && dim && qheads % kvheads == 0 &&
                size_t(max_blocks) * qheads * sizeof(double) <= kLogitsBudget,
            "invalid planned page softmax geometry");
    const uint32_t rows =
        uint32_t(std::min<size_t>(kRowsPerLaunch, kLogitsBudget / (size_t(max_blocks) * qheads * sizeof(double))));
    return align256(kvr_workspace_bytes(1, max_blocks, rows, qheads, kvheads, dim)) +
           Impl::carve_bytes(max_blocks, qheads, kvheads, dim);
}

PageSoftmaxHip::PageSoftmaxHip(int device, void *workspace, size_t bytes, uint32_t max_blocks, uint32_t qheads,
                               uint32_t kvheads, uint32_t dim)
    : impl_(new Impl) {
    const size_t need = workspace_bytes(max_blocks, qheads, kvheads, dim);
    if (!workspace || reinterpret_cast<uintptr_t>(workspace) % 256 || bytes < need)
        throw std::invalid_argument("page softmax borrowed workspace is missing, unaligned or too small");
    Impl &m = *impl_;
    m.device = device;
    m.borrowed = true;
    m.max_blocks = max_blocks;
    m.qheads = qheads;
    m.kvheads = kvheads;
    m.dim = dim;
    DeviceBinding bind(device);
    ok(kvr_create(device, &m.ctx), "page softmax context");
    const uint32_t rows =
        uint32_t(std::min<size_t>(kRowsPerLaunch, kLogitsBudget / (size_t(max_blocks) * qheads * sizeof(double))));
    const size_t ws = align256(kvr_workspace_bytes(1, max_blocks, rows, qheads, kvheads, dim));
    ok(kvr_bind_workspace(m.ctx, workspace, ws), "page softmax workspace");
    uint8_t *b = static_cast<uint8_t *>(workspace) + ws;
    m.q = reinterpret_cast<float *>(b);
    m.q_cap = size_t(rows) * qheads * dim;
    b += align256(size_t(kRowsPerLaunch) * qheads * dim * sizeof(float));
    m.carve_pages(b, max_blocks);
    m.carve_means(b + Impl::page_bytes(max_blocks), max_blocks, kvheads * dim);
}

PageSoftmaxHip::~PageSoftmaxHip() = default;

// One layer's Query rows against its fp16 summaries, in batches of `batch`
// rows staged through the device Query buffer; each call adds its share of
// the scores (the first call of a score() sets them).
void PageSoftmaxHip::Impl::score_layer(const uint16_t *summaries, const float *base, const PageQueryView &v,
                                       uint32_t layer, uint32_t pages, uint32_t batch, kvr_aggregation agg,
                                       uint32_t active, bool &accumulate, hipStream_t s) {
    const size_t qw = size_t(v.query_heads) * v.head_dim;
    for (uint32_t r0 = 0; r0 < v.layer_rows[layer]; r0 += batch) {
        const uint32_t rows = std::min(batch, v.layer_rows[layer] - r0);
        hip_ok(hipMemcpyAsync(q, base + size_t(r0) * qw, size_t(rows) * qw * sizeof(float), hipMemcpyHostToDevice,
                              s),
               "query H2D");
        kvr_query kq{};
        kq.data = q;
        kq.scalar = KVR_FMT_F32;
        kq.rows = rows;
        kq.query_heads = v.query_heads;
        kq.kv_heads = v.kv_heads;
        kq.head_dim = v.head_dim;
        kq.row_stride = qw * sizeof(float);
        kq.head_stride = size_t(v.head_dim) * sizeof(float);
        kq.dim_stride = sizeof(float);
        kq.attention_scale = v.attention_scale;
        ok(kvr_score(ctx, &kq, summaries, 1, pages, mask, agg, active, accumulate, scores, 0, s), "page softmax");
        accumulate = true;
    }
}

uint32_t PageSoftmaxHip::Impl::check_view(const PageQueryView &v, uint32_t layers) {
    require((v.data || v.layer_data) && v.layer_rows && v.layers && v.rows && v.head_dim && v.kv_heads &&
                v.query_heads && v.query_heads % v.kv_heads == 0 && v.layers == layers,
            "page softmax geometry mismatch");
    if (!borrowed) {
        qheads = v.query_heads;
        kvheads = v.kv_heads;
        dim = v.head_dim;
    }
    require(v.query_heads == qheads && v.kv_heads == kvheads && v.head_dim == dim, "page softmax geometry mismatch");
    uint32_t active = 0;
    for (uint32_t l = 0; l < v.layers; ++l) {
        require(v.layer_rows[l] <= v.rows, "page softmax row count exceeds its storage");
        active += v.layer_rows[l] != 0;
    }
    return active;
}

static const float *query_layer(const PageQueryView &v, uint32_t l) {
    const float *base = v.layer_data ? v.layer_data[l] : v.data + size_t(l) * v.rows * v.query_heads * v.head_dim;
    require(base != nullptr, "missing active Query layer storage");
    return base;
}

std::vector<double> PageSoftmaxHip::score(const PageSummaries &sums, PageQueryView v, const QueryScoreFrame &frame,
                                          GqaScoreAggregation aggregation) {
    Impl &m = *impl_;
    const kvr_aggregation agg = to_kvr(aggregation);
    const uint32_t active = m.check_view(v, uint32_t(sums.layers.size()));
    m.check_frame(sums, frame);
    const uint32_t n = uint32_t(frame.starts.size());
    std::vector<double> result(n, 0.0);
    if (std::none_of(frame.score_mask.begin(), frame.score_mask.end(), [](uint8_t x) { return x != 0; }))
        return result;
    if (!active) return result;
    DeviceBinding bind(m.device);
    uint32_t batch = std::min(m.rows_per_call(n), v.rows);
    if (m.borrowed) batch = std::min<uint32_t>(batch, uint32_t(m.q_cap / (size_t(m.qheads) * m.dim)));
    m.reserve(batch, n);
    const hipStream_t s = m.stream();
    StreamDrain drain{s};
    hip_ok(hipMemcpyAsync(m.mask, frame.score_mask.data(), n, hipMemcpyHostToDevice, s), "mask H2D");
    bool accumulate = false;
    for (uint32_t l = 0; l < v.layers; ++l) {
        if (!v.layer_rows[l]) continue;
        require(sums.layers[l] != nullptr, "page softmax missing active layer storage");
        m.score_layer(sums.layers[l], query_layer(v, l), v, l, n, batch, agg, active, accumulate, s);
    }
    result = m.fetch(n, s);
    drain.armed = false;
    return result;
}

std::vector<double> PageSoftmaxHip::score(const HostMeanSource &src, PageQueryView v, const QueryScoreFrame &frame,
                                          GqaScoreAggregation aggregation) {
    Impl &m = *impl_;
    const kvr_aggregation agg = to_kvr(aggregation);
    require(src.has && src.read && src.block_tokens && src.width, "page softmax geometry mismatch");
    const uint32_t active = m.check_view(v, src.layers);
    require(uint64_t(v.kv_heads) * v.head_dim == src.width, "page softmax geometry mismatch");
    const size_t n = frame.starts.size();
    require(n && frame.counts.size() == n && frame.score_mask.size() == n, "page softmax geometry mismatch");
    require(n <= std::numeric_limits<uint32_t>::max(), "page softmax geometry exceeds launch addressing");
    // the stored page behind every scored entry: a whole page of the store
    // inside the accepted prefix (page_softmax.cu:239-244)
    std::vector<uint32_t> page(n, 0);
    size_t scored = 0;
    for (size_t i = 0; i < n; ++i) {
        if (!frame.score_mask[i]) continue;
        const uint64_t begin = frame.starts[i], count = frame.counts[i], acc = frame.accepted_through;
        const uint64_t p = begin / src.block_tokens;
        const bool whole = begin % src.block_tokens == 0 && begin < acc && count && count <= acc - begin &&
                           p <= std::numeric_limits<uint32_t>::max() && src.has(uint32_t(p));
        if (!whole) throw std::invalid_argument("page softmax stale index extent");
        page[i] = uint32_t(p);
        ++scored;
    }
    std::vector<double> result(n, 0.0);
    if (!scored || !active) return result;
    const uint32_t pages = uint32_t(n);
    DeviceBinding bind(m.device);
    uint32_t batch = std::min(m.rows_per_call(pages), v.rows);
    if (m.borrowed) batch = std::min<uint32_t>(batch, uint32_t(m.q_cap / (size_t(m.qheads) * m.dim)));
    m.reserve(batch, pages);
    m.reserve_means(pages, src.width);
    const hipStream_t s = m.stream();
    StreamDrain drain{s};
    hip_ok(hipMemcpyAsync(m.mask, frame.score_mask.data(), n, hipMemcpyHostToDevice, s), "mask H2D");
    std::vector<float> host(size_t(pages) * src.width, 0.0f);
    bool accumulate = false;
    for (uint32_t l = 0; l < v.layers; ++l) {
        if (!v.layer_rows[l]) continue;
        // the host buffer is refilled only once the previous layer's copy
        // has been read
        hip_ok(hipStreamSynchronize(s), "hipStreamSynchronize");
        for (size_t i = 0; i < n; ++i)
            if (frame.score_mask[i]) src.read(page[i], l, host.data() + i * src.width);
        hip_ok(hipMemcpyAsync(m.msum, host.data(), host.size() * sizeof(float), hipMemcpyHostToDevice, s),
               "means H2D");
        // means x (1/1) is the mean itself; the finalize rounds it to the
        // fp16 operand and raises non-finite or out-of-range values
        ok(kvr_summary_finalize(m.ctx, m.msum, m.mcount, pages, src.width, nullptr, m.m16, s), "page means");
        m.score_layer(m.m16, query_layer(v, l), v, l, pages, batch, agg, active, accumulate, s);
    }
    result = m.fetch(pages, s);
    drain.armed = false;
    return result;
}

// The native Query's checks that do not depend on where the summaries come
// from: geometry against the scorer, an eager stream, Q on this device and
// the logits budget.
hipStream_t PageSoftmaxHip::Impl::current_layer_stream(const NativeCurrentLayerQuery &q, uint32_t pages,
                                                       void *producer_stream) {
    if (!borrowed) {
        qheads = q.query_heads;
        kvheads = q.kv_heads;
        dim = q.head_dim;
    }
    require(q.query_heads == qheads && q.kv_heads == kvheads && q.head_dim == dim,
            "native Query or score frame geometry mismatch");
    const hipStream_t s = producer_stream ? static_cast<hipStream_t>(producer_stream) : stream();
    if (capturing(s)) throw std::invalid_argument("native Query selection requires an eager stream");
    hipPointerAttribute_t attr{};
    const hipError_t pe = hipPointerGetAttributes(&attr, q.data);
    if (pe != hipSuccess) (void)hipGetLastError();  // unknown to the runtime: ordinary host memory
    if (pe != hipSuccess || attr.type != hipMemoryTypeDevice || attr.device != device)
        throw std::invalid_argument("native Query is not stored on its scoring device");
    if (size_t(q.rows) * q.query_heads * pages * sizeof(double) > kLogitsBudget)
        throw std::length_error("native Query exceeds planned logits range");
    return s;
}

std::vector<double> PageSoftmaxHip::Impl::current_layer(const uint16_t *summaries, const NativeCurrentLayerQuery &q,
                                                        const QueryScoreFrame &frame, hipStream_t s) {
    const uint32_t n = uint32_t(frame.starts.size());
    hip_ok(hipMemcpyAsync(mask, frame.score_mask.data(), n, hipMemcpyHostToDevice, s), "mask H2D");
    kvr_query kq{};
    kq.data = q.data;
    kq.scalar = query_format(q.scalar);
    kq.rows = q.rows;
    kq.query_heads = q.query_heads;
    kq.kv_heads = q.kv_heads;
    kq.head_dim = q.head_dim;
    kq.row_stride = q.row_stride;
    kq.head_stride = q.head_stride;
    kq.dim_stride = q.dimension_stride;
    kq.attention_scale = q.attention_scale;
    ok(kvr_score(ctx, &kq, summaries, 1, n, mask, KVR_AGG_MEAN, 1, 0, scores, 0, s), "page softmax");
    return fetch(n, s);
}

std::vector<double> PageSoftmaxHip::score_current_layer(const PageSummaries &sums, NativeCurrentLayerQuery q,
                                                        const QueryScoreFrame &frame, void *producer_stream) {
    Impl &m = *impl_;
    validate_native_layer_query(q);
    require(q.layer < sums.layers.size() && sums.layers[q.layer], "native Query layer has no summaries");
    DeviceBinding bind(m.device);
    const hipStream_t s = m.current_layer_stream(q, uint32_t(std::min<size_t>(frame.starts.size(), UINT32_MAX)),
                                                 producer_stream);
    m.check_frame(sums, frame);
    m.reserve(0, uint32_t(frame.starts.size()));
    StreamDrain drain{s};
    auto out = m.current_layer(sums.layers[q.layer], q, frame, s);
    drain.armed = false;
    return out;
}

std::vector<double> PageSoftmaxHip::score_current_layer(const HostMeanSource &src, NativeCurrentLayerQuery q,
                                                        const QueryScoreFrame &frame, void *producer_stream) {
    Impl &m = *impl_;
    validate_native_layer_query(q);
    const size_t n = frame.starts.size();
    const uint32_t bt = src.block_tokens;
    if (!src.read || !src.tokens || q.layer >= src.layers || !bt || uint64_t(q.kv_heads) * q.head_dim != src.width ||
        frame.counts.size() != n || frame.score_mask.size() != n || frame.transport_mask.size() != n || !n ||
        n > std::numeric_limits<uint32_t>::max() || uintptr_t(q.data) > UINTPTR_MAX - q.bytes)
        throw std::invalid_argument("native Query or score frame geometry mismatch");
    // every entry must be a whole page of the target layer's Mean-K as the
    // store holds it now (page_softmax.cu:288-298)
    std::vector<uint32_t> page(n);
    for (size_t i = 0; i < n; ++i) {
        const uint64_t start = frame.starts[i], count = frame.counts[i], acc = frame.accepted_through;
        const uint64_t p = start / bt;
        const bool covered = count && count <= bt && start % bt == 0 && start <= acc && count <= acc - start &&
                             p <= std::numeric_limits<uint32_t>::max() && src.tokens(uint32_t(p), q.layer) == count;
        if (!covered)
            throw std::invalid_argument("native target-layer Mean-K coverage differs from frozen frame");
        page[i] = uint32_t(p);
    }
    DeviceBinding bind(m.device);
    const uint32_t pages = uint32_t(n);
    const hipStream_t s = m.current_layer_stream(q, pages, producer_stream);
    m.reserve(0, pages);
    m.reserve_means(pages, src.width);
    std::vector<float> host(size_t(pages) * src.width, 0.0f);
    for (size_t i = 0; i < n; ++i)
        if (frame.score_mask[i]) src.read(page[i], q.layer, host.data() + i * src.width);
    StreamDrain drain{s};
    hip_ok(hipMemcpyAsync(m.msum, host.data(), host.size() * sizeof(float), hipMemcpyHostToDevice, s), "means H2D");
    ok(kvr_summary_finalize(m.ctx, m.msum, m.mcount, pages, src.width, nullptr, m.m16, s), "page means");
    auto out = m.current_layer(m.m16, q, frame, s);
    drain.armed = false;
    return out;
}

namespace {
// Distinct ascending page ids, each below n.
std::vector<uint32_t> distinct_pages(const std::vector<uint32_t> &ids, uint32_t n, const char *what) {
    std::vector<uint32_t> v(ids);
    std::sort(v.begin(), v.end());
    v.erase(std::unique(v.begin(), v.end()), v.end());
    for (uint32_t id : v) require(id < n, what);
    return v;
}

kvr_media media_of(const MediaRanges &media, uint32_t page_tokens, uint64_t total_tokens,
                   std::vector<uint32_t> &flat) {
    flat.clear();
    for (const auto &r : media) {
        flat.push_back(r.first);
        flat.push_back(r.second);
    }
    kvr_media m{};
    m.ranges = flat.data();
    m.n_ranges = uint32_t(media.size());
    m.page_tokens = page_tokens;
    m.total_tokens = total_tokens;
    return m;
}

kvr_tie_rule tie_of(TieRule t) { return t == TieRule::HigherFirst ? KVR_TIE_HIGHER_FIRST : KVR_TIE_LOWER_FIRST; }
}  // namespace

std::vector<uint32_t> query_fixed_blocks(uint32_t pages, uint32_t budget, uint32_t sink, uint32_t recent,
                                         const MediaRanges &media, uint32_t page_tokens, uint64_t total_tokens,
                                         const std::vector<uint32_t> &mandatory) {
    require(page_tokens, "page_tokens must be nonzero");
    std::vector<uint32_t> flat;
    const kvr_media m = media_of(media, page_tokens, total_tokens, flat);
    std::vector<uint32_t> out(std::max<uint32_t>(pages, 1));
    uint32_t n = 0;
    ok(kvr_query_fixed_pages(pages, budget, sink, recent, &m, mandatory.data(), uint32_t(mandatory.size()),
                             out.data(), &n),
       "query fixed pages");
    out.resize(n);
    return out;
}

// Reads back a device selection of up to k pages; operand and budget
// errors of the device pick come back as the reference's exceptions.
std::vector<uint32_t> PageSoftmaxHip::fetch_pick(const uint32_t *sel, const uint32_t *cnt, uint32_t k, void *stream,
                                                 const char *what) {
    Impl &m = *impl_;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    std::vector<uint32_t> out(k);
    uint32_t count = 0;
    hip_ok(hipMemcpyAsync(out.data(), sel, size_t(k) * 4, hipMemcpyDeviceToHost, s), "selection D2H");
    hip_ok(hipMemcpyAsync(&count, cnt, 4, hipMemcpyDeviceToHost, s), "count D2H");
    hip_ok(hipStreamSynchronize(s), "hipStreamSynchronize");
    const kvr_status st = kvr_check(m.ctx, s);
    if (st == KVR_ERR_SCORES) throw std::invalid_argument("scores must be finite and non-negative");
    ok(st, what);
    out.resize(count);
    return out;
}

std::vector<uint32_t> PageSoftmaxHip::pick(const std::vector<double> &scores, uint32_t budget,
                                           const std::vector<uint32_t> &mandatory, TieRule tie,
                                           bool signed_scores) {
    return pick(scores, budget, mandatory, tie, signed_scores, {}, 1);
}

std::vector<uint32_t> PageSoftmaxHip::pick(const std::vector<double> &scores, uint32_t budget,
                                           const std::vector<uint32_t> &mandatory, TieRule tie, bool signed_scores,
                                           const MediaRanges &media, uint32_t page_tokens) {
    Impl &m = *impl_;
    const uint32_t n = uint32_t(scores.size());
    require(budget, "invalid scored selection frame (budget 0)");
    require(page_tokens, "page_tokens must be nonzero");
    if (!n) return {};
    const std::vector<uint32_t> mand = distinct_pages(mandatory, n, "mandatory page outside the scored index");
    const uint32_t k = std::min(budget, n);
    DeviceBinding bind(m.device);
    m.reserve(0, n);
    const hipStream_t s = m.stream();
    StreamDrain drain{s};
    hip_ok(hipMemcpyAsync(m.scores, scores.data(), size_t(n) * 8, hipMemcpyHostToDevice, s), "scores H2D");
    std::vector<uint32_t> flat, groups(2 * std::max<size_t>(media.size(), 1));
    uint32_t n_groups = 0;
    if (!media.empty()) {
        const kvr_media md = media_of(media, page_tokens, uint64_t(n) * page_tokens, flat);
        ok(kvr_media_page_groups(&md, n, KVR_MEDIA_OVERLAP, groups.data(), &n_groups), "media groups");
    }
    if (!n_groups) {
        if (mand.size() > budget)
            throw std::runtime_error("mandatory scored content is cold, incomplete or exceeds budget");
        ok(kvr_select_topk(m.ctx, m.scores, 1, n, k, mand.data(), uint32_t(mand.size()), tie_of(tie), signed_scores,
                           m.sel, m.cnt, s),
           "pick scored blocks");
    } else {
        hip_ok(hipMemcpyAsync(m.groups, groups.data(), size_t(n_groups) * 8, hipMemcpyHostToDevice, s), "groups H2D");
        if (!mand.empty())
            hip_ok(hipMemcpyAsync(m.fixed, mand.data(), mand.size() * 4, hipMemcpyHostToDevice, s), "fixed H2D");
        kvr_page_policy pol{};
        pol.fixed = m.fixed;
        pol.n_fixed = uint32_t(mand.size());
        pol.groups = m.groups;
        pol.n_groups = n_groups;
        ok(kvr_select_pages(m.ctx, m.scores, 1, n, k, &pol, tie_of(tie), signed_scores, m.sel, m.cnt, s),
           "pick scored blocks");
    }
    auto out = fetch_pick(m.sel, m.cnt, k, s, "pick scored blocks");
    drain.armed = false;
    return out;
}

std::vector<uint32_t> PageSoftmaxHip::pick_topk(const std::vector<double> &scores, uint32_t budget, uint32_t sink,
                                                uint32_t recent, const std::vector<uint32_t> &mandatory,
                                                const MediaRanges &media, uint32_t page_tokens,
                                                uint64_t total_tokens) {
    Impl &m = *impl_;
    const uint32_t n = uint32_t(scores.size());
    require(page_tokens, "page_tokens must be nonzero");
    if (!n) return {};
    if (!budget || n <= budget) {
        std::vector<uint32_t> all(n);
        for (uint32_t i = 0; i < n; ++i) all[i] = i;
        return all;
    }
    // pick_topk_ungrouped: the kept pages on the host, the fill on the device
    std::vector<uint32_t> kept(n);
    uint32_t n_kept = 0;
    ok(kvr_topk_fixed_pages(n, budget, sink, recent, mandatory.data(), uint32_t(mandatory.size()), kept.data(),
                            &n_kept),
       "top-k fixed pages");
    DeviceBinding bind(m.device);
    m.reserve(0, n);
    const hipStream_t s = m.stream();
    StreamDrain drain{s};
    hip_ok(hipMemcpyAsync(m.scores, scores.data(), size_t(n) * 8, hipMemcpyHostToDevice, s), "scores H2D");
    if (n_kept)
        hip_ok(hipMemcpyAsync(m.fixed, kept.data(), size_t(n_kept) * 4, hipMemcpyHostToDevice, s), "fixed H2D");
    kvr_page_policy first{};
    first.fixed = m.fixed;
    first.n_fixed = n_kept;
    ok(kvr_select_pages(m.ctx, m.scores, 1, n, budget, &first, KVR_TIE_HIGHER_FIRST, 1, m.sel, m.cnt, s),
       "pick top-k blocks");
    if (media.empty()) {
        auto out = fetch_pick(m.sel, m.cnt, budget, s, "pick top-k blocks");
        drain.armed = false;
        return out;
    }
    // constrain_media: the ungrouped pick's pages first, media groups whole
    std::vector<uint32_t> flat, groups(2 * media.size());
    const kvr_media md = media_of(media, page_tokens, total_tokens, flat);
    uint32_t n_groups = 0, n_fixed = 0;
    std::vector<uint32_t> fixed(n);
    ok(kvr_media_page_groups(&md, n, KVR_MEDIA_IN_ORDER, groups.data(), &n_groups), "media groups");
    ok(kvr_media_fixed_pages(n, budget, sink, &md, mandatory.data(), uint32_t(mandatory.size()), fixed.data(),
                             &n_fixed),
       "media fixed pages");
    hip_ok(hipStreamSynchronize(s), "hipStreamSynchronize");  // m.fixed is rewritten below
    if (n_groups)
        hip_ok(hipMemcpyAsync(m.groups, groups.data(), size_t(n_groups) * 8, hipMemcpyHostToDevice, s), "groups H2D");
    if (n_fixed)
        hip_ok(hipMemcpyAsync(m.fixed, fixed.data(), size_t(n_fixed) * 4, hipMemcpyHostToDevice, s), "fixed H2D");
    kvr_page_policy second{};
    second.fixed = m.fixed;
    second.n_fixed = n_fixed;
    second.groups = m.groups;
    second.n_groups = n_groups;
    second.preferred = m.sel;
    second.preferred_count = m.cnt;
    second.preferred_stride = budget;
    ok(kvr_select_pages(m.ctx, m.scores, 1, n, budget, &second, KVR_TIE_HIGHER_FIRST, 1, m.sel2, m.cnt2, s),
       "pick top-k blocks");
    auto out = fetch_pick(m.sel2, m.cnt2, budget, s, "pick top-k blocks");
    drain.armed = false;
    return out;
}

// ---- native payload records -------------------------------------------------
namespace {
void plan_require(bool cond, const char *msg) {
    if (!cond) throw MemoryError(MemoryErrorCode::InvalidPlan, msg);
}
uint64_t plan_add(uint64_t a, uint64_t b) {
    uint64_t r;
    plan_require(!__builtin_add_overflow(a, b, &r), "memory size/position overflow");
    return r;
}
uint64_t plan_mul(uint64_t a, uint64_t b) {
    uint64_t r;
    plan_require(!__builtin_mul_overflow(a, b, &r), "memory size overflow");
    return r;
}
bool pow2(uint64_t n) { return n && !(n & (n - 1)); }
// bytes of one token row of a gather source format (0: not a source format)
size_t source_row_bytes(kvr_format f, uint32_t width) {
    if (f == KVR_FMT_F16) return size_t(width) * 2;
    if (width % 32) return 0;
    if (f == KVR_FMT_Q8_0) return size_t(width) / 32 * 34;
    if (f == KVR_FMT_Q4_1) return size_t(width) / 32 * 20;
    if (f == KVR_FMT_Q4_0) return size_t(width) / 32 * 18;
    return 0;
}
}  // namespace

// Rules of a record layout (memory_contract.cpp:51-101), checked plane by
// plane in list order and then shard by shard; the first broken rule throws
// std::invalid_argument with its message.
//  R1 header: format, version, block_tokens, record_bytes and at least one
//     plane; the alignment a power of two dividing record_bytes.
//  R2 a plane has bytes, a power-of-two alignment no larger than the
//     record's, an aligned offset, starts at or after the previous plane's
//     end, and its kind appears once in its shard (layer, rank).
//  R3 a head range is [begin, begin+count) within uint32; count 0 means
//     "all heads" and then begins at 0.
//  R4 every plane of a shard carries the shard's head range.
//  R5 a packed key+value plane has no token rows (token_stride 0).
//  R6 a plane ends inside the record, and block_tokens token rows fit it.
//  R7 a shard holds one packed key+value plane alone, or a key and a value
//     plane (scale planes optional).
//  R8 a layer's shards, by rank, tile its heads from 0 without gaps; a shard
//     of "all heads" is its layer's only shard.
namespace {
struct PayloadShard {
    uint32_t layer, rank, head_begin, head_count;
    unsigned kinds;  // bit per PayloadPlaneKind
};
constexpr unsigned kind_bit(PayloadPlaneKind k) { return 1u << unsigned(k); }
constexpr unsigned kKnownKinds = kind_bit(PayloadPlaneKind::Key) | kind_bit(PayloadPlaneKind::Value) |
                                 kind_bit(PayloadPlaneKind::KeyScale) | kind_bit(PayloadPlaneKind::ValueScale) |
                                 kind_bit(PayloadPlaneKind::PackedKeyValue);
}  // namespace

void PayloadLayout::validate() const {
    const bool header = !format.empty() && version != 0 && block_tokens != 0 && record_bytes != 0 &&
                        !planes.empty() && pow2(alignment) && record_bytes % alignment == 0;
    plan_require(header, "invalid native payload layout");

    std::vector<PayloadShard> shards;  // in order of first appearance
    auto shard_of = [&](const PayloadPlane &p) -> PayloadShard * {
        for (auto &s : shards)
            if (s.layer == p.layer && s.rank == p.rank) return &s;
        return nullptr;
    };
    uint64_t cursor = 0;  // end of the previous plane
    for (const PayloadPlane &p : planes) {
        const unsigned bit = unsigned(p.kind) < 32 ? 1u << unsigned(p.kind) : 0;
        PayloadShard *s = shard_of(p);
        const bool placed = p.bytes != 0 && pow2(p.alignment) && p.alignment <= alignment &&
                            p.offset % p.alignment == 0 && p.offset >= cursor;
        plan_require(placed && !(s && (s->kinds & bit)), "overlapping/duplicate/misaligned payload plane");
        plan_require(p.head_count != 0 ? uint64_t(p.head_begin) + p.head_count <= std::numeric_limits<uint32_t>::max()
                                  : p.head_begin == 0,
                "invalid payload head range");
        if (!s) {
            shards.push_back({p.layer, p.rank, p.head_begin, p.head_count, 0});
            s = &shards.back();
        }
        plan_require(s->head_begin == p.head_begin && s->head_count == p.head_count,
                "a payload shard has inconsistent head ranges");
        plan_require((bit & kKnownKinds) != 0, "unknown payload plane kind");
        s->kinds |= bit;
        plan_require(p.kind != PayloadPlaneKind::PackedKeyValue || p.token_stride == 0,
                "packed KV pages require opaque token addressing");
        cursor = plan_add(p.offset, p.bytes);
        // the record bound is checked before the rows' size is computed: a
        // plane past the record reports that, even when its rows overflow
        const bool inside = cursor <= record_bytes;
        plan_require(inside && (p.token_stride == 0 || plan_mul(p.token_stride, block_tokens) <= p.bytes),
                     "payload plane exceeds its record");
    }

    std::sort(shards.begin(), shards.end(), [](const PayloadShard &a, const PayloadShard &b) {
        return a.layer != b.layer ? a.layer < b.layer : a.rank < b.rank;
    });
    const unsigned kv = kind_bit(PayloadPlaneKind::Key) | kind_bit(PayloadPlaneKind::Value);
    for (const PayloadShard &s : shards) {
        const unsigned packed = kind_bit(PayloadPlaneKind::PackedKeyValue);
        plan_require(s.kinds == packed || ((s.kinds & kv) == kv && (s.kinds & packed) == 0),
                "every attention layer requires key and value planes");
    }
    for (size_t first = 0; first < shards.size();) {
        size_t last = first;
        while (last + 1 < shards.size() && shards[last + 1].layer == shards[first].layer) ++last;
        uint64_t covered = 0;  // heads [0, covered) tiled so far
        for (size_t i = first; i <= last; ++i) {
            if (i > first)
                plan_require(shards[i - 1].head_count != 0 && shards[i].head_count != 0,
                        "multiple payload shards need explicit head ranges");
            plan_require(shards[i].head_begin == covered, "payload heads must cover a contiguous model-order range");
            covered += shards[i].head_count;
        }
        first = last + 1;
    }
}

kvr_plane record_plane(const PayloadLayout &layout, uint32_t layer, PayloadPlaneKind kind, const void *archive,
                       kvr_format format, uint32_t width, uint64_t tokens, kvr_gather_mode mode, void *slots,
                       uint32_t rank) {
    layout.validate();
    require(kind == PayloadPlaneKind::Key || kind == PayloadPlaneKind::Value,
            "only key and value planes are gathered as token rows");
    const PayloadPlane *plane = nullptr;
    for (const auto &p : layout.planes)
        if (p.layer == layer && p.kind == kind && p.rank == rank) plane = &p;
    require(plane != nullptr, "the payload layout has no such plane");
    const size_t row = source_row_bytes(format, width);
    require(row && plane->token_stride == row, "the payload plane's token rows are not contiguous rows of the format");
    kvr_plane out{};
    out.history = static_cast<const uint8_t *>(archive) + plane->offset;
    out.format = format;
    out.width = width;
    out.tokens = tokens;
    out.mode = mode;
    out.slots = slots;
    out.page_stride = layout.record_bytes;
    return out;
}

// ---- graph propagation and LRFU -------------------------------------------
std::vector<double> span_coefficients(const std::vector<GraphMessageSpan> &spans, uint32_t block_tokens,
                                      uint32_t pages, double cross) {
    require(block_tokens != 0, "invalid block size");
    require(std::isfinite(cross) && cross >= 0 && cross <= 1, "invalid attention decay");
    std::vector<std::pair<uint64_t, uint64_t>> by_begin;  // (begin, end) sorted by begin
    std::vector<uint64_t> begins, known_ends;
    for (const auto &sp : spans) {
        by_begin.push_back({sp.begin, sp.end});
        begins.push_back(sp.begin);
        if (sp.end_known) known_ends.push_back(sp.end);
    }
    std::sort(by_begin.begin(), by_begin.end());
    std::sort(begins.begin(), begins.end());
    std::sort(known_ends.begin(), known_ends.end());
    std::vector<uint64_t> reach(by_begin.size());  // max end over spans [0, i]
    for (size_t i = 0; i < by_begin.size(); ++i)
        reach[i] = std::max(by_begin[i].second, i ? reach[i - 1] : 0);
    // some value of a sorted list strictly inside (lo, hi)
    auto inside = [](const std::vector<uint64_t> &v, uint64_t lo, uint64_t hi) {
        const auto it = std::upper_bound(v.begin(), v.end(), lo);
        return it != v.end() && *it < hi;
    };
    std::vector<double> out(pages > 1 ? pages - 1 : 0, 1.0);
    for (uint32_t i = 0; i + 1 < pages; ++i) {
        const uint64_t begin = uint64_t(i) * block_tokens, end = uint64_t(i + 2) * block_tokens;
        // a span holding both pages: among spans beginning at or before
        // `begin`, the furthest end reaches `end`
        const auto k = std::upper_bound(by_begin.begin(), by_begin.end(),
                                        std::make_pair(begin, std::numeric_limits<uint64_t>::max())) -
                       by_begin.begin();
        if (k && reach[k - 1] >= end) continue;
        if (inside(begins, begin, end) || inside(known_ends, begin, end)) out[i] = cross;
    }
    return out;
}

struct GraphRecallHip::Impl {
    int device = 0;
    kvr_context *ctx = nullptr;
    double *scores = nullptr, *hist = nullptr, *nw = nullptr, *mass = nullptr;
    uint8_t *mask = nullptr;
    uint32_t *src = nullptr, *begin = nullptr, *target = nullptr;
    size_t page_cap = 0, row_cap = 0, edge_cap = 0;
    ~Impl() {
        if (ctx) {
            (void)hipSetDevice(device);
            (void)kvr_check(ctx, nullptr);
        }
        for (void *p : {(void *)scores, (void *)hist, (void *)nw, (void *)mask, (void *)src, (void *)begin,
                        (void *)target, (void *)mass})
            if (p) (void)hipFree(p);
        if (ctx) (void)kvr_destroy(ctx);
    }
    // replaces p with a device array of n elements (contents not kept)
    template <class T> static void realloc_dev(T *&p, size_t n) {
        if (p) hip_ok(hipFree(p), "hipFree");
        p = nullptr;
        hip_ok(hipMalloc(reinterpret_cast<void **>(&p), std::max<size_t>(n, 1) * sizeof(T)), "hipMalloc");
    }
    void pages(size_t n) {
        if (n <= page_cap) return;
        realloc_dev(scores, n);
        realloc_dev(hist, n);
        realloc_dev(nw, n);
        realloc_dev(mask, n);
        page_cap = n;
    }
    void rows(size_t r, size_t e) {
        if (r + 1 > row_cap) {
            realloc_dev(src, r + 1);
            realloc_dev(begin, r + 1);
            row_cap = r + 1;
        }
        if (e > edge_cap) {
            realloc_dev(target, e);
            realloc_dev(mass, e);
            edge_cap = e;
        }
    }
    hipStream_t stream() const { return static_cast<hipStream_t>(kvr_select_stream(ctx)); }
};

GraphRecallHip::GraphRecallHip(int device) : impl_(new Impl) {
    impl_->device = device;
    ok(kvr_create(device, &impl_->ctx), "kvr_create");
}
GraphRecallHip::~GraphRecallHip() = default;
kvr_context *GraphRecallHip::context() const { return impl_->ctx; }

std::vector<double> GraphRecallHip::propagate_query_scores(const std::vector<double> &raw,
                                                           const QueryScoreFrame &frame, const GraphView &graph,
                                                           double alpha, double cross) {
    Impl &m = *impl_;
    require(std::isfinite(alpha) && alpha >= 0 && alpha <= 1 && std::isfinite(cross) && cross >= 0 && cross <= 1,
            "invalid attention decay");
    const size_t n = raw.size();
    const uint32_t bt = graph.block_tokens;
    require(bt && frame.starts.size() == n && frame.transport_mask.size() == n &&
                graph.accepted_through == frame.accepted_through,
            "graph and Query have different accepted prefixes");
    for (size_t i = 0; i < n; ++i)
        require(frame.starts[i] == uint64_t(i) * bt, "invalid or duplicate Query graph identity");
    if (!n) return raw;
    if (n > KVR_GRAPH_MAX_PAGES) throw std::length_error("Query frame exceeds KVR_GRAPH_MAX_PAGES pages");
    // the rows propagation reads, by page; targets that are no page of the
    // frame stay as non-nodes so their masses are still checked
    std::vector<uint32_t> src, begin{0}, target;
    std::vector<double> mass;
    for (const auto *chunk : graph.chunks)
        for (const auto &row : *chunk) {
            if (!row.samples || row.source + bt > graph.completed_through || row.source % bt) continue;
            const uint64_t sp = row.source / bt;
            if (sp >= n) continue;
            src.push_back(uint32_t(sp));
            for (const auto &e : row.edges) {
                const uint64_t tp = e.target % bt ? UINT32_MAX : std::min<uint64_t>(e.target / bt, UINT32_MAX);
                target.push_back(uint32_t(tp));
                mass.push_back(e.mass);
            }
            begin.push_back(uint32_t(target.size()));
        }
    std::vector<double> nw;
    if (graph.messages) nw = span_coefficients(*graph.messages, bt, uint32_t(n), cross);
    DeviceBinding bind(m.device);
    m.pages(n);
    m.rows(src.size(), target.size());
    const hipStream_t s = m.stream();
    StreamDrain drain{s};
    hip_ok(hipMemcpyAsync(m.scores, raw.data(), n * 8, hipMemcpyHostToDevice, s), "scores H2D");
    hip_ok(hipMemcpyAsync(m.mask, frame.transport_mask.data(), n, hipMemcpyHostToDevice, s), "mask H2D");
    kvr_page_graph g{};
    g.n_rows = uint32_t(src.size());
    g.n_edges = uint32_t(target.size());
    if (g.n_rows) {
        hip_ok(hipMemcpyAsync(m.src, src.data(), src.size() * 4, hipMemcpyHostToDevice, s), "rows H2D");
        hip_ok(hipMemcpyAsync(m.begin, begin.data(), begin.size() * 4, hipMemcpyHostToDevice, s), "rows H2D");
        g.row_source = m.src;
        g.row_begin = m.begin;
    }
    if (g.n_edges) {
        hip_ok(hipMemcpyAsync(m.target, target.data(), target.size() * 4, hipMemcpyHostToDevice, s), "edges H2D");
        hip_ok(hipMemcpyAsync(m.mass, mass.data(), mass.size() * 8, hipMemcpyHostToDevice, s), "edges H2D");
        g.edge_target = m.target;
        g.edge_mass = m.mass;
    }
    if (!nw.empty()) {
        hip_ok(hipMemcpyAsync(m.nw, nw.data(), nw.size() * 8, hipMemcpyHostToDevice, s), "weights H2D");
        g.neighbor_weight = m.nw;
    }
    ok(kvr_propagate_scores(m.ctx, m.scores, 1, uint32_t(n), m.mask, &g, alpha, s), "propagate Query scores");
    std::vector<double> out(n);
    hip_ok(hipMemcpyAsync(out.data(), m.scores, n * 8, hipMemcpyDeviceToHost, s), "scores D2H");
    hip_ok(hipStreamSynchronize(s), "hipStreamSynchronize");
    drain.armed = false;
    const kvr_status st = kvr_check(m.ctx, s);
    if (st == KVR_ERR_SCORES) throw std::invalid_argument("nonfinite Query graph seed");
    if (st == KVR_ERR_GRAPH) throw std::invalid_argument("invalid attention mass or graph propagation result");
    ok(st, "propagate Query scores");
    return out;
}

std::vector<double> GraphRecallHip::lrfu_candidate(const std::vector<double> &scores,
                                                   const std::vector<double> &committed, double lambda,
                                                   double top_fraction) {
    Impl &m = *impl_;
    const size_t n = scores.size();
    if (!n) return {};
    if (n > KVR_GRAPH_MAX_PAGES) throw std::length_error("LRFU frame exceeds KVR_GRAPH_MAX_PAGES pages");
    const size_t nh = std::min(committed.size(), n);
    DeviceBinding bind(m.device);
    m.pages(n);
    const hipStream_t s = m.stream();
    StreamDrain drain{s};
    hip_ok(hipMemcpyAsync(m.scores, scores.data(), n * 8, hipMemcpyHostToDevice, s), "scores H2D");
    if (nh) hip_ok(hipMemcpyAsync(m.hist, committed.data(), nh * 8, hipMemcpyHostToDevice, s), "history H2D");
    ok(kvr_lrfu_preview(m.ctx, m.scores, 1, uint32_t(n), nh ? m.hist : nullptr, uint32_t(nh), lambda, top_fraction,
                        m.scores, s),
       "LRFU preview");
    std::vector<double> out(n);
    hip_ok(hipMemcpyAsync(out.data(), m.scores, n * 8, hipMemcpyDeviceToHost, s), "candidate D2H");
    hip_ok(hipStreamSynchronize(s), "hipStreamSynchronize");
    drain.armed = false;
    const kvr_status st = kvr_check(m.ctx, s);
    if (st == KVR_ERR_SCORES) throw std::invalid_argument("nonfinite LRFU retrieval score");
    ok(st, "LRFU preview");
    return out;
}

// LRFU history (lrfu.hpp:43-101), as rules:
//  - lambda is a decay in [0, 1], the hit fraction in (0, 1];
//  - a round is opened by begin_round (its counter never wraps) and closed
//    by its one commit; a candidate is derived from the committed scores
//    only, so repeated previews in a round replace each other;
//  - preview outside any round is a logic error, after the round's commit a
//    no-op, and an empty score list withdraws the candidate;
//  - reads see the candidate while there is one, else the committed
//    scores, and 0 past their end;
//  - a checkpoint is the committed state (shared, never copied); one from
//    before the first round holds nothing, and restored scores are finite.
namespace {
bool unit_interval(double x, bool open_low) { return std::isfinite(x) && (open_low ? x > 0 : x >= 0) && x <= 1; }
void check_lrfu_checkpoint(const LrfuState &cp) {
    const bool before_rounds = cp.round == 0;
    if (!cp.scores || (before_rounds && (cp.committed || !cp.scores->empty())))
        throw std::invalid_argument("invalid LRFU checkpoint");
    if (std::any_of(cp.scores->begin(), cp.scores->end(), [](double v) { return !std::isfinite(v); }))
        throw std::invalid_argument("nonfinite LRFU checkpoint");
}
}  // namespace

LrfuHistoryHip::LrfuHistoryHip(GraphRecallHip &device, double lambda, double top_fraction)
    : device_(&device), lambda_(lambda), fraction_(top_fraction) {
    if (!unit_interval(lambda, false) || !unit_interval(top_fraction, true))
        throw std::invalid_argument("invalid LRFU decay or hit fraction");
}
void LrfuHistoryHip::begin_round() {
    if (state_.round == std::numeric_limits<uint64_t>::max()) {
        state_.round = 0;  // the counter wrapped, as an increment would leave it
        throw std::overflow_error("LRFU round overflow");
    }
    state_ = LrfuState{state_.scores, state_.round + 1, false};
    candidate_.reset();
}
void LrfuHistoryHip::preview(const std::vector<double> &scores) {
    const bool open = state_.round != 0 && !state_.committed;
    if (!open) {
        if (state_.round == 0 && !state_.committed) throw std::logic_error("LRFU probe outside a round");
        return;
    }
    if (scores.empty())
        candidate_ = nullptr;
    else
        candidate_ = std::make_shared<const std::vector<double>>(
            device_->lrfu_candidate(scores, *state_.scores, lambda_, fraction_));
}
bool LrfuHistoryHip::commit() noexcept {
    const bool can = candidate_ != nullptr && !state_.committed;
    if (can) {
        state_.committed = true;
        state_.scores.swap(candidate_);
        candidate_ = nullptr;
    }
    return can;
}
double LrfuHistoryHip::score(size_t block) const noexcept {
    const std::vector<double> &seen = candidate_ ? *candidate_ : *state_.scores;
    return block >= seen.size() ? 0.0 : seen[block];
}
void LrfuHistoryHip::restore(const LrfuState &state) {
    check_lrfu_checkpoint(state);
    candidate_ = nullptr;
    state_ = state;
}

size_t PageSoftmaxHip::device_bytes() const {
    size_t b = kvr_device_bytes(impl_->ctx);
    if (!impl_->borrowed)
        b += impl_->q_cap * sizeof(float) + (impl_->page_cap ? impl_->page_cap * 13 + 256 : 0) +
             impl_->mean_cap * 6 + size_t(impl_->mean_pages) * 4;
    return b;
}

kvr_context *PageSoftmaxHip::context() const { return impl_->ctx; }

// ---------------------------------------------------------------------------
// Stage-in entry points.
struct kvmem_gpu_state {
    kvr_context *ctx = nullptr;
    // two pinned slabs: one fills while the other's copy is in flight
    static constexpr size_t kSlab = size_t(32) << 20;
    uint8_t *slab[2] = {nullptr, nullptr};
    hipEvent_t slab_done[2] = {nullptr, nullptr};
    bool slab_busy[2] = {false, false};
    int cur = 0;
    size_t used = 0;
    std::vector<const void *> src;
    std::vector<void *> dst;
    std::vector<size_t> bytes;
    // raw K records of the current slab: each is one gather launch on flush
    struct KRecord {
        const uint8_t *rows;
        uint8_t *dst;
        kvr_format ty;
        uint32_t nt, n_embd, nrot, head_dim, n_rot;
        int32_t pos0;
    };
    std::vector<KRecord> krec;
    float *theta = nullptr;         // device copy of the rotation angles
    std::vector<float> theta_host;  // what it holds
    uint32_t *sel = nullptr;        // device {0, 1}: page 0, one page
    // stage-out records of the current slot: (device source, slot offset, bytes)
    std::vector<const void *> out_src;
    std::vector<size_t> out_off, out_bytes;
    size_t out_used = 0;
    int out_cur = 0;
    hipEvent_t out_done[2] = {nullptr, nullptr};
    // decode running mean-K
    float *acc = nullptr;
    uint32_t *acc_count = nullptr;
    uint32_t n_layer = 0, n_embd = 0;
    std::vector<uint64_t> acc_pos;
};

namespace {
thread_local kvmem_gpu_state *g_state = nullptr;

bool report(const char *what, const char *detail) {
    std::fprintf(stderr, "kvmem stage-in: %s: %s\n", what, detail);
    return false;
}
bool report_kvr(const char *what) { return report(what, kvr_last_error()); }
bool report_hip(const char *what, hipError_t e) { return report(what, hipGetErrorString(e)); }

hipStream_t copy_stream(kvmem_gpu_state *st) { return static_cast<hipStream_t>(kvr_copy_stream(st->ctx)); }

void release_slabs(kvmem_gpu_state *st) {
    for (int i = 0; i < 2; ++i) {
        if (st->slab_done[i]) {
            (void)hipEventSynchronize(st->slab_done[i]);
            (void)hipEventDestroy(st->slab_done[i]);
            st->slab_done[i] = nullptr;
        }
        if (st->slab[i]) (void)kvr_host_free(st->slab[i]);
        st->slab[i] = nullptr;
        st->slab_busy[i] = false;
    }
    st->used = 0;
    st->src.clear();
    st->dst.clear();
    st->bytes.clear();
    st->krec.clear();
    st->out_src.clear();
    st->out_off.clear();
    st->out_bytes.clear();
    st->out_used = 0;
    for (int i = 0; i < 2; ++i) {
        if (st->out_done[i]) (void)hipEventDestroy(st->out_done[i]);
        st->out_done[i] = nullptr;
    }
    if (st->theta) (void)hipFree(st->theta);
    if (st->sel) (void)hipFree(st->sel);
    st->theta = nullptr;
    st->sel = nullptr;
    st->theta_host.clear();
}

int64_t micros_since(std::chrono::steady_clock::time_point t0) {
    return std::chrono::duration_cast<std::chrono::microseconds>(std::chrono::steady_clock::now() - t0).count();
}
}  // namespace

kvmem_gpu_state *kvmem_gpu_state_create() {
    auto *st = new kvmem_gpu_state;
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || kvr_create(device, &st->ctx) != KVR_OK) {
        report_kvr("state create");
        delete st;
        return nullptr;
    }
    if (!g_state) g_state = st;
    return st;
}

void kvmem_gpu_state_free(kvmem_gpu_state *st) {
    if (!st) return;
    if (st->ctx) (void)kvr_check(st->ctx, nullptr);
    release_slabs(st);
    if (st->acc) (void)hipFree(st->acc);
    if (st->acc_count) (void)hipFree(st->acc_count);
    if (st->ctx) (void)kvr_destroy(st->ctx);
    if (g_state == st) g_state = nullptr;
    delete st;
}

void kvmem_gpu_state_make_current(kvmem_gpu_state *st) { g_state = st; }

bool kvmem_stagein_gpu_ready(size_t, size_t) {
    if (!g_state && !kvmem_gpu_state_create()) return false;
    kvmem_gpu_state *st = g_state;
    for (int i = 0; i < 2; ++i) {
        if (st->slab[i]) continue;
        void *p = nullptr;
        if (kvr_host_alloc(kvmem_gpu_state::kSlab, &p) != KVR_OK) return report_kvr("pinned slab");
        st->slab[i] = static_cast<uint8_t *>(p);
        if (hipError_t e = hipEventCreateWithFlags(&st->slab_done[i], hipEventDisableTiming); e != hipSuccess)
            return report_hip("slab event", e);
    }
    return true;
}

void kvmem_stagein_gpu_free() {
    if (!g_state) return;
    kvmem_stagein_sync();
    release_slabs(g_state);
}

bool kvmem_stagein_h2d_bytes(void *gpu_dst, const void *host, size_t n) {
    if (!g_state || !gpu_dst || !host) return report("h2d", "stage-in is not ready or a pointer is null");
    if (!n) return true;
    const hipStream_t s = copy_stream(g_state);
    if (hipError_t e = hipMemcpyAsync(gpu_dst, host, n, hipMemcpyHostToDevice, s); e != hipSuccess)
        return report_hip("h2d", e);
    if (hipError_t e = hipStreamSynchronize(s); e != hipSuccess) return report_hip("h2d fence", e);
    return true;
}

void kvmem_stagein_sync() {
    if (g_state) (void)hipStreamSynchronize(copy_stream(g_state));
}

bool kvmem_stagein_sync_checked() {
    if (!g_state) return report("sync", "stage-in is not ready");
    if (kvr_check(g_state->ctx, kvr_copy_stream(g_state->ctx)) != KVR_OK) return report_kvr("sync");
    return true;
}

bool kvmem_stagein_flush(int64_t *copy_us, int64_t *rope_us, int64_t *hadamard_us, int64_t *set_us) {
    const auto t0 = std::chrono::steady_clock::now();
    if (rope_us) *rope_us = 0;
    if (hadamard_us) *hadamard_us = 0;
    kvmem_gpu_state *st = g_state;
    if (!st) return report("flush", "stage-in is not ready");
    if (st->src.empty() && st->krec.empty()) return true;
    const hipStream_t s = copy_stream(st);
    // one launch moves every queued V record from the pinned slab to its rows
    if (!st->src.empty() &&
        kvr_d2d_batched(st->ctx, st->src.data(), st->dst.data(), st->bytes.data(), uint32_t(st->src.size()), s) !=
            KVR_OK)
        return report_kvr("flush");
    // each raw K record: one gather launch reading the slab over the host
    // link, transforming and writing its rows (dequant, RoPE, Walsh-Hadamard
    // and quant in one pass)
    const auto tk = std::chrono::steady_clock::now();
    for (const auto &r : st->krec) {
        kvr_rope rope{};
        rope.head_dim = r.head_dim;
        rope.n_rot = r.n_rot;
        rope.theta = st->theta;
        rope.fwht = r.nrot;
        rope.pos_base = r.pos0;
        kvr_plane plane{};
        plane.history = r.rows;
        plane.format = r.ty;
        plane.width = r.n_embd;
        plane.tokens = r.nt;
        plane.mode = KVR_GATHER_ROPE_FWHT;
        plane.slots = r.dst;
        plane.rope = &rope;
        if (kvr_stage_in(st->ctx, &plane, 1, 1, r.nt, st->sel, st->sel + 1, 1, KVR_ENGINE_KERNEL, s) != KVR_OK) {
            st->krec.clear();
            return report_kvr("flush raw K");
        }
    }
    const bool had_k = !st->krec.empty();
    st->krec.clear();
    if (had_k && rope_us) *rope_us += micros_since(tk);
    if (hipError_t e = hipEventRecord(st->slab_done[st->cur], s); e != hipSuccess) return report_hip("flush", e);
    st->slab_busy[st->cur] = true;
    st->src.clear();
    st->dst.clear();
    st->bytes.clear();
    st->used = 0;
    st->cur ^= 1;
    if (st->slab_busy[st->cur]) {
        // the other slab's copy must have read it before it is refilled
        if (hipError_t e = hipEventSynchronize(st->slab_done[st->cur]); e != hipSuccess)
            return report_hip("slab reuse", e);
        st->slab_busy[st->cur] = false;
    }
    if (copy_us) *copy_us += micros_since(t0);
    (void)set_us;  // the copy is the set: no separate phase
    return true;
}

bool kvmem_stagein_enqueue_v(const void *packed, size_t nbytes, uint8_t *dst, int64_t *set_us) {
    const auto t0 = std::chrono::steady_clock::now();
    kvmem_gpu_state *st = g_state;
    if (!st || !st->slab[0]) return report("enqueue", "stage-in is not ready");
    if (!st->out_src.empty()) return report("enqueue", "stage-out records are pending");
    if (!packed || !dst) return report("enqueue", "null record or destination");
    if (!nbytes) return true;
    if (nbytes > kvmem_gpu_state::kSlab) return report("enqueue", "record larger than the 32 MiB slab");
    if (st->used + nbytes > kvmem_gpu_state::kSlab || st->src.size() + st->krec.size() >= 8192)
        if (!kvmem_stagein_flush(nullptr, nullptr, nullptr, nullptr)) return false;
    // a fresh slab may still be the target of a stage-out copy
    if (st->used == 0 && st->out_done[st->cur]) (void)hipEventSynchronize(st->out_done[st->cur]);
    uint8_t *slot = st->slab[st->cur] + st->used;
    std::memcpy(slot, packed, nbytes);
    st->src.push_back(slot);
    st->dst.push_back(dst);
    st->bytes.push_back(nbytes);
    st->used += (nbytes + 15) / 16 * 16;  // keep records 16-byte aligned in the slab
    if (set_us) *set_us += micros_since(t0);
    return true;
}

bool kvmem_stagein_enqueue_k(kvr_format ty, const void *packed, size_t nbytes, uint8_t *dst, int64_t nt,
                             int64_t n_embd, int nrot, int n_head, int n_embd_head, int n_rot_rope, int32_t pos0,
                             const float *theta, int n_theta, int64_t *copy_us, int64_t *rope_us,
                             int64_t *hadamard_us, int64_t *set_us) {
    const auto t0 = std::chrono::steady_clock::now();
    kvmem_gpu_state *st = g_state;
    if (!st || !st->slab[0]) return report("enqueue K", "stage-in is not ready");
    if (!st->out_src.empty()) return report("enqueue K", "stage-out records are pending");
    // stagein.cu:817-831: quantized K only, a Walsh-Hadamard size it
    // provides, heads that tile the row
    if (!packed || !dst || (ty != KVR_FMT_Q8_0 && ty != KVR_FMT_Q4_0))
        return report("enqueue K", "null record or a K type other than q8_0 / q4_0");
    if (nrot > 0 && nrot != 64 && nrot != 128 && nrot != 256 && nrot != 512)
        return report("enqueue K", "Walsh-Hadamard size must be 64, 128, 256 or 512");
    if (int64_t(n_head) * n_embd_head != n_embd || nt <= 0 || n_embd <= 0 || n_embd > UINT32_MAX ||
        nt > UINT32_MAX)
        return report("enqueue K", "head geometry does not tile the row");
    if (n_rot_rope < 0 || n_rot_rope % 2 || n_rot_rope > n_embd_head || (n_rot_rope && (!theta || n_theta != n_rot_rope / 2)))
        return report("enqueue K", "rotation needs an even n_rot <= head dim and n_rot/2 angles");
    const size_t row = size_t(n_embd) / 32 * (ty == KVR_FMT_Q8_0 ? 34 : 18);
    if (n_embd % 32 || nbytes != size_t(nt) * row) return report("enqueue K", "record size does not match its rows");
    if (nbytes > kvmem_gpu_state::kSlab) return report("enqueue K", "record larger than the 32 MiB slab");
    if (!st->sel) {
        const uint32_t init[2] = {0, 1};
        if (hipError_t e = hipMalloc(&st->sel, sizeof init); e != hipSuccess) return report_hip("enqueue K", e);
        if (hipError_t e = hipMemcpy(st->sel, init, sizeof init, hipMemcpyHostToDevice); e != hipSuccess)
            return report_hip("enqueue K", e);
    }
    if (n_rot_rope && !std::equal(theta, theta + n_theta, st->theta_host.begin(), st->theta_host.end())) {
        // new angles: queued records still use the old ones, so flush first
        if (!kvmem_stagein_flush(copy_us, rope_us, hadamard_us, set_us)) return false;
        kvmem_stagein_sync();
        if (st->theta) (void)hipFree(st->theta);
        st->theta = nullptr;
        if (hipError_t e = hipMalloc(&st->theta, size_t(n_theta) * sizeof(float)); e != hipSuccess)
            return report_hip("enqueue K", e);
        if (hipError_t e = hipMemcpy(st->theta, theta, size_t(n_theta) * sizeof(float), hipMemcpyHostToDevice);
            e != hipSuccess)
            return report_hip("enqueue K", e);
        st->theta_host.assign(theta, theta + n_theta);
    }
    if (st->used + nbytes > kvmem_gpu_state::kSlab || st->src.size() + st->krec.size() >= 8192)
        if (!kvmem_stagein_flush(copy_us, rope_us, hadamard_us, set_us)) return false;
    // a fresh slab may still be the target of a stage-out copy
    if (st->used == 0 && st->out_done[st->cur]) (void)hipEventSynchronize(st->out_done[st->cur]);
    uint8_t *slot = st->slab[st->cur] + st->used;
    std::memcpy(slot, packed, nbytes);
    st->krec.push_back({slot, dst, ty, uint32_t(nt), uint32_t(n_embd), uint32_t(nrot), uint32_t(n_embd_head),
                        uint32_t(n_rot_rope), pos0});
    st->used += (nbytes + 15) / 16 * 16;
    if (set_us) *set_us += micros_since(t0);
    return true;
}

bool kvmem_stageout_enqueue(const void *gpu_src, size_t nbytes) {
    kvmem_gpu_state *st = g_state;
    // stagein.cu:883-905: no stage-in records pending, the record fits the slot
    if (!st || !st->slab[0] || !st->slab[1] || !gpu_src || !nbytes || !st->src.empty() || !st->krec.empty())
        return false;
    if (nbytes > kvmem_gpu_state::kSlab || st->out_used + nbytes > kvmem_gpu_state::kSlab) return false;
    st->out_src.push_back(gpu_src);
    st->out_off.push_back(st->out_used);
    st->out_bytes.push_back(nbytes);
    st->out_used += nbytes;
    return true;
}

size_t kvmem_stageout_used() { return g_state ? g_state->out_used : 0; }

int kvmem_stageout_submit(int64_t *copy_us) {
    const auto t0 = std::chrono::steady_clock::now();
    kvmem_gpu_state *st = g_state;
    if (!st || st->out_src.empty()) return -1;
    const int slot = st->out_cur;
    const hipStream_t s = copy_stream(st);
    // a stage-in flush still reading this slab finishes first
    if (st->slab_busy[slot]) {
        if (hipError_t e = hipEventSynchronize(st->slab_done[slot]); e != hipSuccess) return report_hip("stage-out", e), -1;
        st->slab_busy[slot] = false;
    }
    if (!st->out_done[slot] && hipEventCreateWithFlags(&st->out_done[slot], hipEventDisableTiming) != hipSuccess)
        return report("stage-out", "event"), -1;
    void *base = nullptr;
    if (hipError_t e = hipHostGetDevicePointer(&base, st->slab[slot], 0); e != hipSuccess)
        return report_hip("stage-out", e), -1;
    std::vector<void *> dst(st->out_src.size());
    for (size_t i = 0; i < dst.size(); ++i) dst[i] = static_cast<uint8_t *>(base) + st->out_off[i];
    // one launch writes every record over the host link into the slot
    if (kvr_d2d_batched(st->ctx, st->out_src.data(), dst.data(), st->out_bytes.data(), uint32_t(dst.size()), s) !=
        KVR_OK)
        return report_kvr("stage-out"), -1;
    if (hipError_t e = hipEventRecord(st->out_done[slot], s); e != hipSuccess) return report_hip("stage-out", e), -1;
    st->out_src.clear();
    st->out_off.clear();
    st->out_bytes.clear();
    st->out_used = 0;
    st->out_cur = 1 - slot;
    if (copy_us) *copy_us += micros_since(t0);
    return slot;
}

bool kvmem_stageout_wait(int slot, int64_t *copy_us) {
    if (slot < 0) return true;
    kvmem_gpu_state *st = g_state;
    if (!st || slot > 1 || !st->out_done[slot]) return false;
    const auto t0 = std::chrono::steady_clock::now();
    if (hipError_t e = hipEventSynchronize(st->out_done[slot]); e != hipSuccess) return report_hip("stage-out wait", e);
    if (copy_us) *copy_us += micros_since(t0);
    return true;
}

const uint8_t *kvmem_stageout_slot_base(int slot) {
    if (!g_state || slot < 0 || slot > 1) return nullptr;
    return g_state->slab[slot];
}

void kvmem_stageout_clear() {
    if (!g_state) return;
    g_state->out_src.clear();
    g_state->out_off.clear();
    g_state->out_bytes.clear();
    g_state->out_used = 0;
}

bool kvmem_d2d_batched(const void *const *src, void *const *dst, const size_t *nbytes, int n) {
    if (!g_state && !kvmem_gpu_state_create()) return false;
    if (n < 0) return report("d2d", "negative op count");
    if (kvr_d2d_batched(g_state->ctx, src, dst, nbytes, uint32_t(n), kvr_copy_stream(g_state->ctx)) != KVR_OK)
        return report_kvr("d2d");
    return true;
}

bool kvmem_meank_ready(uint32_t n_layer, uint32_t n_embd) {
    if (!n_layer || !n_embd) return false;
    if (!g_state && !kvmem_gpu_state_create()) return false;
    kvmem_gpu_state *st = g_state;
    if (st->acc && st->n_layer == n_layer && st->n_embd == n_embd) return true;
    kvmem_meank_free();
    const size_t bytes = size_t(n_layer) * n_embd * sizeof(float);
    if (hipError_t e = hipMalloc(&st->acc, bytes); e != hipSuccess) {
        st->acc = nullptr;
        return report_hip("meank acc", e);
    }
    if (hipError_t e = hipMalloc(&st->acc_count, size_t(n_layer) * sizeof(uint32_t)); e != hipSuccess) {
        st->acc_count = nullptr;
        kvmem_meank_free();
        return report_hip("meank count", e);
    }
    st->n_layer = n_layer;
    st->n_embd = n_embd;
    st->acc_pos.assign(n_layer, 0);
    const hipStream_t s = copy_stream(st);
    if (hipMemsetAsync(st->acc, 0, bytes, s) != hipSuccess ||
        hipMemsetAsync(st->acc_count, 0, size_t(n_layer) * sizeof(uint32_t), s) != hipSuccess) {
        kvmem_meank_free();
        return report("meank", "zeroing failed");
    }
    return true;
}

void kvmem_meank_free() {
    kvmem_gpu_state *st = g_state;
    if (!st) return;
    if (st->acc || st->acc_count) (void)hipStreamSynchronize(copy_stream(st));
    if (st->acc) (void)hipFree(st->acc);
    if (st->acc_count) (void)hipFree(st->acc_count);
    st->acc = nullptr;
    st->acc_count = nullptr;
    st->n_layer = st->n_embd = 0;
    st->acc_pos.clear();
}

void kvmem_meank_zero(uint32_t il) {
    kvmem_gpu_state *st = g_state;
    if (!st || !st->acc || il >= st->n_layer) return;
    (void)hipMemsetAsync(st->acc + size_t(il) * st->n_embd, 0, size_t(st->n_embd) * sizeof(float), copy_stream(st));
    st->acc_pos[il] = 0;
}

bool kvmem_meank_add(uint32_t il, kvr_format ty, const void *gpu_k, uint32_t tok0, uint32_t n_keep,
                     uint32_t n_embd, int64_t ne0, size_t nb0, size_t nb1, size_t nb2) {
    kvmem_gpu_state *st = g_state;
    if (!st || !st->acc || !gpu_k || !n_keep || !n_embd || ne0 <= 0 || il >= st->n_layer || n_embd != st->n_embd ||
        n_embd % uint64_t(ne0))
        return false;
    // One running sum per layer: a single page as long as the layer's
    // position counter, which kvmem_meank_zero resets (position 0 restarts).
    const uint8_t *k = static_cast<const uint8_t *>(gpu_k) + size_t(tok0) * nb2;
    const uint32_t heads = uint32_t(n_embd / uint64_t(ne0));
    if (kvr_summary_accumulate(st->ctx, st->acc + size_t(il) * n_embd, st->acc_count + il, 0xffffffffu, k, ty,
                               st->acc_pos[il], n_keep, heads, uint32_t(ne0), nb2, nb1, nb0,
                               kvr_copy_stream(st->ctx)) != KVR_OK)
        return report_kvr("meank add");
    st->acc_pos[il] += n_keep;
    return true;
}

bool kvmem_meank_d2h(uint32_t il, float *host, uint32_t n_embd) {
    kvmem_gpu_state *st = g_state;
    if (!st || !st->acc || !host || il >= st->n_layer || n_embd != st->n_embd) return false;
    const hipStream_t s = copy_stream(st);
    if (hipError_t e = hipMemcpyAsync(host, st->acc + size_t(il) * n_embd, size_t(n_embd) * sizeof(float),
                                      hipMemcpyDeviceToHost, s);
        e != hipSuccess)
        return report_hip("meank D2H", e);
    if (hipError_t e = hipStreamSynchronize(s); e != hipSuccess) return report_hip("meank D2H", e);
    return true;
}

// ---------------------------------------------------------------------------
RecallTransfer::RecallTransfer(kvr_context *ctx, std::vector<kvr_plane> planes, uint32_t lanes, uint32_t page_tokens,
                               const uint32_t *selected, const uint32_t *count, uint32_t k, kvr_copy_engine engine,
                               void *stream, void *ready)
    : ctx_(ctx), planes_(std::move(planes)), lanes_(lanes ? lanes : 1), page_tokens_(page_tokens), k_(k),
      selected_(selected), count_(count), engine_(engine), stream_(stream), ready_(ready) {
    require(ctx_ && !planes_.empty() && planes_.size() <= KVR_MAX_PLANES && page_tokens_ && k_ && selected_ &&
                count_,
            "invalid recall transfer plan");
    if (!stream_) stream_ = kvr_copy_stream(ctx_);
    hipEvent_t ev = nullptr;
    hip_ok(hipEventCreateWithFlags(&ev, hipEventDisableTiming), "transfer event");
    done_ = ev;
}

RecallTransfer::~RecallTransfer() {
    (void)abort();
    if (done_) (void)hipEventDestroy(static_cast<hipEvent_t>(done_));
}

void RecallTransfer::start_spill() {
    if (phase_ != Phase::Prepared) throw std::logic_error("spill starts once, from a prepared transfer");
    phase_ = Phase::Spilled;
}

void RecallTransfer::start_restore() {
    if (phase_ != Phase::Spilled) throw std::logic_error("restore starts after the spill completed");
    const hipStream_t s = static_cast<hipStream_t>(stream_);
    if (ready_) hip_ok(hipStreamWaitEvent(s, static_cast<hipEvent_t>(ready_), 0), "selection event");
    ok(kvr_stage_in(ctx_, planes_.data(), uint32_t(planes_.size()), lanes_, page_tokens_, selected_, count_, k_,
                    engine_, s),
       "recall restore");
    hip_ok(hipEventRecord(static_cast<hipEvent_t>(done_), s), "transfer event");
    phase_ = Phase::Restoring;
}

TransferPoll RecallTransfer::poll() {
    TransferPoll p;
    switch (phase_) {
    case Phase::Prepared: return p;
    case Phase::Spilled:
    case Phase::Ready:
    case Phase::Published: p.status = TransferStatus::Complete; return p;
    case Phase::Failed:
    case Phase::Aborted:
        p.status = TransferStatus::Failed;
        p.error = error_.empty() ? "transfer aborted" : error_;
        return p;
    case Phase::Restoring: break;
    }
    const hipError_t e = hipEventQuery(static_cast<hipEvent_t>(done_));
    if (e == hipErrorNotReady) return p;
    if (e == hipSuccess) {
        if (kvr_check(ctx_, stream_) == KVR_OK) {
            phase_ = Phase::Ready;
            p.status = TransferStatus::Complete;
            return p;
        }
        error_ = kvr_last_error();
    } else {
        error_ = hipGetErrorString(e);
    }
    phase_ = Phase::Failed;
    p.status = TransferStatus::Failed;
    p.error = error_;
    return p;
}

void RecallTransfer::publish() {
    if (phase_ != Phase::Ready) throw std::logic_error("publish needs a completed restore");
    phase_ = Phase::Published;
}

AbortResult RecallTransfer::abort() noexcept {
    if (phase_ == Phase::Restoring) (void)hipEventSynchronize(static_cast<hipEvent_t>(done_));
    const bool touched = phase_ == Phase::Restoring || phase_ == Phase::Ready || phase_ == Phase::Failed;
    if (phase_ != Phase::Published) phase_ = Phase::Aborted;
    return touched ? AbortResult::SessionInvalidated : AbortResult::PreviousViewPreserved;
}

// ---------------------------------------------------------------------------
SummaryCapture::SummaryCapture(kvr_context *ctx, uint32_t layers, uint32_t max_pages, uint32_t page_tokens,
                               uint32_t kv_heads, uint32_t head_dim)
    : ctx_(ctx), layers_(layers), max_pages_(max_pages), page_tokens_(page_tokens), kv_heads_(kv_heads),
      head_dim_(head_dim) {
    require(ctx_ && layers_ && max_pages_ && page_tokens_ && kv_heads_ && head_dim_, "invalid capture geometry");
    const size_t cells = size_t(layers_) * max_pages_ * kv_heads_ * head_dim_;
    hip_ok(hipMalloc(&sums_, cells * sizeof(float)), "capture sums");
    hip_ok(hipMalloc(&means_, cells * sizeof(float)), "capture means");
    hip_ok(hipMalloc(&summaries_, cells * sizeof(uint16_t)), "capture summaries");
    hip_ok(hipMalloc(&counts_, size_t(layers_) * max_pages_ * sizeof(uint32_t)), "capture counts");
    hip_ok(hipMemset(counts_, 0, size_t(layers_) * max_pages_ * sizeof(uint32_t)), "capture counts");
}

SummaryCapture::~SummaryCapture() {
    (void)kvr_check(ctx_, nullptr);
    (void)hipFree(sums_);
    (void)hipFree(means_);
    (void)hipFree(summaries_);
    (void)hipFree(counts_);
}

void SummaryCapture::capture(uint32_t layer, const void *k, kvr_format scalar, uint64_t pos0, uint32_t n,
                             size_t token_stride, size_t head_stride, size_t dim_stride, void *stream) {
    require(layer < layers_, "capture layer outside the stack");
    if (!n) return;
    require(pos0 + n <= uint64_t(max_pages_) * page_tokens_, "capture beyond the planned pages");
    const size_t width = size_t(kv_heads_) * head_dim_;
    ok(kvr_summary_accumulate(ctx_, sums_ + size_t(layer) * max_pages_ * width, counts_ + size_t(layer) * max_pages_,
                              page_tokens_, k, scalar, pos0, n, kv_heads_, head_dim_, token_stride, head_stride,
                              dim_stride, stream),
       "summary capture");
}

PageSummaries SummaryCapture::finalize(uint32_t pages, void *stream) {
    require(pages && pages <= max_pages_, "finalize beyond the planned pages");
    const size_t width = size_t(kv_heads_) * head_dim_;
    PageSummaries out;
    out.pages = pages;
    out.page_tokens = page_tokens_;
    out.kv_heads = kv_heads_;
    out.head_dim = head_dim_;
    for (uint32_t l = 0; l < layers_; ++l) {
        const size_t off = size_t(l) * max_pages_ * width;
        ok(kvr_summary_finalize(ctx_, sums_ + off, counts_ + size_t(l) * max_pages_, pages, uint32_t(width),
                                means_ + off, summaries_ + off, stream),
           "summary finalize");
        out.layers.push_back(summaries_ + off);
    }
    return out;
}

const float *SummaryCapture::means(uint32_t layer) const {
    require(layer < layers_, "capture layer outside the stack");
    return means_ + size_t(layer) * max_pages_ * kv_heads_ * head_dim_;
}

// ---------------------------------------------------------------------------
// Sampled attention (llama-kvmem-attention-cuda.cu:148-193 is the interface
// mirrored: score() declines with false, stages a mask that is not on the
// device, and returns host masses).
namespace {
bool on_device(const void *p, int &device) {
    hipPointerAttribute_t attr{};
    if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
        (void)hipGetLastError();  // unknown to the runtime: host memory
        return false;
    }
    if (attr.type != hipMemoryTypeDevice && attr.type != hipMemoryTypeManaged) return false;
    device = attr.device;
    return true;
}
}  // namespace

struct AttentionSamplerHip::Impl {
    int device = -1;
    kvr_context *ctx = nullptr;
    void *mask = nullptr, *out = nullptr;
    size_t mask_bytes = 0, out_bytes = 0;
    void grow(void *&buf, size_t &have, size_t need) {
        if (need <= have) return;
        if (buf) hip_ok(hipFree(buf), "hipFree");
        buf = nullptr;
        have = 0;
        hip_ok(hipMalloc(&buf, need), "hipMalloc");
        have = need;
    }
    ~Impl() {
        if (device < 0) return;
        DeviceBinding bind(device);
        if (mask) (void)hipFree(mask);
        if (out) (void)hipFree(out);
        if (ctx) kvr_destroy(ctx);
    }
};

AttentionSamplerHip::AttentionSamplerHip() : impl_(new Impl) {}
AttentionSamplerHip::~AttentionSamplerHip() = default;

bool AttentionSamplerHip::score(const AttentionTensor &q, const AttentionTensor &k, const AttentionTensor &mask,
                                float scale, float softcap, uint32_t block, const std::vector<uint32_t> &rows,
                                std::vector<std::vector<float>> &output) {
    auto scalar = [](kvr_format f) { return f == KVR_FMT_F32 || f == KVR_FMT_F16 || f == KVR_FMT_BF16; };
    const bool key_ok = scalar(k.type) || k.type == KVR_FMT_Q8_0 || k.type == KVR_FMT_Q4_0 || k.type == KVR_FMT_Q5_0;
    if (!scalar(q.type) || !scalar(mask.type) || !key_ok || q.ne[0] > 256 || q.ne[0] % 32 || q.ne[0] <= 0)
        return false;
    int device = -1, key_device = -1, mask_device = -1;
    if (!on_device(q.data, device) || !on_device(k.data, key_device) || device != key_device) return false;
    Impl &m = *impl_;
    if (m.device < 0) {
        m.device = device;
        DeviceBinding bind(device);
        if (kvr_create(device, &m.ctx) != KVR_OK) {
            m.device = -1;
            throw std::runtime_error(std::string("attention sampler context: ") + kvr_last_error());
        }
    }
    if (m.device != device) throw std::runtime_error("attention sampler changed device");
    require(block > 0 && k.ne[1] > 0 && q.ne[2] > 0 && k.ne[2] > 0, "attention sampler geometry");
    DeviceBinding bind(device);
    const uint32_t tokens = uint32_t(k.ne[1]), pages = (tokens + block - 1) / block, n = uint32_t(rows.size());
    output.assign(n, std::vector<float>(pages));
    if (!n) return true;
    const size_t mel = mask.type == KVR_FMT_F32 ? 4 : 2, mrow = size_t(mask.ne[0]) * mel;
    require(mask.ne[0] >= int64_t(tokens), "mask rows shorter than the keys");
    kvr_attention_sample a{};
    a.q = q.data;
    a.q_format = q.type;
    a.q_row_stride = q.nb[1];
    a.q_head_stride = q.nb[2];
    a.k = k.data;
    a.k_format = k.type;
    a.k_row_stride = k.nb[1];
    a.k_head_stride = k.nb[2];
    a.mask_format = mask.type;
    a.head_dim = uint32_t(q.ne[0]);
    a.query_heads = uint32_t(q.ne[2]);
    a.kv_heads = uint32_t(k.ne[2]);
    a.tokens = tokens;
    a.page_tokens = block;
    a.scale = scale;
    a.softcap = softcap;
    a.rows = rows.data();
    a.n_rows = n;
    const hipStream_t s = static_cast<hipStream_t>(kvr_select_stream(m.ctx));
    StreamDrain drain{s};
    std::vector<uint32_t> staged_rows;
    if (on_device(mask.data, mask_device) && mask_device == device) {
        a.mask = mask.data;
        a.mask_row_stride = mask.nb[1];
    } else {
        // the sampled rows only, one after another (the reference's staged
        // mask, llama-kvmem-attention-cuda.cu:163-172)
        m.grow(m.mask, m.mask_bytes, size_t(n) * mrow);
        std::vector<uint8_t> host(size_t(n) * mrow);
        for (uint32_t i = 0; i < n; ++i)
            std::memcpy(host.data() + size_t(i) * mrow,
                        static_cast<const uint8_t *>(mask.data) + size_t(rows[i]) * mask.nb[1], mrow);
        hip_ok(hipMemcpyAsync(m.mask, host.data(), host.size(), hipMemcpyHostToDevice, s), "mask H2D");
        hip_ok(hipStreamSynchronize(s), "mask H2D");
        staged_rows.resize(n);
        for (uint32_t i = 0; i < n; ++i) staged_rows[i] = i;
        a.mask = m.mask;
        a.mask_row_stride = mrow;
        a.mask_rows = staged_rows.data();
    }
    m.grow(m.out, m.out_bytes, size_t(n) * pages * sizeof(float));
    const kvr_status st = kvr_attention_page_mass(m.ctx, &a, static_cast<float *>(m.out), s);
    if (st == KVR_ERR_UNSUPPORTED) return false;
    ok(st, "kvr_attention_page_mass");
    std::vector<float> host(size_t(n) * pages);
    hip_ok(hipMemcpyAsync(host.data(), m.out, host.size() * sizeof(float), hipMemcpyDeviceToHost, s), "mass D2H");
    hip_ok(hipStreamSynchronize(s), "mass D2H");
    drain.armed = false;
    for (uint32_t i = 0; i < n; ++i) std::copy_n(host.data() + size_t(i) * pages, pages, output[i].data());
    return true;
}

}  // namespace kvmem_hip
