// kvmem_memory.cpp -- RecallMemory: the recall part of KVMem's llama memory
// object on the device, and its MemoryBackend side of the contract.
// Everything on the device goes through kvr_* calls and SummaryCapture.
#include "kvmem_hip/kvmem_memory.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <deque>
#include <limits>
#include <stdexcept>

namespace kvmem_hip {
namespace {

void check(kvr_status s, const char *what) {
    if (s == KVR_OK) return;
    const std::string msg = std::string(what) + ": " + kvr_last_error();
    if (s == KVR_ERR_HIP) throw std::runtime_error(msg);
    if (s == KVR_ERR_WORKSPACE) throw std::length_error(msg);
    throw std::invalid_argument(msg);
}
void hip_check(hipError_t e, const char *what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}
[[noreturn]] void plan_error(MemoryErrorCode code, const char *msg) { throw MemoryError(code, msg); }

size_t scalar_bytes(kvr_format f) { return f == KVR_FMT_F32 ? 4 : 2; }
bool query_scalar(kvr_format f) { return f == KVR_FMT_F32 || f == KVR_FMT_F16 || f == KVR_FMT_BF16; }

size_t row_size(kvr_format f, uint32_t width) {
    switch (f) {
    case KVR_FMT_F16: return size_t(width) * 2;
    case KVR_FMT_Q8_0: return size_t(width) / 32 * 34;
    case KVR_FMT_Q4_1: return size_t(width) / 32 * 20;
    case KVR_FMT_Q4_0: return size_t(width) / 32 * 18;
    default: return 0;
    }
}
const char *format_name(kvr_format f) {
    switch (f) {
    case KVR_FMT_F16: return "f16";
    case KVR_FMT_Q8_0: return "q8_0";
    case KVR_FMT_Q4_1: return "q4_1";
    case KVR_FMT_Q4_0: return "q4_0";
    default: return "other";
    }
}

std::atomic<uint64_t> g_sessions{1};

struct Capture {
    const void *tensor;
    int il;
    char which;
};
struct History {
    bool set = false;
    kvr_plane k{}, v{};
};
}  // namespace

struct RecallMemory::Impl {
    RecallMemoryConfig cfg;
    std::vector<uint32_t> layers;     // served model layers, ascending
    kvr_context *ctx = nullptr;
    std::unique_ptr<SummaryCapture> sums;
    // device Query rows per served layer: [max_query_rows][Hq][D] of q_type
    std::vector<uint8_t *> qbuf;
    std::vector<kvr_format> q_type;
    std::vector<uint32_t> q_count;
    // device scoring state
    double *scores = nullptr;
    uint32_t *sel = nullptr, *cnt = nullptr;
    uint8_t *mask = nullptr;
    uint32_t scored_pages = 0, last_k = 0;
    std::vector<double> host_scores;
    // capture state
    std::vector<Capture> pending;
    std::deque<std::vector<int32_t>> positions;
    bool graph_has_q = false, graph_has_k = false;
    bool prefill_capture = true, pinned = false;
    int32_t query_begin = -1, query_end = -1;
    // catalogue
    uint64_t frontier = 0;
    std::vector<uint64_t> content_version, statistics_version;
    uint64_t history_revision = 0, view_version = 0;
    SessionIdentity session;
    bool valid = true;
    std::vector<History> history;
    std::vector<uint64_t> resident;

    hipStream_t stream() const { return static_cast<hipStream_t>(kvr_select_stream(ctx)); }
    hipStream_t copy_stream() const { return static_cast<hipStream_t>(kvr_copy_stream(ctx)); }

    int index_of(int il) const {
        if (il < 0) return -1;
        const auto it = std::lower_bound(layers.begin(), layers.end(), uint32_t(il));
        return it != layers.end() && *it == uint32_t(il) ? int(it - layers.begin()) : -1;
    }
    uint32_t page_count() const { return uint32_t((frontier + cfg.block_tokens - 1) / cfg.block_tokens); }
    uint32_t slot_pages() const { return cfg.budget_pages ? cfg.budget_pages : cfg.max_pages; }
    size_t q_row_bytes(uint32_t i) const { return size_t(cfg.query_heads) * cfg.head_dim * scalar_bytes(q_type[i]); }

    BlockDescriptor block(uint32_t p) const {
        BlockDescriptor b;
        b.session = session;
        b.id = p;
        b.original_start = uint64_t(p) * cfg.block_tokens;
        b.valid_tokens = uint32_t(std::min<uint64_t>(cfg.block_tokens, frontier - b.original_start));
        b.content_version = content_version[p];
        b.statistics_version = statistics_version[p];
        return b;
    }

    void harvest_k(const TensorView &t, uint32_t idx, const std::vector<int32_t> &pos) {
        if (!query_scalar(t.type)) throw std::invalid_argument("captured K must be f32, f16 or bf16");
        if (t.ne[0] != int64_t(cfg.head_dim) || t.ne[1] != int64_t(cfg.kv_heads) || t.ne[2] < int64_t(pos.size()))
            throw std::invalid_argument("captured K does not match the memory's geometry");
        const int32_t pos0 = pos.front();
        for (size_t i = 0; i < pos.size(); ++i)
            if (pos[i] != pos0 + int32_t(i)) throw std::invalid_argument("captured K positions are not consecutive");
        if (pos0 < 0) throw std::invalid_argument("captured K at a negative position");
        sums->capture(idx, t.data, t.type, uint64_t(pos0), uint32_t(pos.size()), t.nb[2], t.nb[1], t.nb[0], stream());
    }

    void harvest_q(const TensorView &t, uint32_t idx, const std::vector<int32_t> &pos,
                   std::vector<const void *> &src, std::vector<void *> &dst, std::vector<size_t> &bytes) {
        if (!query_scalar(t.type)) throw std::invalid_argument("captured Query must be f32, f16 or bf16");
        if (t.ne[0] != int64_t(cfg.head_dim) || t.ne[1] != int64_t(cfg.query_heads) || t.ne[2] < int64_t(pos.size()))
            throw std::invalid_argument("captured Query does not match the memory's geometry");
        const size_t el = scalar_bytes(t.type);
        if (t.nb[0] != el) throw std::invalid_argument("captured Query dims must be contiguous");
        if (q_count[idx] && q_type[idx] != t.type)
            throw std::invalid_argument("captured Query rows change their element type");
        q_type[idx] = t.type;
        const size_t head = size_t(cfg.head_dim) * el, row = head * cfg.query_heads;
        const bool packed = t.nb[1] == head;
        for (size_t i = 0; i < pos.size(); ++i) {
            if (!query_contains(pos[i])) continue;
            if (q_count[idx] >= cfg.max_query_rows) throw std::length_error("Query rows exceed max_query_rows");
            const uint8_t *base = static_cast<const uint8_t *>(t.data) + i * t.nb[2];
            uint8_t *out = qbuf[idx] + size_t(q_count[idx]) * row;
            if (packed) {
                src.push_back(base);
                dst.push_back(out);
                bytes.push_back(row);
            } else {
                for (uint32_t h = 0; h < cfg.query_heads; ++h) {
                    src.push_back(base + h * t.nb[1]);
                    dst.push_back(out + h * head);
                    bytes.push_back(head);
                }
            }
            ++q_count[idx];
        }
    }

    bool query_contains(int32_t p) const {
        return query_begin >= 0 && p >= query_begin && (query_end <= 0 || p < query_end);
    }
    bool want_q_capture() const { return cfg.retrieval && !pinned && query_begin >= 0; }
    bool want_decode_mean() const { return pinned && cfg.retrieval; }
};

RecallMemory::RecallMemory(const RecallMemoryConfig &c) : impl_(new Impl) {
    Impl &m = *impl_;
    m.cfg = c;
    if (!c.n_layer || !c.query_heads || !c.kv_heads || !c.head_dim || c.query_heads % c.kv_heads || !c.block_tokens ||
        !c.max_pages || c.budget_pages > c.max_pages || !c.max_query_rows)
        throw std::invalid_argument("invalid recall memory geometry");
    m.layers = c.layers;
    if (m.layers.empty())
        for (uint32_t l = 0; l < c.n_layer; ++l) m.layers.push_back(l);
    std::sort(m.layers.begin(), m.layers.end());
    m.layers.erase(std::unique(m.layers.begin(), m.layers.end()), m.layers.end());
    if (m.layers.back() >= c.n_layer) throw std::invalid_argument("served layer outside the model");
    m.query_begin = c.query_begin;
    m.query_end = c.query_end;
    m.session.id = g_sessions++;
    m.session.incarnation = 1;
    hip_check(hipSetDevice(c.device), "hipSetDevice");
    check(kvr_create(c.device, &m.ctx), "recall memory context");
    const uint32_t n = uint32_t(m.layers.size());
    try {
        m.sums = std::make_unique<SummaryCapture>(m.ctx, n, c.max_pages, c.block_tokens, c.kv_heads, c.head_dim);
        const size_t qbytes = size_t(c.max_query_rows) * c.query_heads * c.head_dim * 4;
        m.qbuf.assign(n, nullptr);
        for (auto &q : m.qbuf) hip_check(hipMalloc(&q, qbytes), "hipMalloc Query rows");
        hip_check(hipMalloc(&m.scores, size_t(c.max_pages) * 8), "hipMalloc scores");
        hip_check(hipMalloc(&m.sel, size_t(c.max_pages) * 4 + 256), "hipMalloc selection");
        m.cnt = m.sel + c.max_pages;
        hip_check(hipMalloc(&m.mask, c.max_pages), "hipMalloc mask");
    } catch (...) {
        for (auto *q : m.qbuf) (void)hipFree(q);
        (void)hipFree(m.scores);
        (void)hipFree(m.sel);
        m.sums.reset();
        (void)kvr_destroy(m.ctx);
        throw;
    }
    m.q_type.assign(n, KVR_FMT_F32);
    m.q_count.assign(n, 0);
    m.history.assign(n, History{});
    m.content_version.assign(c.max_pages, 0);
    m.statistics_version.assign(c.max_pages, 0);
}

RecallMemory::~RecallMemory() {
    Impl &m = *impl_;
    (void)hipSetDevice(m.cfg.device);
    (void)hipStreamSynchronize(m.stream());
    (void)hipStreamSynchronize(m.copy_stream());
    m.sums.reset();
    for (auto *q : m.qbuf) (void)hipFree(q);
    (void)hipFree(m.scores);
    (void)hipFree(m.sel);
    (void)hipFree(m.mask);
    (void)kvr_destroy(m.ctx);
}

const RecallMemoryConfig &RecallMemory::config() const { return impl_->cfg; }
bool RecallMemory::owns_layer(int il) const { return impl_->index_of(il) >= 0; }
kvr_context *RecallMemory::context() const { return impl_->ctx; }

// ---- capture ------------------------------------------------------------------
void RecallMemory::note_ubatch(std::vector<int32_t> positions) { impl_->positions.push_back(std::move(positions)); }

void RecallMemory::register_capture(const void *tensor, int il, char which) {
    Impl &m = *impl_;
    if (!tensor || m.index_of(il) < 0) return;
    m.pending.push_back({tensor, il, which});
    if (which == 'q') m.graph_has_q = true;
    if (which == 'k') m.graph_has_k = true;
}

void RecallMemory::capture_on_new_graph() {
    Impl &m = *impl_;
    m.pending.clear();
    m.graph_has_q = m.graph_has_k = false;
}

void RecallMemory::harvest(const TensorResolver &resolve) {
    Impl &m = *impl_;
    if (m.pending.empty() || m.positions.empty()) return;
    const std::vector<int32_t> pos = std::move(m.positions.front());
    m.positions.pop_front();
    if (pos.empty()) return;
    hip_check(hipSetDevice(m.cfg.device), "hipSetDevice");
    std::vector<const void *> src;
    std::vector<void *> dst;
    std::vector<size_t> bytes;
    bool any_k = false;
    for (const Capture &c : m.pending) {
        if (c.which != 'k' && c.which != 'q') continue;  // V is not a statistic of this path
        const int idx = m.index_of(c.il);
        TensorView t;
        if (idx < 0 || !resolve || !resolve(c.tensor, t) || !t.data) continue;
        if (c.which == 'k' && (m.prefill_capture || m.want_decode_mean())) {
            m.harvest_k(t, uint32_t(idx), pos);
            any_k = true;
        } else if (c.which == 'q' && m.want_q_capture()) {
            m.harvest_q(t, uint32_t(idx), pos, src, dst, bytes);
        }
    }
    if (!src.empty())
        check(kvr_d2d_batched(m.ctx, src.data(), dst.data(), bytes.data(), uint32_t(src.size()), m.stream()),
              "Query rows");
    if (any_k) {
        const uint64_t end = uint64_t(pos.back()) + 1;
        const uint32_t first = uint32_t(uint64_t(pos.front()) / m.cfg.block_tokens);
        const uint32_t last = uint32_t((end - 1) / m.cfg.block_tokens);
        for (uint32_t p = first; p <= last && p < m.cfg.max_pages; ++p) {
            ++m.content_version[p];
            ++m.statistics_version[p];
        }
        m.frontier = std::max(m.frontier, end);
        ++m.history_revision;
    }
    // the engine may reuse the captured tensors once the harvest returns
    hip_check(hipStreamSynchronize(m.stream()), "hipStreamSynchronize");
    check(kvr_check(m.ctx, m.stream()), "capture");
}

bool RecallMemory::query_contains(int32_t pos) const { return impl_->query_contains(pos); }
bool RecallMemory::query_overlaps(uint32_t n, const int32_t *pos) const {
    if (!impl_->want_q_capture() || !n) return false;
    if (!pos) return true;
    for (uint32_t i = 0; i < n; ++i)
        if (impl_->query_contains(pos[i])) return true;
    return false;
}
bool RecallMemory::want_prefill_capture() const { return impl_->prefill_capture && !impl_->pinned; }
bool RecallMemory::want_q_capture() const { return impl_->want_q_capture(); }
bool RecallMemory::want_decode_mean() const { return impl_->want_decode_mean(); }

// capture_can_reuse (llama-memory-kvmem.cpp:2973-2987): after the pin, a
// decode graph must carry K; a graph's Query nodes must match whether this
// ubatch needs them.
bool RecallMemory::capture_can_reuse(uint32_t n_tokens, uint32_t n_pos, const int32_t *pos) const {
    (void)n_pos;
    const Impl &m = *impl_;
    if (want_decode_mean() && !m.graph_has_k) return false;
    return query_overlaps(n_tokens, pos) == m.graph_has_q;
}

// capture_stamp (llama-memory-kvmem.cpp:2989-3010): one bit per state that
// changes the capture graph's topology.
uint64_t RecallMemory::capture_stamp() const {
    const Impl &m = *impl_;
    uint64_t s = 1;
    if (m.pinned) s |= 2;
    if (want_decode_mean()) s |= 4;
    if (want_q_capture()) s |= 8;
    if (m.graph_has_k) s |= 32;
    if (m.graph_has_q) s |= 64;
    return s;
}

void RecallMemory::reset_query() { std::fill(impl_->q_count.begin(), impl_->q_count.end(), 0u); }
void RecallMemory::end_prefill_capture() { impl_->prefill_capture = false; }
void RecallMemory::pin_working_set() { impl_->pinned = true; }
void RecallMemory::set_query_span(int32_t begin, int32_t end) {
    impl_->query_begin = begin;
    impl_->query_end = end;
}

// ---- recall -------------------------------------------------------------------
uint64_t RecallMemory::frontier() const { return impl_->frontier; }
uint32_t RecallMemory::pages() const { return impl_->page_count(); }
uint32_t RecallMemory::query_rows(uint32_t layer) const {
    const int idx = impl_->index_of(int(layer));
    return idx < 0 ? 0 : impl_->q_count[idx];
}

PageSummaries RecallMemory::summaries() {
    Impl &m = *impl_;
    if (!m.page_count()) throw std::invalid_argument("no pages captured");
    return m.sums->finalize(m.page_count(), m.stream());
}

// score_retrieval (llama-memory-kvmem.cpp:4604-4653) on the device: the
// captured Query of every served layer against the fp16 summaries, softmax
// over the pages of query_score_frame's score mask, the head aggregation,
// summed over the layers with Query rows.
std::vector<double> RecallMemory::score() {
    Impl &m = *impl_;
    const uint32_t pages = m.page_count();
    if (!pages) throw std::invalid_argument("no pages captured");
    hip_check(hipSetDevice(m.cfg.device), "hipSetDevice");
    const hipStream_t s = m.stream();
    const PageSummaries sums = m.sums->finalize(pages, s);
    const uint32_t budget = m.cfg.budget_pages ? m.cfg.budget_pages : pages;
    const QueryScoreFrame frame =
        query_score_frame(m.frontier, m.cfg.block_tokens, budget, m.cfg.sink_pages, m.cfg.recent_pages, {});
    hip_check(hipMemcpyAsync(m.mask, frame.score_mask.data(), pages, hipMemcpyHostToDevice, s), "mask H2D");
    uint32_t active = 0;
    for (uint32_t c : m.q_count) active += c != 0;
    m.host_scores.assign(pages, 0.0);
    m.scored_pages = pages;
    if (!active) {
        hip_check(hipMemcpyAsync(m.scores, m.host_scores.data(), size_t(pages) * 8, hipMemcpyHostToDevice, s),
                  "scores H2D");
        hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
        return m.host_scores;
    }
    int accumulate = 0;
    for (uint32_t i = 0; i < m.layers.size(); ++i) {
        if (!m.q_count[i]) continue;
        const size_t el = scalar_bytes(m.q_type[i]);
        kvr_query q{};
        q.data = m.qbuf[i];
        q.scalar = m.q_type[i];
        q.rows = m.q_count[i];
        q.query_heads = m.cfg.query_heads;
        q.kv_heads = m.cfg.kv_heads;
        q.head_dim = m.cfg.head_dim;
        q.row_stride = m.q_row_bytes(i);
        q.head_stride = size_t(m.cfg.head_dim) * el;
        q.dim_stride = el;
        kvr_aggregation agg = m.cfg.aggregation == GqaScoreAggregation::Max        ? KVR_AGG_MAX
                              : m.cfg.aggregation == GqaScoreAggregation::MaxLogit ? KVR_AGG_MAX_LOGIT
                                                                                    : KVR_AGG_MEAN;
        check(kvr_score(m.ctx, &q, sums.layers[i], 1, pages, m.mask, agg, active, accumulate, m.scores, 0, s),
              "page scores");
        accumulate = 1;
    }
    hip_check(hipMemcpyAsync(m.host_scores.data(), m.scores, size_t(pages) * 8, hipMemcpyDeviceToHost, s),
              "scores D2H");
    hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
    check(kvr_check(m.ctx, s), "page scores");
    return m.host_scores;
}

// query_fixed_blocks (kvmem_store.cpp:381-408) then pick_scored_blocks
// (:418-451) over the last score(): sink and recent pages kept, the rest by
// score with the configured tie rule, ascending ids.
std::vector<uint32_t> RecallMemory::select() {
    Impl &m = *impl_;
    const uint32_t pages = m.scored_pages;
    if (!pages) throw std::logic_error("select before score");
    const uint32_t budget = m.cfg.budget_pages ? std::min(m.cfg.budget_pages, pages) : pages;
    const std::vector<uint32_t> fixed = query_fixed_blocks(pages, budget, m.cfg.sink_pages, m.cfg.recent_pages, {},
                                                           m.cfg.block_tokens, m.frontier, {});
    hip_check(hipSetDevice(m.cfg.device), "hipSetDevice");
    const hipStream_t s = m.stream();
    check(kvr_select_topk(m.ctx, m.scores, 1, pages, budget, fixed.data(), uint32_t(fixed.size()),
                          m.cfg.tie == TieRule::HigherFirst ? KVR_TIE_HIGHER_FIRST : KVR_TIE_LOWER_FIRST, 0, m.sel,
                          m.cnt, s),
          "page selection");
    std::vector<uint32_t> out(budget);
    uint32_t count = 0;
    hip_check(hipMemcpyAsync(out.data(), m.sel, size_t(budget) * 4, hipMemcpyDeviceToHost, s), "selection D2H");
    hip_check(hipMemcpyAsync(&count, m.cnt, 4, hipMemcpyDeviceToHost, s), "count D2H");
    hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
    check(kvr_check(m.ctx, s), "page selection");
    out.resize(std::min(count, budget));
    m.last_k = budget;
    return out;
}

const double *RecallMemory::device_scores() const { return impl_->scores; }
const uint32_t *RecallMemory::device_selection() const { return impl_->sel; }
const uint32_t *RecallMemory::device_count() const { return impl_->cnt; }

void RecallMemory::set_history(uint32_t layer, const kvr_plane &k, const kvr_plane &v) {
    Impl &m = *impl_;
    const int idx = m.index_of(int(layer));
    if (idx < 0) throw std::invalid_argument("history for a layer this memory does not serve");
    if (!k.history || !v.history || !k.slots || !v.slots || !row_size(k.format, k.width) ||
        !row_size(v.format, v.width))
        throw std::invalid_argument("history planes need pinned rows, slots and a stage-in format");
    m.history[idx] = {true, k, v};
}

// ---- MemoryBackend ----------------------------------------------------------------
MemoryStamp RecallMemory::stamp() const noexcept {
    const Impl &m = *impl_;
    MemoryStamp s;
    s.valid = m.valid;
    s.session = m.session;
    s.history_revision = m.history_revision;
    s.view_version = m.view_version;
    s.frontier = m.frontier;
    s.execution_history = 0;
    return s;
}

MemorySnapshot RecallMemory::snapshot() const {
    const Impl &m = *impl_;
    MemorySnapshot snap;
    snap.stamp = stamp();
    for (uint32_t p = 0; p < m.page_count(); ++p) {
        BlockCopies c;
        c.block = m.block(p);
        c.host_version = c.block.content_version;  // the pinned history is every page's current copy
        snap.blocks.push_back(c);
    }
    snap.resident = m.resident;
    return snap;
}

// The payload of one page as a record holds it: every served layer's K then
// V rows of the history formats.
MemoryDescriptor RecallMemory::descriptor() const {
    const Impl &m = *impl_;
    MemoryDescriptor d;
    d.identity = {"kvmem_hip", "recall-1", m.cfg.model, "recall-pages-1"};
    d.capabilities.page_tokens = m.cfg.block_tokens;
    d.capabilities.max_position = uint64_t(m.cfg.max_pages) * m.cfg.block_tokens;
    d.capabilities.native_payload = true;
    d.capabilities.sparse_view = true;
    d.capabilities.original_rope_positions = true;
    d.capabilities.pre_rope_statistics = true;
    d.capabilities.state_checkpoint = false;
    d.capabilities.asynchronous_transfer = true;
    PayloadLayout &l = d.layout;
    l.version = 1;
    l.block_tokens = m.cfg.block_tokens;
    l.alignment = 256;
    std::string fmt = "kvmem_hip/";
    uint64_t off = 0;
    for (uint32_t i = 0; i < m.layers.size(); ++i) {
        if (!m.history[i].set) continue;
        for (const kvr_plane *p : {&m.history[i].k, &m.history[i].v}) {
            PayloadPlane pl;
            pl.layer = m.layers[i];
            pl.kind = p == &m.history[i].k ? PayloadPlaneKind::Key : PayloadPlaneKind::Value;
            pl.token_stride = row_size(p->format, p->width);
            pl.bytes = pl.token_stride * m.cfg.block_tokens;
            pl.alignment = 256;
            pl.offset = (off + 255) / 256 * 256;
            off = pl.offset + pl.bytes;
            l.planes.push_back(pl);
            if (i == 0) fmt += std::string(format_name(p->format)) + (pl.kind == PayloadPlaneKind::Key ? "k-" : "v");
        }
    }
    l.format = fmt;
    l.record_bytes = (off + 255) / 256 * 256;
    return d;
}

// The restore of a prepared view: one gather of the view's pages from the
// pinned history into the slots, on the memory's copy stream; publish makes
// the view resident.
class RecallPlanTransfer final : public MemoryTransfer {
public:
    RecallPlanTransfer(RecallMemory &mem, std::vector<uint64_t> ids, uint32_t *sel, std::vector<kvr_plane> planes)
        : mem_(mem), ids_(std::move(ids)), sel_(sel) {
        const uint32_t k = uint32_t(ids_.size());
        auto &m = *mem_.impl_;
        t_ = std::make_unique<RecallTransfer>(m.ctx, std::move(planes), 1, m.cfg.block_tokens, sel_, sel_ + m.cfg.max_pages,
                                              std::max<uint32_t>(k, 1), KVR_ENGINE_KERNEL, m.copy_stream(), nullptr);
    }
    ~RecallPlanTransfer() override {
        t_.reset();
        (void)hipFree(sel_);
    }
    void start_spill() override { t_->start_spill(); }
    TransferPoll poll() override { return t_->poll(); }
    void start_restore() override { t_->start_restore(); }
    void publish(const ExecutionView &view) override {
        std::vector<uint64_t> ids;
        for (const auto &b : view.blocks) ids.push_back(b.block.id);
        if (ids != ids_) throw MemoryError(MemoryErrorCode::InvalidPlan, "published view differs from the prepared one");
        t_->publish();
        auto &m = *mem_.impl_;
        m.resident = ids_;
        ++m.view_version;
    }
    AbortResult abort() noexcept override { return t_->abort(); }

private:
    RecallMemory &mem_;
    std::vector<uint64_t> ids_;
    uint32_t *sel_;
    std::unique_ptr<RecallTransfer> t_;
};

std::unique_ptr<MemoryTransfer> RecallMemory::prepare(const WorkingSetPlan &plan) {
    Impl &m = *impl_;
    if (!m.valid) plan_error(MemoryErrorCode::InvalidSession, "recall memory was invalidated");
    if (!(plan.expected == stamp())) plan_error(MemoryErrorCode::Stale, "working-set plan does not match the memory stamp");
    std::vector<uint64_t> ids;
    const uint32_t pages = m.page_count();
    for (size_t i = 0; i < plan.next.blocks.size(); ++i) {
        const ViewBlock &vb = plan.next.blocks[i];
        if (vb.block.id >= pages || (!ids.empty() && vb.block.id <= ids.back()))
            plan_error(MemoryErrorCode::InvalidPlan, "view blocks must be distinct pages in ascending order");
        if (!(vb.block == m.block(uint32_t(vb.block.id))))
            plan_error(MemoryErrorCode::Stale, "view block is not the page's current version");
        if (vb.compact_start != uint64_t(i) * m.cfg.block_tokens)
            plan_error(MemoryErrorCode::InvalidPlan, "view block i must start at slot i");
        ids.push_back(vb.block.id);
    }
    if (ids.size() > m.slot_pages()) plan_error(MemoryErrorCode::BudgetExceeded, "view exceeds the slot pages");
    std::vector<kvr_plane> planes;
    for (const History &h : m.history) {
        if (!h.set) plan_error(MemoryErrorCode::Unsupported, "no pinned history for a served layer");
        planes.push_back(h.k);
        planes.push_back(h.v);
    }
    hip_check(hipSetDevice(m.cfg.device), "hipSetDevice");
    uint32_t *sel = nullptr;
    hip_check(hipMalloc(&sel, size_t(m.cfg.max_pages) * 4 + 256), "hipMalloc plan selection");
    try {
        std::vector<uint32_t> host(ids.begin(), ids.end());
        const uint32_t count = uint32_t(host.size());
        const hipStream_t s = m.copy_stream();
        if (count) hip_check(hipMemcpyAsync(sel, host.data(), size_t(count) * 4, hipMemcpyHostToDevice, s), "plan H2D");
        hip_check(hipMemcpyAsync(sel + m.cfg.max_pages, &count, 4, hipMemcpyHostToDevice, s), "plan H2D");
        hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
        return std::make_unique<RecallPlanTransfer>(*this, std::move(ids), sel, std::move(planes));
    } catch (...) {
        (void)hipFree(sel);
        throw;
    }
}

void RecallMemory::invalidate() noexcept {
    impl_->valid = false;
    impl_->resident.clear();
}

std::vector<uint64_t> RecallMemory::resident() const { return impl_->resident; }

}  // namespace kvmem_hip
