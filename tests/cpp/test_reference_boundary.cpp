// The adapter-side glue of INTEGRATION.md, compiled against the reference's
// own public headers (kvmem/include) and linked with the reference's host
// library as built in oracle/_ref.  TEST ONLY: built by
// kvmem_amd/build.py when the reference tree is present, never linked into
// the product libraries.
//
//   test_reference_boundary --cpu   the conversions are field for field,
//                                   query_score_frame agrees with the
//                                   reference's on random frames
//   test_reference_boundary --gpu   PageSoftmaxHip scores the reference's
//                                   own RawKvStore (score and
//                                   score_current_layer, unchanged call
//                                   shapes) like kvmem::page_softmax_scores;
//                                   a RecallTransfer driven through
//                                   kvmem::MemoryTransfer restores pages
#include "kvmem/graph_recall.hpp"
#include "kvmem/memory_contract.hpp"
#include "kvmem/native_layer_query.hpp"
#include "kvmem/raw_kv_store.hpp"

#include "kvmem_hip/kvmem_hip.hpp"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <functional>
#include <iostream>
#include <memory>
#include <random>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <vector>

// ---- the conversions an adapter writes (scorer swap) -------
#define SAME_FIELD(A, B, f) \
    static_assert(std::is_same_v<decltype(A::f), decltype(B::f)>, #A "::" #f " differs from " #B "::" #f)
SAME_FIELD(kvmem::PageQueryView, kvmem_hip::PageQueryView, data);
SAME_FIELD(kvmem::PageQueryView, kvmem_hip::PageQueryView, layer_rows);
SAME_FIELD(kvmem::PageQueryView, kvmem_hip::PageQueryView, layers);
SAME_FIELD(kvmem::PageQueryView, kvmem_hip::PageQueryView, rows);
SAME_FIELD(kvmem::PageQueryView, kvmem_hip::PageQueryView, query_heads);
SAME_FIELD(kvmem::PageQueryView, kvmem_hip::PageQueryView, kv_heads);
SAME_FIELD(kvmem::PageQueryView, kvmem_hip::PageQueryView, head_dim);
SAME_FIELD(kvmem::PageQueryView, kvmem_hip::PageQueryView, layer_data);
SAME_FIELD(kvmem::PageQueryView, kvmem_hip::PageQueryView, attention_scale);
SAME_FIELD(kvmem::QueryScoreFrame, kvmem_hip::QueryScoreFrame, starts);
SAME_FIELD(kvmem::QueryScoreFrame, kvmem_hip::QueryScoreFrame, counts);
SAME_FIELD(kvmem::QueryScoreFrame, kvmem_hip::QueryScoreFrame, score_mask);
SAME_FIELD(kvmem::QueryScoreFrame, kvmem_hip::QueryScoreFrame, transport_mask);
SAME_FIELD(kvmem::QueryScoreFrame, kvmem_hip::QueryScoreFrame, accepted_through);
SAME_FIELD(kvmem::NativeCurrentLayerQuery, kvmem_hip::NativeCurrentLayerQuery, data);
SAME_FIELD(kvmem::NativeCurrentLayerQuery, kvmem_hip::NativeCurrentLayerQuery, bytes);
SAME_FIELD(kvmem::NativeCurrentLayerQuery, kvmem_hip::NativeCurrentLayerQuery, layer);
SAME_FIELD(kvmem::NativeCurrentLayerQuery, kvmem_hip::NativeCurrentLayerQuery, rows);
SAME_FIELD(kvmem::NativeCurrentLayerQuery, kvmem_hip::NativeCurrentLayerQuery, query_heads);
SAME_FIELD(kvmem::NativeCurrentLayerQuery, kvmem_hip::NativeCurrentLayerQuery, kv_heads);
SAME_FIELD(kvmem::NativeCurrentLayerQuery, kvmem_hip::NativeCurrentLayerQuery, head_dim);
SAME_FIELD(kvmem::NativeCurrentLayerQuery, kvmem_hip::NativeCurrentLayerQuery, attention_scale);
SAME_FIELD(kvmem::NativeCurrentLayerQuery, kvmem_hip::NativeCurrentLayerQuery, row_stride);
SAME_FIELD(kvmem::NativeCurrentLayerQuery, kvmem_hip::NativeCurrentLayerQuery, head_stride);
SAME_FIELD(kvmem::NativeCurrentLayerQuery, kvmem_hip::NativeCurrentLayerQuery, dimension_stride);
SAME_FIELD(kvmem::PayloadPlane, kvmem_hip::PayloadPlane, offset);
SAME_FIELD(kvmem::PayloadPlane, kvmem_hip::PayloadPlane, bytes);
SAME_FIELD(kvmem::PayloadPlane, kvmem_hip::PayloadPlane, token_stride);
SAME_FIELD(kvmem::PayloadLayout, kvmem_hip::PayloadLayout, record_bytes);
#undef SAME_FIELD
static_assert(std::is_base_of_v<std::runtime_error, kvmem_hip::MemoryError>);

namespace adapter {
kvmem_hip::PageQueryView to_hip(const kvmem::PageQueryView &v) {
    kvmem_hip::PageQueryView h;
    h.data = v.data;
    h.layer_rows = v.layer_rows;
    h.layers = v.layers;
    h.rows = v.rows;
    h.query_heads = v.query_heads;
    h.kv_heads = v.kv_heads;
    h.head_dim = v.head_dim;
    h.layer_data = v.layer_data;
    h.attention_scale = v.attention_scale;
    return h;
}
kvmem_hip::QueryScoreFrame to_hip(const kvmem::QueryScoreFrame &f) {
    return {f.starts, f.counts, f.score_mask, f.transport_mask, f.accepted_through};
}
kvmem_hip::NativeCurrentLayerQuery to_hip(const kvmem::NativeCurrentLayerQuery &q) {
    kvmem_hip::NativeCurrentLayerQuery h;
    h.data = q.data;
    h.bytes = q.bytes;
    h.layer = q.layer;
    h.rows = q.rows;
    h.query_heads = q.query_heads;
    h.kv_heads = q.kv_heads;
    h.head_dim = q.head_dim;
    h.attention_scale = q.attention_scale;
    h.scalar = q.scalar == kvmem::NativeQueryScalar::Float16    ? kvmem_hip::NativeQueryScalar::Float16
               : q.scalar == kvmem::NativeQueryScalar::BFloat16 ? kvmem_hip::NativeQueryScalar::BFloat16
                                                                : kvmem_hip::NativeQueryScalar::Float32;
    h.row_stride = q.row_stride;
    h.head_stride = q.head_stride;
    h.dimension_stride = q.dimension_stride;
    return h;
}
kvmem_hip::GqaScoreAggregation to_hip(kvmem::GqaScoreAggregation a) {
    return a == kvmem::GqaScoreAggregation::Max ? kvmem_hip::GqaScoreAggregation::Max
                                                : kvmem_hip::GqaScoreAggregation::Mean;
}

// INTEGRATION.md, MemoryTransfer forwarding
class KvrRecallTransfer final : public kvmem::MemoryTransfer {
public:
    explicit KvrRecallTransfer(std::unique_ptr<kvmem_hip::RecallTransfer> t) : t_(std::move(t)) {}
    void start_spill() override { t_->start_spill(); }
    kvmem::TransferPoll poll() override {
        auto p = t_->poll();
        return {p.status == kvmem_hip::TransferStatus::Complete ? kvmem::TransferStatus::Complete
                : p.status == kvmem_hip::TransferStatus::Failed ? kvmem::TransferStatus::Failed
                                                                 : kvmem::TransferStatus::Pending,
                p.error};
    }
    void start_restore() override { t_->start_restore(); }
    void publish(const kvmem::ExecutionView &) override { t_->publish(); }
    kvmem::AbortResult abort() noexcept override {
        return t_->abort() == kvmem_hip::AbortResult::PreviousViewPreserved
                   ? kvmem::AbortResult::PreviousViewPreserved
                   : kvmem::AbortResult::SessionInvalidated;
    }

private:
    std::unique_ptr<kvmem_hip::RecallTransfer> t_;
};
}  // namespace adapter

namespace {
void require(bool ok, const std::string &msg) {
    if (!ok) throw std::runtime_error(msg);
}
void hip(hipError_t e, const char *what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

uint16_t f16_bits(float x) {
    _Float16 h = static_cast<_Float16>(x);
    uint16_t b;
    std::memcpy(&b, &h, 2);
    return b;
}

// A reference RawKvStore holding fp16 keys [layers][tokens][width].
std::unique_ptr<kvmem::RawKvStore> make_store(const std::vector<uint16_t> &keys, uint32_t layers, uint32_t tokens,
                                              uint32_t width, uint32_t block) {
    kvmem::RawKvStoreConfig cfg;
    cfg.n_layer = layers;
    cfg.n_embd_k = width;
    cfg.n_embd_v = 0;
    cfg.block_tokens = block;
    auto store = std::make_unique<kvmem::RawKvStore>(cfg);
    for (uint32_t l = 0; l < layers; ++l)
        store->write_layer_tokens_f16(0, tokens, l, keys.data() + size_t(l) * tokens * width, nullptr);
    return store;
}

void conversions() {
    std::vector<float> q(8);
    std::vector<uint32_t> rows{1, 0};
    kvmem::PageQueryView v;
    v.data = q.data();
    v.layer_rows = rows.data();
    v.layers = 2;
    v.rows = 1;
    v.query_heads = 4;
    v.kv_heads = 2;
    v.head_dim = 2;
    v.attention_scale = .5f;
    const auto h = adapter::to_hip(v);
    require(h.data == v.data && h.layer_rows == v.layer_rows && h.layers == 2 && h.rows == 1 && h.query_heads == 4 &&
                h.kv_heads == 2 && h.head_dim == 2 && h.attention_scale == .5f,
            "PageQueryView conversion");
    kvmem::NativeCurrentLayerQuery n;
    n.data = q.data();
    n.bytes = 32;
    n.layer = 1;
    n.rows = 1;
    n.query_heads = 4;
    n.kv_heads = 2;
    n.head_dim = 2;
    n.scalar = kvmem::NativeQueryScalar::Float32;
    n.row_stride = 32;
    n.head_stride = 8;
    n.dimension_stride = 4;
    const auto hn = adapter::to_hip(n);
    require(hn.layer == 1 && hn.bytes == 32 && hn.row_stride == 32 && hn.head_stride == 8 &&
                hn.dimension_stride == 4 && hn.scalar == kvmem_hip::NativeQueryScalar::Float32,
            "NativeCurrentLayerQuery conversion");
    kvmem_hip::validate_native_layer_query(hn);
    kvmem::validate_native_layer_query(n);
}

void frames() {
    std::mt19937_64 rng(91);
    for (int t = 0; t < 3000; ++t) {
        const uint32_t bt = 1 + uint32_t(rng() % 300), budget = uint32_t(rng() % 40), sink = uint32_t(rng() % 4),
                       recent = uint32_t(rng() % 6);
        const uint64_t accepted = rng() % 20000;
        std::vector<uint32_t> fixed;
        for (int i = int(rng() % 4); i > 0; --i) fixed.push_back(uint32_t(rng() % 80));
        std::string mine, theirs;
        kvmem_hip::QueryScoreFrame a;
        kvmem::QueryScoreFrame b;
        try {
            a = kvmem_hip::query_score_frame(accepted, bt, budget, sink, recent, fixed);
        } catch (const std::exception &e) {
            mine = e.what();
        }
        try {
            b = kvmem::query_score_frame(accepted, bt, budget, sink, recent, fixed);
        } catch (const std::exception &e) {
            theirs = e.what();
        }
        require(mine.empty() == theirs.empty(), "query_score_frame: one side threw: '" + mine + "' / '" + theirs + "'");
        const auto c = adapter::to_hip(b);
        require(a.starts == c.starts && a.counts == c.counts && a.score_mask == c.score_mask &&
                    a.transport_mask == c.transport_mask && a.accepted_through == c.accepted_through,
                "query_score_frame differs from the reference's");
    }
}

// PageSoftmaxHip::score / score_current_layer on the reference's own
// RawKvStore, against kvmem::page_softmax_scores on the same store.
void scores_on_reference_store() {
    const uint32_t layers = 3, tokens = 4000, kvh = 2, hd = 64, hq = 8, width = kvh * hd, block = 128, rows = 3;
    std::mt19937_64 rng(92);
    std::normal_distribution<float> nd(0.f, 1.f);
    std::vector<uint16_t> keys(size_t(layers) * tokens * width);
    for (auto &k : keys) k = f16_bits(nd(rng));
    auto store = make_store(keys, layers, tokens, width, block);
    std::vector<float> q(size_t(layers) * rows * hq * hd);
    for (auto &x : q) x = nd(rng);
    std::vector<uint32_t> layer_rows{rows, 0, 2};
    kvmem::PageQueryView view;
    view.data = q.data();
    view.layer_rows = layer_rows.data();
    view.layers = layers;
    view.rows = rows;
    view.query_heads = hq;
    view.kv_heads = kvh;
    view.head_dim = hd;
    kvmem_hip::PageSoftmaxHip scorer(0);
    const uint32_t pages = (tokens + block - 1) / block;
    for (auto agg : {kvmem::GqaScoreAggregation::Mean, kvmem::GqaScoreAggregation::Max}) {
        for (uint32_t budget : {pages, 12u}) {
            const auto frame = kvmem::query_score_frame(tokens, block, budget, 1, 2, {5});
            const auto want = kvmem::page_softmax_scores(*store, view, frame, agg);
            // the adapter's call, unchanged but for the namespaces of the view and frame
            const auto got = scorer.score(*store, adapter::to_hip(view), adapter::to_hip(frame), adapter::to_hip(agg));
            require(got.size() == want.size(), "score size");
            for (size_t i = 0; i < got.size(); ++i)
                require(std::fabs(got[i] - want[i]) <= 1e-9 * std::max(1.0, std::fabs(want[i])),
                        "score on the reference store differs at page " + std::to_string(i));
        }
    }
    // a frame entry the store does not hold is a stale index extent
    auto stale = kvmem::query_score_frame(tokens + 5 * block, block, pages + 5, 0, 0, {});
    bool threw = false;
    try {
        scorer.score(*store, adapter::to_hip(view), adapter::to_hip(stale));
    } catch (const std::invalid_argument &) {
        threw = true;
    }
    require(threw, "stale frame accepted");

    // current layer: device Query of layer 2, Mean, against the reference's
    // multi-layer scores with only layer 2 active
    const uint32_t layer = 2;
    float *qd = nullptr;
    hip(hipMalloc(&qd, size_t(rows) * hq * hd * 4), "hipMalloc");
    hip(hipMemcpy(qd, q.data() + size_t(layer) * rows * hq * hd, size_t(rows) * hq * hd * 4, hipMemcpyHostToDevice),
        "H2D");
    kvmem::NativeCurrentLayerQuery nq;
    nq.data = qd;
    nq.bytes = size_t(rows) * hq * hd * 4;
    nq.layer = layer;
    nq.rows = rows;
    nq.query_heads = hq;
    nq.kv_heads = kvh;
    nq.head_dim = hd;
    nq.scalar = kvmem::NativeQueryScalar::Float32;
    nq.row_stride = size_t(hq) * hd * 4;
    nq.head_stride = size_t(hd) * 4;
    nq.dimension_stride = 4;
    const auto frame = kvmem::query_score_frame(tokens, block, 20, 1, 2, {});
    std::vector<uint32_t> only{0, 0, rows};
    kvmem::PageQueryView single = view;
    single.layer_rows = only.data();
    const auto want = kvmem::page_softmax_scores(*store, single, frame, kvmem::GqaScoreAggregation::Mean);
    const auto got = scorer.score_current_layer(*store, adapter::to_hip(nq), adapter::to_hip(frame), nullptr);
    for (size_t i = 0; i < got.size(); ++i)
        require(std::fabs(got[i] - want[i]) <= 1e-9 * std::max(1.0, std::fabs(want[i])),
                "current-layer score on the reference store differs at page " + std::to_string(i));
    hip(hipFree(qd), "hipFree");
}

// A RecallTransfer driven through the reference's MemoryTransfer interface.
void transfer_through_reference_interface() {
    const uint32_t tokens = 1024, width = 256, pt = 128, k = 3;
    kvr_context *ctx = nullptr;
    require(kvr_create(0, &ctx) == KVR_OK, "kvr_create");
    void *hist = nullptr;
    require(kvr_host_alloc(size_t(tokens) * width * 2, &hist) == KVR_OK, "kvr_host_alloc");
    auto *h = static_cast<uint8_t *>(hist);
    for (size_t i = 0; i < size_t(tokens) * width * 2; ++i) h[i] = uint8_t(i * 131 + 7);
    const uint32_t sel[k] = {1, 4, 6}, cnt = k;
    uint32_t *seld = nullptr, *cntd = nullptr;
    uint8_t *slots = nullptr;
    hip(hipMalloc(&seld, sizeof sel), "hipMalloc");
    hip(hipMalloc(&cntd, 4), "hipMalloc");
    hip(hipMalloc(&slots, size_t(k) * pt * width * 2), "hipMalloc");
    hip(hipMemcpy(seld, sel, sizeof sel, hipMemcpyHostToDevice), "H2D");
    hip(hipMemcpy(cntd, &cnt, 4, hipMemcpyHostToDevice), "H2D");
    kvr_plane plane{};
    plane.history = hist;
    plane.format = KVR_FMT_F16;
    plane.width = width;
    plane.tokens = tokens;
    plane.mode = KVR_GATHER_COPY;
    plane.slots = slots;
    {
        std::unique_ptr<kvmem::MemoryTransfer> t = std::make_unique<adapter::KvrRecallTransfer>(
            std::make_unique<kvmem_hip::RecallTransfer>(ctx, std::vector<kvr_plane>{plane}, 1, pt, seld, cntd, k));
        t->start_spill();
        while (t->poll().status == kvmem::TransferStatus::Pending) {
        }
        t->start_restore();
        kvmem::TransferPoll p;
        while ((p = t->poll()).status == kvmem::TransferStatus::Pending) {
        }
        require(p.status == kvmem::TransferStatus::Complete, "restore failed: " + p.error);
        t->publish(kvmem::ExecutionView{});
    }
    std::vector<uint8_t> got(size_t(k) * pt * width * 2);
    hip(hipMemcpy(got.data(), slots, got.size(), hipMemcpyDeviceToHost), "D2H");
    const size_t span = size_t(pt) * width * 2;
    for (uint32_t s = 0; s < k; ++s)
        require(std::memcmp(got.data() + s * span, h + size_t(sel[s]) * span, span) == 0, "restored page bytes");
    (void)hipFree(seld);
    (void)hipFree(cntd);
    (void)hipFree(slots);
    (void)kvr_host_free(hist);
    (void)kvr_destroy(ctx);
}
}  // namespace

int main(int argc, char **argv) {
    const bool gpu = argc > 1 && std::string(argv[1]) == "--gpu";
    std::vector<std::pair<const char *, std::function<void()>>> tests = {{"conversions", conversions},
                                                                        {"frames", frames}};
    if (gpu)
        tests = {{"scores_on_reference_store", scores_on_reference_store},
                 {"transfer_through_reference_interface", transfer_through_reference_interface}};
    for (auto &[name, fn] : tests) {
        std::cout << "RUN  " << name << std::endl;
        try {
            fn();
        } catch (const std::exception &e) {
            std::cout << "FAIL " << name << ": " << e.what() << std::endl;
            return 1;
        }
        std::cout << "PASS " << name << std::endl;
    }
    return 0;
}
