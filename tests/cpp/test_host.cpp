// Tests of the C++ host layer (include/kvmem_hip/kvmem_hip.hpp), written like
// the reference's own C++ tests (kvmem/tests/graph_recall_test.cpp,
// graph_recall_cuda_test.cpp): plain main, `require`, exceptions as failures.
// The oracle (oracle/kvr_oracle.h) is the checker.
//   test_host --cpu   host-only checks (no device calls)
//   test_host --gpu   scorer, selection, stage-in, transfer and capture on cuda:0
#include "kvmem_hip/kvmem_hip.hpp"
#include "kvr_oracle.h"

#include <dlfcn.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <iostream>
#include <map>
#include <numeric>
#include <random>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

namespace kh = kvmem_hip;

namespace {

void require(bool ok, const std::string &msg) {
    if (!ok) throw std::runtime_error(msg);
}
template <class E, class F> void rejects(F f, const std::string &msg) {
    bool thrown = false;
    try {
        f();
    } catch (const E &) {
        thrown = true;
    }
    require(thrown, msg);
}
void hip(hipError_t e, const char *what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

template <class T> struct Dev {
    T *p = nullptr;
    size_t n = 0;
    explicit Dev(size_t count) : n(count) { hip(hipMalloc(&p, std::max<size_t>(1, n) * sizeof(T)), "hipMalloc"); }
    Dev(const std::vector<T> &h) : Dev(h.size()) { up(h); }
    ~Dev() { (void)hipFree(p); }
    Dev(const Dev &) = delete;
    void up(const std::vector<T> &h) {
        hip(hipMemcpy(p, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice), "H2D");
    }
    std::vector<T> down() const {
        std::vector<T> h(n);
        hip(hipMemcpy(h.data(), p, n * sizeof(T), hipMemcpyDeviceToHost), "D2H");
        return h;
    }
};

double rel_err(const std::vector<double> &a, const std::vector<double> &b) {
    double w = 0;
    for (size_t i = 0; i < a.size(); ++i) w = std::max(w, std::abs(a[i] - b[i]) / std::max(std::abs(b[i]), 1e-300));
    return w;
}

// ---- host-only -------------------------------------------------------------
void frames() {
    // graph_recall_test.cpp:23-31
    auto frame = kh::query_score_frame(12, 4, 2, 0, 0, {2});
    require(frame.score_mask == std::vector<uint8_t>({1, 1, 1}), "mandatory changed softmax denominator");
    require(frame.transport_mask == std::vector<uint8_t>({1, 1, 0}), "mandatory transported graph mass");
    auto small = kh::query_score_frame(11, 4, 4, 1, 1, {0, 2});
    require(small.score_mask == std::vector<uint8_t>({1, 1, 1}) &&
                small.transport_mask == std::vector<uint8_t>({0, 0, 0}) && small.counts.back() == 3,
            "small-history or partial-tail domain mismatch");
    auto constrained = kh::query_score_frame(12, 4, 2, 1, 1, {0, 2});
    require(constrained.score_mask == std::vector<uint8_t>({0, 1, 0}), "keep-band score mask mismatch");
    rejects<std::invalid_argument>([] { kh::query_score_frame(12, 0, 2, 0, 0, {}); }, "zero block size accepted");
    rejects<std::invalid_argument>([] { kh::query_score_frame(12, 4, 0, 0, 0, {}); }, "zero budget accepted");
    rejects<std::invalid_argument>([] { kh::query_score_frame(12, 4, 2, 0, 0, {3}); }, "outside fixed block accepted");
    // against the oracle on random frames
    std::mt19937_64 rng(7);
    for (int trial = 0; trial < 300; ++trial) {
        const uint64_t accepted = rng() % 5000;
        const uint32_t bt = 1 + rng() % 300, budget = 1 + rng() % 40, sink = rng() % 5, recent = rng() % 5;
        const uint32_t pages = uint32_t((accepted + bt - 1) / bt);
        std::vector<uint32_t> fixed;
        for (uint32_t i = 0; pages && i < 3; ++i) fixed.push_back(uint32_t(rng() % pages));
        auto f = kh::query_score_frame(accepted, bt, budget, sink, recent, fixed);
        std::vector<uint64_t> st(pages + 1);
        std::vector<uint32_t> ct(pages + 1);
        std::vector<uint8_t> sm(pages + 1), tm(pages + 1);
        require(orc_query_score_frame(accepted, bt, budget, sink, recent, fixed.data(), uint32_t(fixed.size()),
                                      st.data(), ct.data(), sm.data(), tm.data()) == ORC_OK,
                "oracle frame failed");
        for (uint32_t i = 0; i < pages; ++i)
            require(f.starts[i] == st[i] && f.counts[i] == ct[i] && f.score_mask[i] == sm[i] &&
                        f.transport_mask[i] == tm[i],
                    "frame differs from the oracle");
    }
}

void native_query_geometry() {
    alignas(16) static uint16_t storage[4 * 8 * 64];
    kh::NativeCurrentLayerQuery q;
    q.data = storage;
    q.bytes = sizeof storage;
    q.rows = 4;
    q.query_heads = 8;
    q.kv_heads = 2;
    q.head_dim = 64;
    q.scalar = kh::NativeQueryScalar::Float16;
    q.row_stride = 8 * 64 * 2;
    q.head_stride = 64 * 2;
    q.dimension_stride = 2;
    kh::validate_native_layer_query(q);
    auto heads_outer = q;  // [head][row][dim] is a valid permutation
    heads_outer.head_stride = 4 * 64 * 2;
    heads_outer.row_stride = 64 * 2;
    kh::validate_native_layer_query(heads_outer);
    auto overlap = q;
    overlap.row_stride = 64 * 2;
    rejects<std::invalid_argument>([&] { kh::validate_native_layer_query(overlap); }, "overlapping strides accepted");
    auto small = q;
    small.bytes = sizeof storage - 2;
    rejects<std::invalid_argument>([&] { kh::validate_native_layer_query(small); }, "extent overflow accepted");
    auto group = q;
    group.kv_heads = 3;
    rejects<std::invalid_argument>([&] { kh::validate_native_layer_query(group); }, "ragged GQA group accepted");
    auto misaligned = q;
    misaligned.data = reinterpret_cast<const uint8_t *>(storage) + 1;
    rejects<std::invalid_argument>([&] { kh::validate_native_layer_query(misaligned); }, "misaligned Query accepted");
}

void workspace_geometry() {
    const size_t a = kh::PageSoftmaxHip::workspace_bytes(7, 8, 2, 256);
    const size_t b = kh::PageSoftmaxHip::workspace_bytes(8192, 8, 2, 256);
    require(a > 0 && b > a && a % 256 == 0, "workspace arithmetic");
    rejects<std::invalid_argument>([] { kh::PageSoftmaxHip::workspace_bytes(0, 8, 2, 64); }, "zero pages planned");
    rejects<std::invalid_argument>([] { kh::PageSoftmaxHip::workspace_bytes(8, 6, 4, 64); }, "ragged group planned");
    rejects<std::invalid_argument>([] { kh::PageSoftmaxHip::workspace_bytes(1u << 22, 32, 8, 128); },
                                   "logits beyond 64 MiB planned");
}

void stagein_without_state() {
    uint8_t b = 0;
    require(!kh::kvmem_stagein_enqueue_v(&b, 1, &b, nullptr), "enqueue accepted before gpu_ready");
    require(!kh::kvmem_stagein_sync_checked(), "sync_checked without a state");
}

// ---- device ----------------------------------------------------------------
struct Stack {
    uint32_t layers, pages, rows, dim, qheads, kvheads;
    std::vector<float> means;  // [layers][pages][kw]
    std::vector<float> query;  // [layers][rows][qheads][dim]
    std::vector<Dev<uint16_t> *> dev;
    kh::PageSummaries sums;
    ~Stack() {
        for (auto *d : dev) delete d;
    }
};

// graph_recall_cuda_test.cpp:18-35 closed-form inputs: per-block key sums of
// four tokens, mean = sum * (1/4).
void build_stack(Stack &s) {
    const size_t kw = size_t(s.kvheads) * s.dim, qw = size_t(s.qheads) * s.dim;
    s.means.assign(size_t(s.layers) * s.pages * kw, 0.f);
    for (uint32_t l = 0; l < s.layers; ++l)
        for (uint32_t b = 0; b < s.pages; ++b)
            for (size_t d = 0; d < kw; ++d)
                s.means[(size_t(l) * s.pages + b) * kw + d] =
                    float(int((b * 13 + d * 7 + l * 11) % 101) - 50) / 16 * (1.0f / 4);
    s.query.resize(size_t(s.layers) * s.rows * qw);
    for (size_t d = 0; d < s.query.size(); ++d) s.query[d] = float(int((d * 17) % 127) - 63) / 32;
    s.sums.pages = s.pages;
    s.sums.page_tokens = 4;
    s.sums.kv_heads = s.kvheads;
    s.sums.head_dim = s.dim;
    for (uint32_t l = 0; l < s.layers; ++l) {
        std::vector<uint16_t> h(size_t(s.pages) * kw);
        for (size_t i = 0; i < h.size(); ++i) h[i] = orc_f32_to_f16(s.means[size_t(l) * s.pages * kw + i]);
        s.dev.push_back(new Dev<uint16_t>(h));
        s.sums.layers.push_back(s.dev.back()->p);
    }
}

void qualification() {
    kh::PageSoftmaxHip scorer(0);
    struct Shape { uint32_t blocks, rows, dim, qheads, kvheads; };
    for (auto agg : {kh::GqaScoreAggregation::Mean, kh::GqaScoreAggregation::Max, kh::GqaScoreAggregation::MaxLogit})
        for (auto sh : {Shape{7, 129, 256, 8, 2}, Shape{8192, 2, 64, 4, 1}, Shape{8193, 2, 64, 4, 1},
                        Shape{32769, 1, 64, 2, 1}}) {
            Stack s{2, sh.blocks, sh.rows, sh.dim, sh.qheads, sh.kvheads};
            build_stack(s);
            const uint32_t counts[]{sh.rows, sh.rows};
            auto frame = kh::query_score_frame(uint64_t(sh.blocks) * 4, 4, 3, 1, 1, {0, sh.blocks - 1});
            kh::PageQueryView view{s.query.data(), counts, 2, sh.rows, sh.qheads, sh.kvheads, sh.dim};
            std::vector<double> expected(sh.blocks);
            const int oagg = agg == kh::GqaScoreAggregation::Mean ? ORC_AGG_MEAN
                             : agg == kh::GqaScoreAggregation::Max ? ORC_AGG_MAX : ORC_AGG_MAX_LOGIT;
            require(orc_page_softmax_scores(s.means.data(), s.query.data(), counts, 2, sh.rows, sh.qheads,
                                            sh.kvheads, sh.dim, sh.blocks, frame.score_mask.data(), 0, oagg,
                                            expected.data()) == ORC_OK,
                    "oracle scores failed");
            const auto actual = scorer.score(s.sums, view, frame, agg);
            require(actual.size() == expected.size(), "score length");
            for (size_t b = 0; b < actual.size(); ++b)
                require(std::isfinite(actual[b]) && std::abs(actual[b] - expected[b]) <= 2e-6 + expected[b] * 3e-5,
                        "page softmax differs from the oracle beyond the reference bound");
            const double err = rel_err(actual, expected);
            require(err <= 1e-9, "page softmax differs from the oracle beyond 1e-9");
            const double mass = std::accumulate(actual.begin(), actual.end(), 0.0);
            if (agg != kh::GqaScoreAggregation::MaxLogit)
                require(std::abs(mass - sh.rows) <= sh.rows * 1e-12 * 64, "softmax mass was lost");
            if (sh.blocks == 7) {
                const size_t bytes = kh::PageSoftmaxHip::workspace_bytes(sh.blocks, sh.qheads, sh.kvheads, sh.dim);
                Dev<uint8_t> ws(bytes);
                kh::PageSoftmaxHip borrowed(0, ws.p, bytes, sh.blocks, sh.qheads, sh.kvheads, sh.dim);
                const auto planned = borrowed.score(s.sums, view, frame, agg);
                require(rel_err(planned, expected) <= 1e-9, "planned workspace differs from the oracle");
                require(borrowed.device_bytes() <= bytes, "borrowed scorer owns device memory");
                Stack big{2, 8, sh.rows, sh.dim, sh.qheads, sh.kvheads};
                build_stack(big);
                auto f8 = kh::query_score_frame(8 * 4, 4, 3, 1, 1, {});
                rejects<std::length_error>([&] { borrowed.score(big.sums, view, f8, agg); },
                                           "borrowed workspace grew");
            }
            std::cout << "  agg=" << int(agg) << " pages=" << sh.blocks << " rows=" << sh.rows << " D=" << sh.dim
                      << " rel_err=" << err << "\n";
        }
    Stack s{2, 16, 2, 64, 4, 1};
    build_stack(s);
    const uint32_t counts[]{2, 2};
    kh::PageQueryView view{s.query.data(), counts, 2, 2, 4, 1, 64};
    auto short_frame = kh::query_score_frame(17 * 4, 4, 3, 0, 0, {});
    rejects<std::invalid_argument>([&] { scorer.score(s.sums, view, short_frame); }, "frame beyond summaries accepted");
    kh::PageQueryView bad = view;
    bad.kv_heads = 3;
    auto frame = kh::query_score_frame(16 * 4, 4, 3, 0, 0, {});
    rejects<std::invalid_argument>([&] { scorer.score(s.sums, bad, frame); }, "ragged heads accepted");
}

void current_layer() {
    kh::PageSoftmaxHip scorer(0);
    const uint32_t pages = 300, rows = 3, qh = 8, kvh = 2, dim = 64;
    Stack s{2, pages, rows, dim, qh, kvh};
    build_stack(s);
    // layer 1's query rows as fp16 in [head][row][dim] order on the device
    const size_t qw = size_t(qh) * dim;
    std::vector<uint16_t> qh16(size_t(qh) * rows * dim);
    std::vector<float> qf(size_t(rows) * qw);
    for (uint32_t r = 0; r < rows; ++r)
        for (uint32_t h = 0; h < qh; ++h)
            for (uint32_t d = 0; d < dim; ++d) {
                const float x = s.query[size_t(rows) * qw + r * qw + h * dim + d];
                const uint16_t b = orc_f32_to_f16(x);
                qh16[(size_t(h) * rows + r) * dim + d] = b;
                qf[r * qw + h * dim + d] = orc_f16_to_f32(b);
            }
    Dev<uint16_t> qd(qh16);
    kh::NativeCurrentLayerQuery q;
    q.data = qd.p;
    q.bytes = qh16.size() * 2;
    q.layer = 1;
    q.rows = rows;
    q.query_heads = qh;
    q.kv_heads = kvh;
    q.head_dim = dim;
    q.scalar = kh::NativeQueryScalar::Float16;
    q.row_stride = dim * 2;
    q.head_stride = size_t(rows) * dim * 2;
    q.dimension_stride = 2;
    auto frame = kh::query_score_frame(uint64_t(pages) * 4, 4, 10, 2, 3, {});
    hipStream_t producer;
    hip(hipStreamCreateWithFlags(&producer, hipStreamNonBlocking), "stream");
    const auto got = scorer.score_current_layer(s.sums, q, frame, producer);
    hip(hipStreamDestroy(producer), "stream");
    const uint32_t one[]{rows};
    std::vector<double> expected(pages);
    require(orc_page_softmax_scores(s.means.data() + size_t(pages) * kvh * dim, qf.data(), one, 1, rows, qh, kvh,
                                    dim, pages, frame.score_mask.data(), 0, ORC_AGG_MEAN, expected.data()) == ORC_OK,
            "oracle scores failed");
    require(rel_err(got, expected) <= 1e-9, "current-layer scores differ from the oracle");
    for (uint32_t j = 0; j < pages; ++j)
        if (!frame.score_mask[j]) require(got[j] == 0.0, "masked page scored");
    std::vector<float> host_q(size_t(rows) * qw);
    kh::NativeCurrentLayerQuery on_host = q;
    on_host.data = host_q.data();
    on_host.bytes = host_q.size() * 4;
    on_host.scalar = kh::NativeQueryScalar::Float32;
    on_host.row_stride = qw * 4;
    on_host.head_stride = dim * 4;
    on_host.dimension_stride = 4;
    rejects<std::invalid_argument>([&] { scorer.score_current_layer(s.sums, on_host, frame, nullptr); },
                                   "host Query accepted as device Query");
}

void pick() {
    kh::PageSoftmaxHip scorer(0);
    std::mt19937_64 rng(11);
    for (int trial = 0; trial < 60; ++trial) {
        const uint32_t n = 1 + uint32_t(rng() % 3000), budget = 1 + uint32_t(rng() % 100);
        std::vector<double> scores(n);
        std::uniform_real_distribution<double> u(0, 1);
        for (auto &x : scores) x = u(rng);
        for (uint32_t i = 0; i < n / 3; ++i) scores[rng() % n] = scores[rng() % n];  // exact ties
        std::vector<uint32_t> mand;
        for (uint32_t i = 0; i < std::min<uint32_t>({3, budget, n}); ++i) mand.push_back(uint32_t(rng() % n));
        std::sort(mand.begin(), mand.end());
        mand.erase(std::unique(mand.begin(), mand.end()), mand.end());
        for (auto tie : {kh::TieRule::LowerFirst, kh::TieRule::HigherFirst}) {
            const auto got = scorer.pick(scores, budget, mand, tie);
            std::vector<uint32_t> want(std::min(budget, n) + 1);
            uint32_t nw = 0;
            require(orc_pick_scored_blocks(scores.data(), n, mand.data(), uint32_t(mand.size()), budget,
                                           tie == kh::TieRule::HigherFirst ? ORC_TIE_HIGHER_FIRST
                                                                           : ORC_TIE_LOWER_FIRST,
                                           0, want.data(), &nw) == ORC_OK,
                    "oracle pick failed");
            want.resize(nw);
            require(got == want, "selection differs from the oracle");
        }
    }
    // layerwise_selection_test.cpp:184-194: equal mass over six pages keeps {4,5}
    require(scorer.pick(std::vector<double>(6, 1.0 / 6), 2, {}, kh::TieRule::HigherFirst) ==
                std::vector<uint32_t>({4, 5}),
            "reference tie rule");
    // graph_recall_test.cpp:101-105: signed order
    require(scorer.pick({-.8, -.2, -.5}, 2, {}, kh::TieRule::HigherFirst, true) == std::vector<uint32_t>({1, 2}),
            "signed order");
    rejects<std::invalid_argument>([&] { scorer.pick({-.8, -.2, -.5}, 2); }, "negative scores accepted");
    rejects<std::runtime_error>([&] { scorer.pick({1, 2, 3}, 1, {0, 1}); }, "mandatory over budget accepted");
    require(scorer.pick({3, 1, 2}, 10) == std::vector<uint32_t>({0, 1, 2}), "budget above page count");
}

void stagein() {
    require(kh::kvmem_stagein_gpu_ready(0, 0), "gpu_ready");
    const size_t total = size_t(48) << 20;
    Dev<uint8_t> dst(total);
    hip(hipMemset(dst.p, 0, total), "memset");
    std::mt19937_64 rng(5);
    std::vector<uint8_t> want(total, 0);
    size_t off = 0;
    int records = 0;
    while (off < total - (1 << 20)) {
        const size_t n = 1 + rng() % (600 << 10);
        std::vector<uint8_t> rec(n);
        for (auto &b : rec) b = uint8_t(rng());
        require(kh::kvmem_stagein_enqueue_v(rec.data(), n, dst.p + off, nullptr), "enqueue_v");
        std::memcpy(want.data() + off, rec.data(), n);
        std::fill(rec.begin(), rec.end(), 0);  // the caller's buffer is reusable on return
        off += n + rng() % 64;
        ++records;
    }
    int64_t copy_us = 0, rope_us = -1, had_us = -1, set_us = 0;
    require(kh::kvmem_stagein_flush(&copy_us, &rope_us, &had_us, &set_us), "flush");
    require(kh::kvmem_stagein_sync_checked(), "sync_checked");
    require(dst.down() == want, "staged bytes differ");
    std::vector<uint8_t> host(4096);
    for (size_t i = 0; i < host.size(); ++i) host[i] = uint8_t(i * 7);
    require(kh::kvmem_stagein_h2d_bytes(dst.p + 123, host.data(), host.size()), "h2d_bytes");
    std::vector<const void *> src{dst.p + 123};
    std::vector<void *> to{dst.p + (40 << 20)};
    std::vector<size_t> nb{host.size()};
    require(kh::kvmem_d2d_batched(src.data(), to.data(), nb.data(), 1), "d2d");
    require(kh::kvmem_stagein_sync_checked(), "sync_checked");
    const auto back = dst.down();
    require(std::equal(host.begin(), host.end(), back.begin() + 123) &&
                std::equal(host.begin(), host.end(), back.begin() + (40 << 20)),
            "h2d / d2d bytes differ");
    std::cout << "  " << records << " records, " << off << " bytes through two 32 MiB slabs\n";
}

void meank() {
    const uint32_t layers = 2, heads = 2, dim = 64, embd = heads * dim, tokens = 10;
    require(kh::kvmem_meank_ready(layers, embd), "meank_ready");
    // fp16 K [token][head][dim] with padding between tokens
    const size_t nb0 = 2, nb1 = dim * 2, nb2 = embd * 2 + 32;
    std::vector<uint16_t> k(tokens * nb2 / 2);
    orc_synth_normal_f16(3, 9, k.size(), k.data());
    Dev<uint16_t> kd(k);
    require(kh::kvmem_meank_add(1, KVR_FMT_F16, kd.p, 0, 4, embd, dim, nb0, nb1, nb2), "meank add");
    require(kh::kvmem_meank_add(1, KVR_FMT_F16, kd.p, 4, 6, embd, dim, nb0, nb1, nb2), "meank add");
    std::vector<float> got(embd), want(embd, 0.f);
    require(kh::kvmem_meank_d2h(1, got.data(), embd), "meank d2h");
    for (uint32_t c = 0; c < embd; ++c)
        for (uint32_t t = 0; t < tokens; ++t)
            want[c] += orc_f16_to_f32(k[(t * nb2 + (c / dim) * nb1 + (c % dim) * nb0) / 2]);
    require(std::memcmp(got.data(), want.data(), embd * 4) == 0, "running mean-K differs from the token-order sum");
    kh::kvmem_meank_zero(1);
    require(kh::kvmem_meank_d2h(1, got.data(), embd), "meank d2h");
    require(std::all_of(got.begin(), got.end(), [](float x) { return x == 0.f; }), "meank_zero left values");
    require(!kh::kvmem_meank_add(5, KVR_FMT_F16, kd.p, 0, 1, embd, dim, nb0, nb1, nb2), "layer out of range");
    kh::kvmem_meank_free();
}

void transfer() {
    kvr_context *ctx = nullptr;
    require(kvr_create(0, &ctx) == KVR_OK, "context");
    const uint32_t T = 4096, W = 256, PT = 256, P = T / PT, K = 5;
    std::vector<uint16_t> hist(size_t(T) * W);
    orc_synth_normal_f16(4, 1, hist.size(), hist.data());
    void *pin = nullptr;
    require(kvr_host_alloc(hist.size() * 2, &pin) == KVR_OK, "pinned");
    std::memcpy(pin, hist.data(), hist.size() * 2);
    std::vector<double> scores(P);
    for (uint32_t j = 0; j < P; ++j) scores[j] = double((j * 7) % P);
    Dev<double> sd(scores);
    Dev<uint32_t> sel(K), cnt(1);
    Dev<uint16_t> slots(size_t(K) * PT * W);
    require(kvr_select_topk(ctx, sd.p, 1, P, K, nullptr, 0, KVR_TIE_LOWER_FIRST, 0, sel.p, cnt.p, nullptr) == KVR_OK,
            "select");
    kvr_plane plane{};
    plane.history = pin;
    plane.format = KVR_FMT_F16;
    plane.width = W;
    plane.tokens = T;
    plane.mode = KVR_GATHER_COPY;
    plane.slots = slots.p;
    hipEvent_t ready;
    hip(hipEventCreateWithFlags(&ready, hipEventDisableTiming), "event");
    hip(hipEventRecord(ready, static_cast<hipStream_t>(kvr_select_stream(ctx))), "event");
    {
        kh::RecallTransfer t(ctx, {plane}, 1, PT, sel.p, cnt.p, K, KVR_ENGINE_KERNEL, nullptr, ready);
        require(t.poll().status == kh::TransferStatus::Pending, "pending before spill");
        rejects<std::logic_error>([&] { t.start_restore(); }, "restore before spill accepted");
        t.start_spill();
        require(t.poll().status == kh::TransferStatus::Complete, "spill completes at once");
        rejects<std::logic_error>([&] { t.publish(); }, "publish before restore accepted");
        t.start_restore();
        const auto t0 = std::chrono::steady_clock::now();
        kh::TransferPoll p;
        while ((p = t.poll()).status == kh::TransferStatus::Pending) {
            require(std::chrono::steady_clock::now() - t0 < std::chrono::seconds(10), "restore never completed");
            std::this_thread::sleep_for(std::chrono::microseconds(100));
        }
        require(p.status == kh::TransferStatus::Complete, "restore failed: " + p.error);
        t.publish();
        require(t.published(), "published");
    }
    const auto picked = sel.down();
    std::vector<uint8_t> want(size_t(K) * PT * W * 2);
    require(orc_gather(reinterpret_cast<const uint8_t *>(hist.data()), ORC_FMT_F16, W, T, PT, picked.data(), K,
                       ORC_GATHER_COPY, want.data()) == ORC_OK,
            "oracle gather");
    const auto got = slots.down();
    require(std::memcmp(got.data(), want.data(), want.size()) == 0, "restored slots differ from the oracle gather");
    {
        kh::RecallTransfer fresh(ctx, {plane}, 1, PT, sel.p, cnt.p, K);
        require(fresh.abort() == kh::AbortResult::PreviousViewPreserved, "abort before restore keeps the view");
        kh::RecallTransfer used(ctx, {plane}, 1, PT, sel.p, cnt.p, K);
        used.start_spill();
        used.start_restore();
        require(used.abort() == kh::AbortResult::SessionInvalidated, "abort after restore invalidates");
        require(used.poll().status == kh::TransferStatus::Failed, "aborted transfer polls failed");
    }
    hip(hipEventDestroy(ready), "event");
    require(kvr_check(ctx, nullptr) == KVR_OK, "check");
    kvr_host_free(pin);
    kvr_destroy(ctx);
}

void capture() {
    kvr_context *ctx = nullptr;
    require(kvr_create(0, &ctx) == KVR_OK, "context");
    const uint32_t layers = 2, pages = 16, pt = 64, kvh = 2, dim = 64, W = kvh * dim, T = pages * pt - 19;
    {  // the capture is destroyed before its context
    kh::SummaryCapture cap(ctx, layers, pages, pt, kvh, dim);
    std::vector<std::vector<float>> k(layers);
    std::vector<Dev<float> *> kd;
    for (uint32_t l = 0; l < layers; ++l) {
        k[l].resize(size_t(T) * W);
        orc_synth_normal_f32(8, 20 + l, k[l].size(), k[l].data());
        kd.push_back(new Dev<float>(k[l]));
    }
    std::mt19937_64 rng(2);
    for (uint32_t l = 0; l < layers; ++l)
        for (uint32_t pos = 0; pos < T;) {
            const uint32_t n = std::min<uint32_t>(T - pos, 1 + uint32_t(rng() % 150));
            cap.capture(l, kd[l]->p + size_t(pos) * W, KVR_FMT_F32, pos, n, W * 4, dim * 4, 4);
            pos += n;
        }
    const uint32_t full = (T + pt - 1) / pt;
    auto sums = cap.finalize(full);
    require(sums.layers.size() == layers && sums.pages == full, "finalized geometry");
    require(kvr_check(ctx, nullptr) == KVR_OK, "check");
    for (uint32_t l = 0; l < layers; ++l) {
        std::vector<float> means(size_t(full) * W);
        std::vector<uint16_t> s16(size_t(full) * W);
        hip(hipMemcpy(means.data(), cap.means(l), means.size() * 4, hipMemcpyDeviceToHost), "D2H");
        hip(hipMemcpy(s16.data(), sums.layers[l], s16.size() * 2, hipMemcpyDeviceToHost), "D2H");
        for (uint32_t p = 0; p < full; ++p) {
            const uint32_t t0 = p * pt, n = std::min(pt, T - t0);
            for (uint32_t c = 0; c < W; ++c) {
                float acc = 0.f;
                for (uint32_t t = 0; t < n; ++t) acc += k[l][size_t(t0 + t) * W + c];
                const float mean = acc * (1.0f / float(n));
                require(std::memcmp(&means[size_t(p) * W + c], &mean, 4) == 0, "captured mean-K differs");
                require(s16[size_t(p) * W + c] == orc_f32_to_f16(mean), "captured fp16 summary differs");
            }
        }
    }
    for (auto *d : kd) delete d;
    }
    kvr_destroy(ctx);
}

// AttentionSamplerHip (llama_kvmem_attention_cuda::score): q8_0 keys, f32
// Q, f16 causal mask on the device and staged from host memory, against the
// oracle's dense FP64 masses; declines what the reference declines.
void attention() {
    const uint32_t dim = 64, heads = 8, kvh = 2, tokens = 700, block = 64, qrows = 12;
    const uint32_t pages = (tokens + block - 1) / block, hb = dim / 32 * 34, krow = kvh * hb;
    std::vector<uint8_t> k(size_t(tokens) * krow);
    orc_synth_q8_0(9, 40, uint64_t(tokens) * kvh * dim / 32, 0.01f, 0.05f, k.data());
    std::vector<float> q(size_t(qrows) * heads * dim);
    orc_synth_normal_f32(9, 41, q.size(), q.data());
    std::vector<uint16_t> mask(size_t(qrows) * tokens);
    for (uint32_t r = 0; r < qrows; ++r)
        for (uint32_t t = 0; t < tokens; ++t)
            mask[size_t(r) * tokens + t] = t <= tokens - qrows + r ? 0 : 0xfc00;  // 0 or -inf
    Dev<uint8_t> kd(k);
    Dev<float> qd(q);
    Dev<uint16_t> md(mask);
    kh::AttentionTensor tq, tk, tm;
    tq.data = qd.p, tq.type = KVR_FMT_F32, tq.ne[0] = dim, tq.ne[1] = qrows, tq.ne[2] = heads;
    tq.nb[1] = size_t(heads) * dim * 4, tq.nb[2] = size_t(dim) * 4;
    tk.data = kd.p, tk.type = KVR_FMT_Q8_0, tk.ne[0] = dim, tk.ne[1] = tokens, tk.ne[2] = kvh;
    tk.nb[1] = krow, tk.nb[2] = hb;
    tm.data = md.p, tm.type = KVR_FMT_F16, tm.ne[0] = tokens, tm.ne[1] = qrows, tm.nb[1] = size_t(tokens) * 2;
    const std::vector<uint32_t> rows = {11, 3, 7};
    const float scale = 0.125f;
    std::vector<double> want(rows.size() * pages);
    require(orc_attention_page_mass(reinterpret_cast<const uint8_t *>(q.data()), ORC_FMT_F32, tq.nb[1], tq.nb[2],
                                    k.data(), ORC_FMT_Q8_0, krow, hb,
                                    reinterpret_cast<const uint8_t *>(mask.data()), ORC_FMT_F16, tm.nb[1], dim,
                                    heads, kvh, tokens, block, scale, 0.0f, rows.data(), uint32_t(rows.size()),
                                    want.data()) == ORC_OK,
            "oracle attention");
    kh::AttentionSamplerHip sampler;
    auto check = [&](const std::vector<std::vector<float>> &got, const char *what) {
        require(got.size() == rows.size(), what);
        for (size_t i = 0; i < rows.size(); ++i)
            for (uint32_t p = 0; p < pages; ++p) {
                const double w = want[i * pages + p], g = got[i][p];
                if (!(std::fabs(g - w) <= 1e-6 + 2e-4 * std::fabs(w)))
                    throw std::runtime_error(std::string(what) + ": mass differs from the oracle");
            }
    };
    std::vector<std::vector<float>> out;
    require(sampler.score(tq, tk, tm, scale, 0.0f, block, rows, out), "device mask declined");
    check(out, "device mask");
    kh::AttentionTensor th = tm;
    th.data = mask.data();  // host memory: the sampled rows are staged
    require(sampler.score(tq, tk, th, scale, 0.0f, block, rows, out), "host mask declined");
    check(out, "staged mask");
    kh::AttentionTensor bad = tq;
    bad.ne[0] = 48;
    require(!sampler.score(bad, tk, tm, scale, 0.0f, block, rows, out), "head dim 48 accepted");
    bad = tq;
    bad.data = q.data();  // Q in host memory
    require(!sampler.score(bad, tk, tm, scale, 0.0f, block, rows, out), "host Q accepted");
    bad = tk;
    bad.type = KVR_FMT_Q4_1;
    require(!sampler.score(tq, bad, tm, scale, 0.0f, block, rows, out), "q4_1 keys accepted");
}

// kvmem_stagein_enqueue_k through the slab: raw q8_0 K records rotated,
// Walsh-Hadamard transformed and requantized on flush, beside a V record;
// bytes equal to the oracle's transform.  Rejections as the reference's.
void stagein_raw_k() {
    require(kh::kvmem_stagein_gpu_ready(0, 0), "gpu_ready");
    const uint32_t nt = 37, n_embd = 256, head = 64, n_rot = 64, nrot = 64, row = n_embd / 32 * 34;
    std::vector<float> theta(n_rot / 2);
    for (uint32_t i = 0; i < n_rot / 2; ++i) theta[i] = std::pow(10000.0f, -2.0f * float(i) / float(n_rot));
    const int32_t pos0[3] = {0, 4096, 777777};
    std::vector<std::vector<uint8_t>> recs(3);
    std::vector<Dev<uint8_t> *> dsts;
    for (int r = 0; r < 3; ++r) {
        recs[r].resize(size_t(nt) * row);
        orc_synth_q8_0(12, 60 + r, uint64_t(nt) * n_embd / 32, 0.01f, 0.05f, recs[r].data());
        dsts.push_back(new Dev<uint8_t>(recs[r].size()));
    }
    std::vector<uint8_t> v(4096, 0x5A);
    Dev<uint8_t> vd(v.size());
    for (int r = 0; r < 3; ++r)
        require(kh::kvmem_stagein_enqueue_k(KVR_FMT_Q8_0, recs[r].data(), recs[r].size(), dsts[r]->p, nt, n_embd,
                                            nrot, n_embd / head, head, n_rot, pos0[r], theta.data(),
                                            int(theta.size()), nullptr, nullptr, nullptr, nullptr),
                "enqueue_k");
    require(kh::kvmem_stagein_enqueue_v(v.data(), v.size(), vd.p, nullptr), "enqueue_v");
    int64_t copy_us = 0, rope_us = 0, had_us = 0, set_us = 0;
    require(kh::kvmem_stagein_flush(&copy_us, &rope_us, &had_us, &set_us), "flush");
    kh::kvmem_stagein_sync();
    require(kh::kvmem_stagein_sync_checked(), "sync_checked");
    for (int r = 0; r < 3; ++r) {
        std::vector<uint8_t> want(recs[r].size());
        require(orc_rope_fwht_rows(recs[r].data(), ORC_FMT_Q8_0, n_embd, nt, pos0[r], head, n_rot, theta.data(),
                                   nrot, want.data()) == ORC_OK,
                "oracle transform");
        require(dsts[r]->down() == want, "raw K record differs from the oracle's transform");
    }
    require(vd.down() == v, "V record");
    std::vector<uint8_t> scratch(size_t(nt) * row);
    require(!kh::kvmem_stagein_enqueue_k(KVR_FMT_Q4_1, scratch.data(), scratch.size(), dsts[0]->p, nt, n_embd, 0,
                                         4, head, 0, 0, nullptr, 0, nullptr, nullptr, nullptr, nullptr),
            "q4_1 K accepted");
    require(!kh::kvmem_stagein_enqueue_k(KVR_FMT_Q8_0, scratch.data(), scratch.size(), dsts[0]->p, nt, n_embd, 32,
                                         4, head, 0, 0, nullptr, 0, nullptr, nullptr, nullptr, nullptr),
            "Walsh-Hadamard 32 accepted");
    require(!kh::kvmem_stagein_enqueue_k(KVR_FMT_Q8_0, scratch.data(), scratch.size(), dsts[0]->p, nt, n_embd, 0,
                                         3, head, 0, 0, nullptr, 0, nullptr, nullptr, nullptr, nullptr),
            "heads not tiling the row accepted");
    for (auto *d : dsts) delete d;
    kh::kvmem_stagein_gpu_free();
}

// Stage-out (kvmem_stageout_*): device records packed into the pinned slot
// by one batched copy, two submits alternating slots; refused beside
// pending stage-in records, as the reference does.
void stageout() {
    require(kh::kvmem_stagein_gpu_ready(0, 0), "gpu_ready");
    std::mt19937_64 rng(9);
    for (int round = 0; round < 2; ++round) {
        std::vector<std::vector<uint8_t>> recs;
        std::vector<Dev<uint8_t> *> devs;
        size_t total = 0;
        for (int i = 0; i < 7; ++i) {
            std::vector<uint8_t> r(1 + rng() % 200000);
            for (auto &b : r) b = uint8_t(rng());
            devs.push_back(new Dev<uint8_t>(r));
            total += r.size();
            recs.push_back(std::move(r));
        }
        for (size_t i = 0; i < recs.size(); ++i)
            require(kh::kvmem_stageout_enqueue(devs[i]->p, recs[i].size()), "stageout enqueue");
        require(kh::kvmem_stageout_used() == total, "stageout used");
        const int slot = kh::kvmem_stageout_submit(nullptr);
        require(slot == round, "slots alternate");
        require(kh::kvmem_stageout_wait(slot, nullptr), "stageout wait");
        const uint8_t *base = kh::kvmem_stageout_slot_base(slot);
        size_t off = 0;
        for (const auto &r : recs) {
            require(std::memcmp(base + off, r.data(), r.size()) == 0, "staged-out bytes differ");
            off += r.size();
        }
        for (auto *d : devs) delete d;
    }
    std::vector<uint8_t> v(64, 1);
    Dev<uint8_t> vd(v.size());
    require(kh::kvmem_stagein_enqueue_v(v.data(), v.size(), vd.p, nullptr), "enqueue_v");
    require(!kh::kvmem_stageout_enqueue(vd.p, 64), "stage-out accepted beside a pending stage-in record");
    require(kh::kvmem_stagein_flush(nullptr, nullptr, nullptr, nullptr), "flush");
    kh::kvmem_stagein_sync();
    require(kh::kvmem_stageout_enqueue(vd.p, 64), "stage-out after the flush");
    require(!kh::kvmem_stagein_enqueue_v(v.data(), v.size(), vd.p, nullptr), "stage-in accepted beside stage-out");
    kh::kvmem_stageout_clear();
    require(kh::kvmem_stageout_used() == 0, "cleared");
    kh::kvmem_stagein_gpu_free();
}

// PayloadLayout::validate (kvmem/src/host/memory_contract.cpp:51-106) and
// record_plane on the layouts it accepts and each rule it enforces.
void payload_layout() {
    using K = kh::PayloadPlaneKind;
    kh::PayloadLayout ok;
    ok.format = "test-q8k-f16v";
    ok.version = 1;
    ok.block_tokens = 64;
    ok.alignment = 256;
    ok.planes = {{0, K::Key, 0, 64 * 272, 16, 272}, {0, K::Value, 17408, 64 * 512, 16, 512},
                 {1, K::Key, 50176, 64 * 272, 16, 272}, {1, K::Value, 67584, 64 * 512, 16, 512}};
    ok.record_bytes = 100352;
    ok.validate();
    uint8_t base[16];
    const kvr_plane p = kh::record_plane(ok, 1, K::Value, base, KVR_FMT_F16, 256, 1000, KVR_GATHER_COPY, nullptr);
    require(p.history == base + 67584 && p.page_stride == 100352 && p.width == 256, "record plane");
    auto rejects = [](const kh::PayloadLayout &l) {
        try {
            l.validate();
        } catch (const kh::MemoryError &e) {
            return e.code() == kh::MemoryErrorCode::InvalidPlan;
        }
        return false;
    };
    auto bad = ok;
    bad.format.clear();
    require(rejects(bad), "empty format accepted");
    bad = ok;
    bad.record_bytes = 100000;  // not a multiple of the alignment
    require(rejects(bad), "unaligned record accepted");
    bad = ok;
    bad.planes[1].offset = 17000;  // overlaps the key plane
    require(rejects(bad), "overlapping planes accepted");
    bad = ok;
    bad.planes[1].offset = 17416;  // not 16-aligned
    require(rejects(bad), "misaligned plane accepted");
    bad = ok;
    bad.planes[3].kind = K::Key;  // layer 1 without a value plane, key twice
    require(rejects(bad), "duplicate kind accepted");
    bad = ok;
    bad.planes[3].kind = K::ValueScale;  // layer 1 lacks its value plane
    require(rejects(bad), "layer without value plane accepted");
    bad = ok;
    bad.planes[0].token_stride = 273;  // 64 rows of 273 B exceed the plane
    require(rejects(bad), "token rows beyond the plane accepted");
    bad = ok;
    bad.planes[3].bytes = 40000;  // runs past the record
    require(rejects(bad), "plane past its record accepted");
    bad = ok;
    bad.planes[0].head_count = 4;  // a head range on one plane of the shard only
    require(rejects(bad), "inconsistent head ranges accepted");
    bool threw = false;
    try {
        kh::record_plane(ok, 0, K::Key, base, KVR_FMT_F16, 256, 1000, KVR_GATHER_COPY, nullptr);  // 272 B rows
    } catch (const std::invalid_argument &) {
        threw = true;
    }
    require(threw, "record plane with a mismatched row size accepted");
}

// ---- the reference's own validators, from oracle/_ref (when built) ---------
struct RefBuild {
    void *so = nullptr;
    const char *(*last_error)() = nullptr;
    int (*payload_validate)(const char *, uint32_t, uint32_t, uint64_t, uint64_t, const uint64_t *,
                            uint32_t) = nullptr;
    int (*native_query_validate)(uintptr_t, size_t, uint32_t, uint32_t, uint32_t, uint32_t, float, int, size_t,
                                 size_t, size_t) = nullptr;
    int (*lrfu_script)(double, double, const int *, const uint32_t *, uint32_t, const double *, uint32_t, int *,
                       double *) = nullptr;
};
std::string g_exe_dir = ".";
const RefBuild *reference_build() {
    static RefBuild rb;
    static bool tried = false;
    if (!tried) {
        tried = true;
        const std::string path = g_exe_dir + "/../../../oracle/_ref/libkvmem_ref.so";
        rb.so = dlopen(path.c_str(), RTLD_NOW | RTLD_LOCAL);
        if (rb.so) {
            rb.last_error = reinterpret_cast<decltype(rb.last_error)>(dlsym(rb.so, "ref_last_error"));
            rb.payload_validate = reinterpret_cast<decltype(rb.payload_validate)>(dlsym(rb.so, "ref_payload_validate"));
            rb.native_query_validate =
                reinterpret_cast<decltype(rb.native_query_validate)>(dlsym(rb.so, "ref_native_query_validate"));
            rb.lrfu_script = reinterpret_cast<decltype(rb.lrfu_script)>(dlsym(rb.so, "ref_lrfu_script"));
        }
    }
    return rb.so && rb.payload_validate && rb.native_query_validate && rb.lrfu_script ? &rb : nullptr;
}

// PayloadLayout::validate against the reference's on random layouts: valid
// ones (layers of one or two rank shards with explicit or "all" head ranges,
// key/value/scale or packed planes, aligned back to back), each then mutated
// in up to three fields.  Both must accept, or both reject with one message.
void payload_layout_vs_reference() {
    const RefBuild *ref = reference_build();
    if (!ref) {
        std::cout << "  reference build absent: nothing to compare" << std::endl;
        return;
    }
    using K = kh::PayloadPlaneKind;
    std::mt19937_64 rng(77);
    auto pick = [&](uint64_t n) { return n ? rng() % n : 0; };
    int accepted = 0, rejected = 0;
    std::map<std::string, int> by_message;
    for (int trial = 0; trial < 20000; ++trial) {
        kh::PayloadLayout l;
        l.format = pick(60) ? "fmt" : "";
        l.version = pick(60) ? 1 + uint32_t(pick(7)) : 0;
        l.block_tokens = uint32_t(1 + pick(128)) * (pick(60) ? 1 : 0);
        l.alignment = uint64_t(1) << pick(9);
        const uint32_t layers = 1 + uint32_t(pick(3));
        uint64_t off = 0;
        for (uint32_t layer = 0; layer < layers; ++layer) {
            const uint32_t ranks = 1 + uint32_t(pick(2));
            const bool sharded = ranks > 1 || pick(2);
            uint32_t head = 0;
            for (uint32_t rank = 0; rank < ranks; ++rank) {
                const uint32_t hc = sharded && pick(12) ? 1 + uint32_t(pick(4)) : 0;
                std::vector<K> kinds;
                if (pick(5) == 0)
                    kinds = {K::PackedKeyValue};
                else {
                    kinds = {K::Key, K::Value};
                    if (pick(2)) kinds.push_back(K::KeyScale);
                    if (pick(2)) kinds.push_back(K::ValueScale);
                }
                for (K k : kinds) {
                    kh::PayloadPlane p;
                    p.layer = layer * 3;
                    p.kind = k;
                    p.alignment = uint64_t(1) << pick(5);
                    p.token_stride = k == K::PackedKeyValue ? 0 : 16 * (1 + pick(8));
                    p.bytes = p.token_stride ? p.token_stride * std::max<uint32_t>(1, l.block_tokens) : 64 + pick(999);
                    p.offset = (off + p.alignment - 1) / p.alignment * p.alignment;
                    p.rank = rank;
                    p.head_begin = sharded ? head : 0;
                    p.head_count = hc;
                    off = p.offset + p.bytes;
                    l.planes.push_back(p);
                }
                head += hc;
            }
        }
        l.record_bytes = (off + l.alignment - 1) / l.alignment * l.alignment + l.alignment * pick(2);
        const int mutations = int(pick(4));
        for (int m = 0; m < mutations && !l.planes.empty(); ++m) {
            kh::PayloadPlane &p = l.planes[pick(l.planes.size())];
            switch (pick(12)) {
            case 0: p.offset += pick(3) ? pick(64) : 0 - pick(64); break;
            case 1: p.bytes = pick(3) ? p.bytes + pick(300) : 0; break;
            case 2: p.alignment = pick(4) ? uint64_t(1) << pick(12) : 3 + pick(5); break;
            case 3: p.kind = K(pick(20) ? pick(5) : 5 + pick(3)); break;
            case 4: p.head_begin = uint32_t(pick(6)); break;
            case 5: p.head_count = pick(5) ? uint32_t(pick(6)) : 0xffffffffu; break;
            case 6: p.token_stride = pick(3) ? p.token_stride + pick(40) : pick(2) ? 0 : ~uint64_t(0) / 3; break;
            case 7: p.rank = uint32_t(pick(3)); break;
            case 8: p.layer = uint32_t(pick(3) * 3); break;
            case 9: l.record_bytes = pick(2) ? l.record_bytes - pick(512) : l.record_bytes + pick(512); break;
            case 10: l.planes.erase(l.planes.begin() + long(pick(l.planes.size()))); break;
            default: p.offset = pick(2) ? ~uint64_t(0) - pick(100) : p.offset; p.bytes += pick(2) ? ~uint64_t(0) / 2 : 0;
            }
        }
        std::string mine;
        try {
            l.validate();
        } catch (const kh::MemoryError &e) {
            require(e.code() == kh::MemoryErrorCode::InvalidPlan, "payload error code");
            mine = e.what();
        }
        std::vector<uint64_t> rows;
        for (const auto &p : l.planes)
            for (uint64_t v : {uint64_t(p.layer), uint64_t(p.kind), p.offset, p.bytes, p.alignment, p.token_stride,
                               uint64_t(p.rank), uint64_t(p.head_begin), uint64_t(p.head_count)})
                rows.push_back(v);
        const int rc = ref->payload_validate(l.format.c_str(), l.version, l.block_tokens, l.record_bytes,
                                             l.alignment, rows.data(), uint32_t(l.planes.size()));
        const std::string theirs = rc ? ref->last_error() : "";
        if (mine != theirs)
            throw std::runtime_error("payload layout trial " + std::to_string(trial) + ": mine '" + mine +
                                     "', reference '" + theirs + "'");
        (mine.empty() ? accepted : rejected)++;
        if (!mine.empty()) ++by_message[mine];
    }
    require(accepted > 1000 && rejected > 1000, "payload fuzz reached both outcomes");
    require(by_message.size() == 12, "payload fuzz reached every rule");
    std::cout << "  " << accepted << " accepted, " << rejected << " rejected, all as the reference" << std::endl;
    for (const auto &m : by_message) std::cout << "    " << m.second << " x " << m.first << std::endl;
}

// validate_native_layer_query against the reference's on random geometries:
// the six axis orders, padded strides, counts of 1, equal strides,
// overlapping and huge strides, extents around the exact span.
void native_query_vs_reference() {
    const RefBuild *ref = reference_build();
    if (!ref) {
        std::cout << "  reference build absent: nothing to compare" << std::endl;
        return;
    }
    std::mt19937_64 rng(78);
    auto pick = [&](uint64_t n) { return n ? rng() % n : 0; };
    int accepted = 0, rejected = 0;
    for (int trial = 0; trial < 50000; ++trial) {
        kh::NativeCurrentLayerQuery q;
        const int scalar = int(pick(3));
        const size_t el = scalar == 0 ? 4 : 2;
        q.scalar = kh::NativeQueryScalar(scalar);
        q.data = reinterpret_cast<const void *>(uintptr_t(4096) + (pick(8) ? 0 : pick(4)));
        q.rows = uint32_t(pick(6));
        q.kv_heads = 1 + uint32_t(pick(4)) * (pick(20) ? 1 : 0);
        q.query_heads = q.kv_heads * uint32_t(pick(4)) + (pick(10) ? 0 : 1);
        q.head_dim = uint32_t(1 + pick(8)) * (pick(20) ? 1 : 0);
        q.attention_scale = pick(15) ? float(pick(100)) / 64 : (pick(2) ? -1.f : NAN);
        uint32_t count[3] = {q.rows, q.query_heads, q.head_dim};
        int order[3] = {0, 1, 2};
        std::shuffle(order, order + 3, rng);
        size_t stride[3], span = el;
        for (int i = 0; i < 3; ++i) {
            const int a = order[i];
            stride[a] = span + el * pick(3) * (pick(3) == 0);
            if (pick(8) == 0) stride[a] = pick(2) ? span - el : el * pick(3);
            if (pick(40) == 0) stride[a] = ~size_t(0) / 2 + pick(3);
            if (pick(40) == 0) stride[a] += 1;
            span += stride[a] * (count[a] ? count[a] - 1 : 0);
        }
        q.row_stride = stride[0];
        q.head_stride = stride[1];
        q.dimension_stride = stride[2];
        q.bytes = pick(4) ? span : span + el * (pick(2) ? 1 : -1);
        std::string mine;
        try {
            kh::validate_native_layer_query(q);
        } catch (const std::invalid_argument &e) {
            mine = e.what();
        }
        const int rc = ref->native_query_validate(uintptr_t(q.data), q.bytes, q.rows, q.query_heads, q.kv_heads,
                                                  q.head_dim, q.attention_scale, scalar, q.row_stride,
                                                  q.head_stride, q.dimension_stride);
        const std::string theirs = rc ? ref->last_error() : "";
        if (mine != theirs)
            throw std::runtime_error("native query trial " + std::to_string(trial) + ": mine '" + mine +
                                     "', reference '" + theirs + "'");
        (mine.empty() ? accepted : rejected)++;
    }
    require(accepted > 5000 && rejected > 5000, "native query fuzz reached both outcomes");
    std::cout << "  " << accepted << " accepted, " << rejected << " rejected, all as the reference" << std::endl;
}

// span_coefficients (sorted sweep) against the oracle's pair-by-pair
// restatement of span_coefficient, on random spans (some open-ended).
void graph_spans() {
    std::mt19937_64 rng(21);
    for (int round = 0; round < 50; ++round) {
        const uint32_t bt = 1 + uint32_t(rng() % 64), pages = 1 + uint32_t(rng() % 300);
        std::vector<kh::GraphMessageSpan> spans(rng() % 20);
        std::vector<uint64_t> b, e;
        std::vector<uint8_t> k;
        for (auto &sp : spans) {
            sp.begin = rng() % (uint64_t(pages) * bt + 1);
            sp.end = sp.begin + rng() % (uint64_t(bt) * 8 + 1);
            sp.end_known = rng() % 4 != 0;
            b.push_back(sp.begin);
            e.push_back(sp.end);
            k.push_back(sp.end_known);
        }
        const auto got = kh::span_coefficients(spans, bt, pages, .25);
        std::vector<double> want(pages, 1.0);
        require(orc_span_coefficients(b.data(), e.data(), k.data(), uint32_t(spans.size()), bt, pages, .25,
                                      want.data()) == ORC_OK,
                "oracle spans");
        want.resize(pages - 1);
        require(got == want, "span coefficients differ from the pair-by-pair restatement");
    }
}

// GraphRecallHip / LrfuHistoryHip on the reference's known answers
// (kvmem/tests/graph_recall_test.cpp:107-126, 312-322;
// kvmem_store_test.cpp:1195-1202).
void graph() {
    kh::GraphRecallHip dev(0);
    std::vector<kh::GraphRow> rows = {{64, 1, {{0, .8}}}, {128, 1, {{64, 1.0}}}};
    kh::GraphView g;
    g.block_tokens = 64;
    g.accepted_through = g.completed_through = 192;
    g.chunks = {&rows};
    auto frame = kh::query_score_frame(192, 64, 2, 0, 0, {});
    auto near = [](const std::vector<double> &a, const std::vector<double> &b) {
        if (a.size() != b.size()) return false;
        for (size_t i = 0; i < a.size(); ++i)
            if (std::abs(a[i] - b[i]) > 1e-12) return false;
        return true;
    };
    require(near(dev.propagate_query_scores({1, 0, 1}, frame, g), {.95, .2, .85}), "lifecycle");
    frame.transport_mask[0] = 0;
    require(near(dev.propagate_query_scores({8, 0, 1}, frame, g), {8, .15, .85}), "fixed page");
    // a row whose source block is not complete is not read
    g.completed_through = 128;
    frame.transport_mask[0] = 1;
    require(near(dev.propagate_query_scores({1, 0, 1}, frame, g), {.95, .1, .95}), "incomplete source read");
    std::vector<kh::GraphRow> none;
    std::vector<kh::GraphMessageSpan> spans = {{0, 64, true}, {64, 192, true}};
    kh::GraphView m;
    m.block_tokens = 64;
    m.accepted_through = m.completed_through = 192;
    m.chunks = {&none};
    m.messages = &spans;
    const auto crossed = dev.propagate_query_scores({1, 0, 0}, frame, m);
    require(std::abs(crossed[0] - .9875) < 1e-12 && std::abs(crossed[1] - .0125) < 1e-12, "message locality");
    bool threw = false;
    try {
        dev.propagate_query_scores({0, std::nan(""), 0}, frame, m);
    } catch (const std::invalid_argument &) {
        threw = true;
    }
    require(threw, "nonfinite seed accepted");
    threw = false;
    m.accepted_through = 128;
    try {
        dev.propagate_query_scores({1, 0, 0}, frame, m);
    } catch (const std::invalid_argument &) {
        threw = true;
    }
    require(threw, "mismatched accepted prefix accepted");

    kh::LrfuHistoryHip h(dev, .5, .5);
    h.begin_round();
    h.preview({.1, .2, .6, .8});
    require(h.score(0) == 0 && h.score(1) == 0 && h.score(2) == .6 && h.score(3) == .8, "LRFU first round");
    require(h.commit(), "commit");
    const auto checkpoint = h.checkpoint();
    h.begin_round();
    h.preview({-.8, -.2, .4, .8});
    h.preview({-.8, -.2, .4, .8});
    require(std::abs(h.score(0) + .8) < 1e-12 && std::abs(h.score(1) + .2) < 1e-12 &&
                std::abs(h.score(2) - .7) < 1e-12 && std::abs(h.score(3) - 1.2) < 1e-12,
            "LRFU second round");
    require(h.commit() && !h.commit(), "one commit per round");
    h.restore(checkpoint);
    require(h.score(0) == 0 && h.score(2) == .6, "LRFU restore");
}

// LrfuHistoryHip against the reference's LrfuHistory on random scripts of
// rounds, previews (repeated, empty, of varying length), commits,
// checkpoints and restores: the same outcome of every step (success, throw,
// refused commit) and the same scores bit for bit after it.
void lrfu_vs_reference() {
    const RefBuild *ref = reference_build();
    require(ref != nullptr, "the reference build (oracle/_ref) is needed for this test");
    kh::GraphRecallHip dev(0);
    std::mt19937_64 rng(79);
    std::uniform_real_distribution<double> val(-1, 1);
    const uint32_t probe = 12;
    for (int script = 0; script < 60; ++script) {
        const double lambda = std::vector<double>{0, .25, .5, 1}[rng() % 4];
        const double fraction = std::vector<double>{.1, .5, .9, 1}[rng() % 4];
        const uint32_t n_ops = 6 + uint32_t(rng() % 20);
        std::vector<int> ops(n_ops);
        std::vector<uint32_t> lens(n_ops, 0);
        std::vector<double> values;
        for (uint32_t i = 0; i < n_ops; ++i) {
            const int r = int(rng() % 10);
            ops[i] = r < 2 ? 0 : r < 6 ? 1 : r < 8 ? 2 : r < 9 ? 3 : 4;
            if (ops[i] == 1) {
                lens[i] = rng() % 8 == 0 ? 0 : 1 + uint32_t(rng() % probe);
                for (uint32_t j = 0; j < lens[i]; ++j) values.push_back(rng() % 5 == 0 ? 0.0 : val(rng));
            }
        }
        std::vector<int> want_r(n_ops);
        std::vector<double> want_s(size_t(n_ops) * probe);
        require(ref->lrfu_script(lambda, fraction, ops.data(), lens.data(), n_ops, values.data(), probe,
                                 want_r.data(), want_s.data()) == 0,
                "reference LRFU script");
        kh::LrfuHistoryHip h(dev, lambda, fraction);
        kh::LrfuState kept;
        size_t cursor = 0;
        for (uint32_t i = 0; i < n_ops; ++i) {
            int r = 0;
            try {
                switch (ops[i]) {
                case 0: h.begin_round(); break;
                case 1: h.preview(std::vector<double>(values.begin() + long(cursor),
                                                      values.begin() + long(cursor + lens[i])));
                    break;
                case 2: r = h.commit() ? 0 : 2; break;
                case 3: kept = h.checkpoint(); break;
                default: h.restore(kept); break;
                }
            } catch (const std::exception &) {
                r = 1;
            }
            if (ops[i] == 1) cursor += lens[i];
            const std::string at = "LRFU script " + std::to_string(script) + " step " + std::to_string(i);
            require(r == want_r[i], at + ": outcome differs from the reference");
            for (uint32_t b = 0; b < probe; ++b) {
                const double got = h.score(b), want = want_s[size_t(i) * probe + b];
                require(std::memcmp(&got, &want, 8) == 0, at + ": score differs from the reference");
            }
        }
    }
}

}  // namespace

int main(int argc, char **argv) {
    const bool gpu = argc > 1 && std::string(argv[1]) == "--gpu";
    {
        const std::string self = argv[0];
        const size_t slash = self.rfind('/');
        if (slash != std::string::npos) g_exe_dir = self.substr(0, slash);
    }
    std::vector<std::pair<const char *, std::function<void()>>> tests = {
        {"frames", frames}, {"native_query_geometry", native_query_geometry},
        {"workspace_geometry", workspace_geometry}, {"stagein_without_state", stagein_without_state},
        {"graph_spans", graph_spans}, {"payload_layout", payload_layout},
        {"payload_layout_vs_reference", payload_layout_vs_reference},
        {"native_query_vs_reference", native_query_vs_reference}};
    if (gpu)
        tests = {{"qualification", qualification}, {"current_layer", current_layer}, {"pick", pick},
                 {"stagein", stagein},           {"meank", meank},                 {"transfer", transfer},
                 {"capture", capture}, {"attention", attention}, {"stagein_raw_k", stagein_raw_k},
                 {"stageout", stageout}, {"graph", graph}, {"lrfu_vs_reference", lrfu_vs_reference}};
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
