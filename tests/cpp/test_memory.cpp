// Tests of the llama.cpp hooks, the memory-factory hook and RecallMemory's
// memory-backend side (include/kvmem_hip/llama_kvmem_hooks.h,
// kvmem_memory.hpp).  This program plays the engine: its own ggml_tensor,
// llama_model and llama_memory_i types and an EngineBridge over them (the
// library only sees them as opaque pointers).  The oracle is the checker.
//   test_memory --cpu   decline rules, memory plans, execution states
//   test_memory --gpu   prefill capture through the hooks, scores and
//                       selection against the oracle, restore through
//                       prepare / MemoryTransfer, decode mean-K after the
//                       pin, attention samples, plan errors
#include "kvmem_hip/llama_kvmem_hooks.h"
#include "kvr_oracle.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <functional>
#include <iostream>
#include <memory>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

namespace kh = kvmem_hip;

// ---- the test engine's types ----------------------------------------------------
struct ggml_tensor {
    kh::TensorView view;
};
struct ggml_backend_sched {
    int synchronized = 0;
};
struct llama_model {
    kh::ModelFacts facts;
};
struct llama_memory_params {};
struct llama_cparams {
    uint32_t n_ctx = 0, n_seq_max = 1;
};
struct llama_memory_i {
    std::unique_ptr<kh::RecallMemory> memory;
    ~llama_memory_i() { kh::unbind_memory(memory.get()); }
};

namespace {

void require(bool ok, const std::string &msg) {
    if (!ok) throw std::runtime_error(msg);
}
void hip(hipError_t e, const char *what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}
template <class F> kh::MemoryErrorCode plan_error(F f) {
    try {
        f();
    } catch (const kh::MemoryError &e) {
        return e.code();
    }
    throw std::runtime_error("plan accepted");
}

void install_bridge() {
    kh::EngineBridge b;
    b.describe = [](const llama_model &m, const llama_memory_params &, const llama_cparams &c, kh::ModelFacts &f) {
        f = m.facts;
        f.n_ctx_seq = c.n_ctx;
        f.n_seq_max = c.n_seq_max;
        return true;
    };
    b.wrap = [](std::unique_ptr<kh::RecallMemory> mem, const kh::ModelFacts &) {
        auto *w = new llama_memory_i;
        w->memory = std::move(mem);
        return w;
    };
    b.tensor_view = [](const ggml_tensor *t, kh::TensorView &v) {
        v = t->view;
        return true;
    };
    b.synchronize = [](ggml_backend_sched *s) {
        hip(hipDeviceSynchronize(), "hipDeviceSynchronize");
        ++s->synchronized;
    };
    kh::set_engine_bridge(b);
}

llama_kvmem_params enabled_params() {
    llama_kvmem_params p{};
    p.enabled = true;
    p.method = 1;
    p.block_tokens = 64;
    p.budget = 640;
    p.sink_tokens = 64;
    p.recent_tokens = 100;
    p.query_begin = 1500;
    p.query_end = 1530;
    p.query_end = 1530;
    return p;
}

llama_model test_model() {
    llama_model m;
    m.facts.n_layer = 3;
    m.facts.attention_layers = {0, 2};  // layer 1 has no KV (a hybrid model's recurrent layer)
    m.facts.query_heads = 8;
    m.facts.kv_heads = 2;
    m.facts.head_dim = 64;
    m.facts.model = "test-3l";
    return m;
}

// ---- CPU ----------------------------------------------------------------------------
void declines_and_plans() {
    install_bridge();
    llama_model model = test_model();
    llama_memory_params mp;
    llama_cparams cp;
    cp.n_ctx = 2048;
    llama_kvmem_set_params(nullptr);
    require(!llama_kvmem_get_params()->enabled, "defaults are disabled");
    require(!llama_memory_kvmem_maybe_create(model, mp, cp), "disabled memory created");
    llama_kvmem_params p = enabled_params();
    llama_kvmem_set_params(&p);
    cp.n_seq_max = 2;
    require(!llama_memory_kvmem_maybe_create(model, mp, cp), "n_seq_max 2 accepted");
    cp.n_seq_max = 1;
    for (int rule = 0; rule < 4; ++rule) {
        llama_model m = model;
        if (rule == 0) m.facts.recurrent = true;
        if (rule == 1) m.facts.sliding_window = true;
        if (rule == 2) m.facts.mtp_context = true;
        if (rule == 3) m.facts.companion = true;
        require(!llama_memory_kvmem_maybe_create(m, mp, cp), "declined model accepted, rule " + std::to_string(rule));
    }
    // the plan: pages of 64 over 2048 tokens, budget 640 -> 10 pages, one
    // sink page, 100 recent tokens -> 2 pages, 30 Query rows
    const auto c = kh::plan_recall_memory(p, [&] {
        kh::ModelFacts f = model.facts;
        f.n_ctx_seq = 2048;
        return f;
    }());
    require(c.block_tokens == 64 && c.max_pages == 32 && c.budget_pages == 10 && c.sink_pages == 1 &&
                c.recent_pages == 2 && c.max_query_rows == 30 && c.layers == std::vector<uint32_t>({0, 2}) &&
                c.tie == kh::TieRule::HigherFirst && c.retrieval,
            "memory plan");
    llama_kvmem_params d{};
    d.enabled = true;
    d.method = 1;
    d.query_begin = -1;
    const auto c2 = kh::plan_recall_memory(d, [&] {
        kh::ModelFacts f = model.facts;
        f.n_ctx_seq = 1000;
        return f;
    }());
    require(c2.block_tokens == 32 && c2.max_pages == 32 && c2.budget_pages == 0 && c2.sink_pages == 1 &&
                c2.recent_pages == 0,
            "default memory plan");
    // execution states keep their own parameters
    llama_kvmem_execution_state *s = llama_kvmem_execution_create();
    llama_kvmem_execution_state *prev = llama_kvmem_execution_exchange(s);
    require(!llama_kvmem_get_params()->enabled, "a new execution state starts disabled");
    require(!llama_kvmem_ubatch_needs_q_capture(4, 1, nullptr), "disabled state wants Query");
    llama_kvmem_execution_exchange(prev);
    llama_kvmem_execution_free(s);
    require(llama_kvmem_get_params()->enabled && llama_kvmem_get_params()->budget == 640, "parameters kept");
    const llama_pos in[2] = {1499, 1500}, out[2] = {1, 2};
    require(llama_kvmem_ubatch_needs_q_capture(2, 1, in) && !llama_kvmem_ubatch_needs_q_capture(2, 1, out),
            "Query span from the parameters");
    require(!llama_kvmem_eval_callback(nullptr, true, nullptr) && llama_kvmem_capture_stamp() == 0,
            "unbound hooks");
    llama_kvmem_set_params(nullptr);
}

// ---- GPU ------------------------------------------------------------------------------
template <class T> struct Dev {
    T *p = nullptr;
    size_t n = 0;
    explicit Dev(size_t count) : n(count) { hip(hipMalloc(&p, std::max<size_t>(n, 1) * sizeof(T)), "hipMalloc"); }
    explicit Dev(const std::vector<T> &h) : Dev(h.size()) {
        hip(hipMemcpy(p, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice), "H2D");
    }
    ~Dev() { (void)hipFree(p); }
    std::vector<T> down() const {
        std::vector<T> h(n);
        hip(hipMemcpy(h.data(), p, n * sizeof(T), hipMemcpyDeviceToHost), "D2H");
        return h;
    }
};

struct Host {
    void *p = nullptr;
    explicit Host(size_t bytes) { require(kvr_host_alloc(bytes, &p) == KVR_OK, "kvr_host_alloc"); }
    ~Host() { (void)kvr_host_free(p); }
};

void end_to_end() {
    install_bridge();
    const uint32_t L = 3, HQ = 8, HKV = 2, D = 64, W = HKV * D, BT = 64, TOK = 1600, UB = 512;
    const std::vector<uint32_t> attn = {0, 2};
    llama_model model = test_model();
    llama_memory_params mp;
    llama_cparams cp;
    cp.n_ctx = 2048;
    llama_kvmem_params p = enabled_params();
    llama_kvmem_set_params(&p);
    std::unique_ptr<llama_memory_i> wrapper(llama_memory_kvmem_maybe_create(model, mp, cp));
    require(wrapper && kh::current_memory() == wrapper->memory.get(), "memory created and bound");
    kh::RecallMemory &mem = *wrapper->memory;
    require(mem.owns_layer(0) && !mem.owns_layer(1) && mem.owns_layer(2), "served layers");

    // key history and Query rows (host copies for the oracle)
    std::mt19937_64 rng(5);
    std::normal_distribution<float> nd(0.f, 1.f);
    std::vector<std::vector<uint16_t>> keys(L, std::vector<uint16_t>(size_t(TOK + 1) * W));
    std::vector<std::vector<float>> qall(L, std::vector<float>(size_t(TOK) * HQ * D));
    for (uint32_t l = 0; l < L; ++l) {
        for (auto &k : keys[l]) k = orc_f32_to_f16(nd(rng));
        for (auto &q : qall[l]) q = nd(rng);
    }
    ggml_backend_sched sched;
    for (uint32_t pos0 = 0; pos0 < TOK; pos0 += UB) {
        const uint32_t n = std::min(UB, TOK - pos0);
        std::vector<llama_pos> pos(n);
        for (uint32_t i = 0; i < n; ++i) pos[i] = llama_pos(pos0 + i);
        const bool need_q = llama_kvmem_ubatch_needs_q_capture(n, 1, pos.data());
        require(need_q == (pos0 <= 1529 && pos0 + n > 1500), "Query overlap of a ubatch");
        // the engine's tensors of this ubatch: K f16 [n][HKV][D]; Q f32
        // [n][HQ][D], layer 2's heads padded by 16 floats
        std::vector<std::unique_ptr<Dev<uint16_t>>> kdev;
        std::vector<std::unique_ptr<Dev<float>>> qdev;
        std::vector<ggml_tensor> kt(L), qt(L);
        llama_kvmem_capture_on_new_graph(0);
        for (uint32_t l = 0; l < L; ++l) {
            std::vector<uint16_t> kk(keys[l].begin() + size_t(pos0) * W, keys[l].begin() + size_t(pos0 + n) * W);
            kdev.push_back(std::make_unique<Dev<uint16_t>>(kk));
            kt[l].view.data = kdev.back()->p;
            kt[l].view.type = KVR_FMT_F16;
            kt[l].view.ne[0] = D, kt[l].view.ne[1] = HKV, kt[l].view.ne[2] = n, kt[l].view.ne[3] = 1;
            kt[l].view.nb[0] = 2, kt[l].view.nb[1] = D * 2, kt[l].view.nb[2] = size_t(W) * 2;
            const uint32_t hs = l == 2 ? D + 16 : D;  // head stride in floats
            std::vector<float> qq(size_t(n) * HQ * hs, 0.f);
            for (uint32_t t = 0; t < n; ++t)
                for (uint32_t h = 0; h < HQ; ++h)
                    std::memcpy(&qq[(size_t(t) * HQ + h) * hs], &qall[l][((size_t(pos0) + t) * HQ + h) * D], D * 4);
            qdev.push_back(std::make_unique<Dev<float>>(qq));
            qt[l].view.data = qdev.back()->p;
            qt[l].view.type = KVR_FMT_F32;
            qt[l].view.ne[0] = D, qt[l].view.ne[1] = HQ, qt[l].view.ne[2] = n, qt[l].view.ne[3] = 1;
            qt[l].view.nb[0] = 4, qt[l].view.nb[1] = size_t(hs) * 4, qt[l].view.nb[2] = size_t(HQ) * hs * 4;
            llama_kvmem_register_capture(&kt[l], int(l), 'k');
            if (need_q) llama_kvmem_register_capture(&qt[l], int(l), 'q');
            llama_kvmem_register_capture(&kt[l], int(l), 'v');
        }
        require(llama_kvmem_capture_can_reuse(n, 1, pos.data(), 0), "graph built for this ubatch is reusable");
        mem.note_ubatch(pos);
        const int synced = sched.synchronized;
        llama_kvmem_harvest_ubatch(&sched, 0);
        require(sched.synchronized == synced + 1, "harvest synchronizes the scheduler");
    }
    require(mem.frontier() == TOK && mem.pages() == 25, "frontier after prefill");
    require(mem.query_rows(0) == 30 && mem.query_rows(2) == 30 && mem.query_rows(1) == 0, "Query rows kept");

    // scores and selection against the oracle
    const uint32_t P = mem.pages();
    std::vector<float> means(size_t(attn.size()) * P * W), sums(size_t(P) * W);
    std::vector<float> q(size_t(attn.size()) * 30 * HQ * D);
    for (size_t i = 0; i < attn.size(); ++i) {
        require(orc_page_summaries(keys[attn[i]].data(), ORC_FMT_F16, TOK, W, BT, sums.data(),
                                   means.data() + i * P * W) == ORC_OK,
                "oracle summaries");
        std::memcpy(q.data() + i * 30 * HQ * D, &qall[attn[i]][size_t(1500) * HQ * D], size_t(30) * HQ * D * 4);
    }
    std::vector<uint64_t> st(P);
    std::vector<uint32_t> ct(P);
    std::vector<uint8_t> sm(P), tm(P);
    require(orc_query_score_frame(TOK, BT, 10, 1, 2, nullptr, 0, st.data(), ct.data(), sm.data(), tm.data()) == ORC_OK,
            "oracle frame");
    const uint32_t rows[2] = {30, 30};
    std::vector<double> want(P);
    require(orc_page_softmax_scores(means.data(), q.data(), rows, 2, 30, HQ, HKV, D, P, sm.data(), 0.f, ORC_AGG_MEAN,
                                    want.data()) == ORC_OK,
            "oracle scores");
    const auto got = mem.score();
    for (uint32_t i = 0; i < P; ++i)
        require(std::fabs(got[i] - want[i]) <= 1e-9 * std::max(1.0, std::fabs(want[i])),
                "score differs from the oracle at page " + std::to_string(i));
    std::vector<uint32_t> fixed(P), picked(P);
    uint32_t nf = 0, np = 0;
    require(orc_query_fixed_blocks(P, 10, 1, 2, nullptr, 0, TOK, BT, nullptr, 0, fixed.data(), &nf) == ORC_OK,
            "oracle fixed pages");
    require(orc_pick_scored_blocks(want.data(), P, fixed.data(), nf, 10, ORC_TIE_HIGHER_FIRST, 0, picked.data(), &np) ==
                ORC_OK,
            "oracle pick");
    picked.resize(np);
    const auto sel = mem.select();
    require(sel == picked, "selection differs from the oracle");

    // restore through the memory-backend contract
    std::vector<std::unique_ptr<Host>> hist;
    std::vector<std::unique_ptr<Dev<uint8_t>>> slots;
    std::vector<std::vector<uint8_t>> vals;
    for (uint32_t l : attn) {
        auto kh_ = std::make_unique<Host>(size_t(TOK) * W * 2);
        std::memcpy(kh_->p, keys[l].data(), size_t(TOK) * W * 2);
        auto vh = std::make_unique<Host>(size_t(TOK) * W * 2);
        std::vector<uint8_t> v(size_t(TOK) * W * 2);
        for (auto &b : v) b = uint8_t(rng());
        std::memcpy(vh->p, v.data(), v.size());
        vals.push_back(v);
        slots.push_back(std::make_unique<Dev<uint8_t>>(size_t(10) * BT * W * 2));
        slots.push_back(std::make_unique<Dev<uint8_t>>(size_t(10) * BT * W * 2));
        kvr_plane kp{}, vp{};
        kp.history = kh_->p, kp.format = KVR_FMT_F16, kp.width = W, kp.tokens = TOK, kp.mode = KVR_GATHER_COPY;
        kp.slots = slots[slots.size() - 2]->p;
        vp = kp;
        vp.history = vh->p;
        vp.slots = slots.back()->p;
        mem.set_history(l, kp, vp);
        hist.push_back(std::move(kh_));
        hist.push_back(std::move(vh));
    }
    const kh::MemoryDescriptor desc = mem.descriptor();
    desc.layout.validate();
    require(desc.layout.planes.size() == 4 && desc.capabilities.page_tokens == BT && desc.capabilities.sparse_view,
            "descriptor");
    const kh::MemorySnapshot snap = mem.snapshot();
    require(snap.blocks.size() == P && snap.resident.empty() && snap.stamp == mem.stamp() && snap.stamp.valid,
            "snapshot");
    kh::WorkingSetPlan plan;
    plan.expected = snap.stamp;
    for (size_t i = 0; i < sel.size(); ++i) {
        kh::ViewBlock vb;
        vb.block = snap.blocks[sel[i]].block;
        vb.compact_start = uint64_t(i) * BT;
        plan.next.blocks.push_back(vb);
        plan.restore.push_back(vb.block);
    }
    {
        auto t = mem.prepare(plan);
        t->start_spill();
        kh::TransferPoll pl;
        while ((pl = t->poll()).status == kh::TransferStatus::Pending) {
        }
        t->start_restore();
        while ((pl = t->poll()).status == kh::TransferStatus::Pending) {
        }
        require(pl.status == kh::TransferStatus::Complete, "restore failed: " + pl.error);
        t->publish(plan.next);
    }
    std::vector<uint64_t> ids(sel.begin(), sel.end());
    require(mem.resident() == ids && mem.stamp().view_version == snap.stamp.view_version + 1, "published view");
    const size_t span = size_t(BT) * W * 2;
    for (size_t i = 0; i < attn.size(); ++i) {
        const auto ks = slots[2 * i]->down(), vs = slots[2 * i + 1]->down();
        for (size_t s = 0; s < sel.size(); ++s) {
            const size_t n = std::min<size_t>(span, size_t(TOK) * W * 2 - sel[s] * span);
            require(std::memcmp(ks.data() + s * span, reinterpret_cast<const uint8_t *>(keys[attn[i]].data()) + sel[s] * span,
                                n) == 0,
                    "restored K bytes");
            require(std::memcmp(vs.data() + s * span, vals[i].data() + sel[s] * span, n) == 0, "restored V bytes");
        }
    }

    // plan errors
    require(plan_error([&] { mem.prepare(plan); }) == kh::MemoryErrorCode::Stale, "old stamp accepted");
    kh::WorkingSetPlan big = plan;
    big.expected = mem.stamp();
    big.next.blocks.clear();
    for (uint32_t i = 0; i < 11; ++i) {
        kh::ViewBlock vb;
        vb.block = mem.snapshot().blocks[i].block;
        vb.compact_start = uint64_t(i) * BT;
        big.next.blocks.push_back(vb);
    }
    require(plan_error([&] { mem.prepare(big); }) == kh::MemoryErrorCode::BudgetExceeded, "11 pages accepted");
    kh::WorkingSetPlan unordered = big;
    unordered.next.blocks.resize(3);
    std::swap(unordered.next.blocks[0], unordered.next.blocks[1]);
    require(plan_error([&] { mem.prepare(unordered); }) == kh::MemoryErrorCode::InvalidPlan, "unordered view accepted");

    // decode after the pin: K of position 1600 opens page 25
    llama_kvmem_end_prefill_capture();
    llama_kvmem_pin_working_set();
    require(llama_kvmem_want_decode_mean() && !llama_kvmem_want_prefill_capture(), "pinned");
    const llama_pos dpos = llama_pos(TOK);
    llama_kvmem_capture_on_new_graph(0);
    require(!llama_kvmem_capture_can_reuse(1, 1, &dpos, 0), "a pinned decode graph without K is reusable");
    std::vector<uint16_t> krow(keys[0].begin() + size_t(TOK) * W, keys[0].begin() + size_t(TOK + 1) * W);
    Dev<uint16_t> kd(krow);
    ggml_tensor kdt;
    kdt.view = {kd.p, KVR_FMT_F16, {D, HKV, 1, 1}, {2, D * 2, size_t(W) * 2, size_t(W) * 2}};
    llama_kvmem_register_capture(&kdt, 0, 'k');
    require(llama_kvmem_capture_can_reuse(1, 1, &dpos, 0), "a pinned decode graph with K is not reusable");
    const auto before = mem.stamp();
    mem.note_ubatch({dpos});
    llama_kvmem_harvest_ubatch(&sched, 0);
    require(mem.frontier() == TOK + 1 && mem.pages() == 26 && mem.stamp().history_revision == before.history_revision + 1,
            "decode token captured");
    const auto s16 = mem.summaries();
    std::vector<uint16_t> page25(W);
    hip(hipMemcpy(page25.data(), s16.layers[0] + size_t(25) * W, W * 2, hipMemcpyDeviceToHost), "D2H");
    for (uint32_t c = 0; c < W; ++c) {
        float r = 0;
        require(orc_recall_fp16(orc_f16_to_f32(krow[c]), &r) == ORC_OK && orc_f32_to_f16(r) == page25[c],
                "decode page summary is the token's K");
    }
    kh::WorkingSetPlan stale = plan;
    stale.expected = before;
    require(plan_error([&] { mem.prepare(stale); }) == kh::MemoryErrorCode::Stale, "plan older than a capture accepted");

    // attention samples of layer 0 through the hook equal the sampler's own
    {
        const uint32_t qrows = 130, tokens = 700;
        std::vector<float> aq(size_t(qrows) * HQ * D);
        for (auto &x : aq) x = nd(rng);
        std::vector<uint16_t> ak(size_t(tokens) * W), am(size_t(qrows) * tokens);
        for (auto &x : ak) x = orc_f32_to_f16(nd(rng));
        for (uint32_t r = 0; r < qrows; ++r)
            for (uint32_t t = 0; t < tokens; ++t) am[size_t(r) * tokens + t] = t <= tokens - qrows + r ? 0 : 0xfc00;
        Dev<float> qd(aq);
        Dev<uint16_t> kd2(ak), md(am);
        ggml_tensor tq, tk, tmask;
        tq.view = {qd.p, KVR_FMT_F32, {D, qrows, HQ, 1}, {4, size_t(HQ) * D * 4, size_t(D) * 4, 0}};
        tk.view = {kd2.p, KVR_FMT_F16, {D, tokens, HKV, 1}, {2, size_t(W) * 2, size_t(D) * 2, 0}};
        tmask.view = {md.p, KVR_FMT_F16, {tokens, qrows, 1, 1}, {2, size_t(tokens) * 2, 0, 0}};
        llama_kvmem_capture_on_new_graph(0);
        llama_kvmem_capture_attention(nullptr, nullptr, &tq, &tk, &tmask, 0.125f, 0.0f, 0.0f, 0);
        llama_kvmem_capture_attention(nullptr, nullptr, &tq, &tk, &tmask, 0.125f, 1.0f, 0.0f, 0);  // declined
        llama_kvmem_register_capture(&kdt, 0, 'k');
        const llama_pos p2 = llama_pos(TOK + 1);
        mem.note_ubatch({p2});
        llama_kvmem_harvest_ubatch(&sched, 0);
        const auto masses = kh::take_attention_masses();
        kh::AttentionSamplerHip sampler;
        auto view = [](const ggml_tensor &t) {
            kh::AttentionTensor a;
            a.data = t.view.data, a.type = t.view.type;
            for (int i = 0; i < 3; ++i) a.ne[i] = t.view.ne[i], a.nb[i] = t.view.nb[i];
            return a;
        };
        std::vector<std::vector<float>> out;
        require(sampler.score(view(tq), view(tk), view(tmask), 0.125f, 0.0f, BT, {127, 129}, out), "sampler");
        const uint32_t pages = (tokens + BT - 1) / BT;
        require(masses.size() == pages, "attention masses per page");
        double total = 0;
        for (uint32_t pg = 0; pg < pages; ++pg) {
            const double w = (double(out[0][pg]) + out[1][pg]) / 2;
            require(std::fabs(masses[pg] - w) <= 1e-9, "hook masses differ from the sampler's");
            total += masses[pg];
        }
        require(std::fabs(total - 1.0) < 1e-5, "masses sum to one");
    }

    mem.invalidate();
    plan.expected = mem.stamp();
    require(plan_error([&] { mem.prepare(plan); }) == kh::MemoryErrorCode::InvalidSession, "invalidated memory prepared");
    wrapper.reset();
    require(kh::current_memory() == nullptr && llama_kvmem_capture_stamp() == 0, "memory unbound on destruction");
    llama_kvmem_set_params(nullptr);
}

}  // namespace

int main(int argc, char **argv) {
    const bool gpu = argc > 1 && std::string(argv[1]) == "--gpu";
    std::vector<std::pair<const char *, std::function<void()>>> tests = {{"declines_and_plans", declines_and_plans}};
    if (gpu) tests = {{"end_to_end", end_to_end}};
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
