// kvr_policy.cpp -- host-side page policies around the scored pick: media
// page groups and the fixed-page lists of KvMemStore's pickers.  None of
// them reads a score, so they run on the host before the device selection
// (kvr_select_pages / kvr_layer_recall.policy) that does.
//
// Rules restated here (kvmem/src/host/kvmem_store.cpp):
//  - a media token range [first, end) covers pages [first / pt,
//    min(pages, ceil(end / pt)));
//  - OVERLAP groups (scored_media_group, :18-32): ranges sharing a page join,
//    transitively; a page in no range is alone;
//  - IN_ORDER groups (constrain_media, :453-468): ranges starting at or past
//    the history's end, or empty, are dropped; in list order, a range that
//    starts before the last group's end extends that end, else starts a
//    group;
//  - keeping a page keeps its whole group, or nothing when the group does
//    not fit; a required keep that does not fit fails the pick.
#include "kvrecall.h"

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <string>
#include <vector>

namespace kvr {
// kvr_capi.cpp's error reporting (the thread's kvr_last_error message).
kvr_status set_error(kvr_status s, const char *message);
}  // namespace kvr

namespace {

kvr_status fail(kvr_status s, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    return kvr::set_error(s, buf);
}

struct Span {
    uint32_t begin, end;  // pages [begin, end); may be empty (IN_ORDER keeps it for merging)
};

kvr_status check_media(const kvr_media *m) {
    if (!m) return KVR_OK;
    if (m->n_ranges && !m->ranges) return fail(KVR_ERR_INVALID, "media ranges missing");
    if (!m->page_tokens) return fail(KVR_ERR_INVALID, "media page_tokens must be nonzero");
    return KVR_OK;
}

std::vector<Span> group_spans(const kvr_media *m, uint32_t pages, kvr_media_merge merge) {
    std::vector<Span> v;
    if (!m) return v;
    const uint64_t pt = m->page_tokens;
    for (uint32_t r = 0; r < m->n_ranges; ++r) {
        const uint32_t first_tok = m->ranges[2 * r], end_tok = m->ranges[2 * r + 1];
        const uint32_t lo = uint32_t(first_tok / pt);
        const uint32_t hi = uint32_t(std::min<uint64_t>(pages, (uint64_t(end_tok) + pt - 1) / pt));
        if (merge == KVR_MEDIA_IN_ORDER) {
            if (first_tok >= m->total_tokens || end_tok <= first_tok) continue;
            if (!v.empty() && lo < v.back().end) v.back().end = std::max(v.back().end, hi);
            else v.push_back({lo, hi});
        } else if (lo < hi) {
            v.push_back({lo, hi});
        }
    }
    if (merge == KVR_MEDIA_OVERLAP) {
        // components of "shares a page": sweep in start order
        std::sort(v.begin(), v.end(), [](const Span &a, const Span &b) { return a.begin < b.begin; });
        std::vector<Span> merged;
        for (const Span &s : v) {
            if (!merged.empty() && s.begin < merged.back().end) merged.back().end = std::max(merged.back().end, s.end);
            else merged.push_back(s);
        }
        v.swap(merged);
    }
    return v;
}

// Pages chosen one keep at a time under a budget, each keep taking its whole
// group.  Groups are disjoint and ascending (the empty ones never match).
class Keeper {
public:
    Keeper(uint32_t pages, uint32_t budget, std::vector<Span> groups)
        : kept_(pages, 0), budget_(budget), groups_(std::move(groups)) {}

    uint32_t count() const { return count_; }
    bool full() const { return count_ >= budget_; }

    Span group_of(uint32_t page) const {
        auto it = std::upper_bound(groups_.begin(), groups_.end(), page,
                                   [](uint32_t p, const Span &s) { return p < s.begin; });
        if (it != groups_.begin()) {
            --it;
            if (page >= it->begin && page < it->end) return *it;
        }
        return {page, page + 1};
    }

    // false when the group does not fit (nothing kept)
    bool keep(uint32_t page) {
        const Span g = group_of(page);
        uint32_t need = 0;
        for (uint32_t p = g.begin; p < g.end; ++p) need += !kept_[p];
        if (count_ + need > budget_) return false;
        for (uint32_t p = g.begin; p < g.end; ++p) kept_[p] = 1;
        count_ += need;
        return true;
    }
    // a page on its own, no group (the ungrouped picker)
    void keep_alone(uint32_t page) {
        if (!kept_[page]) {
            kept_[page] = 1;
            ++count_;
        }
    }

    uint32_t emit(uint32_t *out) const {
        uint32_t o = 0;
        for (uint32_t p = 0; p < kept_.size(); ++p)
            if (kept_[p]) out[o++] = p;
        return o;
    }

private:
    std::vector<uint8_t> kept_;
    uint32_t count_ = 0, budget_;
    std::vector<Span> groups_;
};

kvr_status all_pages(uint32_t pages, uint32_t *out, uint32_t *n_out) {
    for (uint32_t p = 0; p < pages; ++p) out[p] = p;
    *n_out = pages;
    return KVR_OK;
}

}  // namespace

extern "C" {

kvr_status kvr_media_page_groups(const kvr_media *media, uint32_t pages, kvr_media_merge merge, uint32_t *groups,
                                 uint32_t *n_groups) {
    if (!n_groups || (media && media->n_ranges && !groups)) return fail(KVR_ERR_INVALID, "missing group output");
    if (merge != KVR_MEDIA_OVERLAP && merge != KVR_MEDIA_IN_ORDER) return fail(KVR_ERR_INVALID, "unknown merge rule");
    *n_groups = 0;
    if (kvr_status s = check_media(media)) return s;
    uint32_t o = 0;
    for (const Span &g : group_spans(media, pages, merge)) {
        const uint32_t end = std::min(g.end, pages);
        if (g.begin >= end) continue;
        groups[2 * o] = g.begin;
        groups[2 * o + 1] = end;
        ++o;
    }
    *n_groups = o;
    return KVR_OK;
}

kvr_status kvr_query_fixed_pages(uint32_t pages, uint32_t budget, uint32_t sink, uint32_t recent,
                                 const kvr_media *media, const uint32_t *mandatory, uint32_t n_mandatory,
                                 uint32_t *out, uint32_t *n_out) {
    if (!out || !n_out || (n_mandatory && !mandatory)) return fail(KVR_ERR_INVALID, "missing fixed-page arguments");
    *n_out = 0;
    if (kvr_status s = check_media(media)) return s;
    if (!budget || pages <= budget) return all_pages(pages, out, n_out);
    Keeper k(pages, budget, group_spans(media, pages, KVR_MEDIA_OVERLAP));
    auto required = [&](uint32_t page, const char *what) -> kvr_status {
        if (page >= pages) return fail(KVR_ERR_INVALID, "%s page %u is outside %u pages", what, page, pages);
        if (!k.keep(page))
            return fail(KVR_ERR_BUDGET, "%s page %u with its media group exceeds the selection budget %u", what, page,
                        budget);
        return KVR_OK;
    };
    for (uint32_t p = 0; p < std::min(pages, sink); ++p)
        if (kvr_status s = required(p, "sink")) return s;
    if (media && media->n_ranges) {
        const uint32_t first = media->ranges[2 * (media->n_ranges - 1)];
        if (first < media->total_tokens)
            if (kvr_status s = required(first / media->page_tokens, "last media")) return s;
    }
    for (uint32_t i = 0; i < n_mandatory; ++i)
        if (kvr_status s = required(mandatory[i], "mandatory")) return s;
    for (uint32_t i = 0; i < std::min(pages, recent); ++i) k.keep(pages - 1 - i);  // best effort
    *n_out = k.emit(out);
    return KVR_OK;
}

kvr_status kvr_topk_fixed_pages(uint32_t pages, uint32_t budget, uint32_t sink, uint32_t recent,
                                const uint32_t *mandatory, uint32_t n_mandatory, uint32_t *out, uint32_t *n_out) {
    if (!out || !n_out || (n_mandatory && !mandatory)) return fail(KVR_ERR_INVALID, "missing fixed-page arguments");
    *n_out = 0;
    if (!budget || pages <= budget) return all_pages(pages, out, n_out);
    Keeper k(pages, budget, {});
    for (uint32_t p = 0; p < std::min(sink, pages) && !k.full(); ++p) k.keep_alone(p);
    for (uint32_t i = n_mandatory; i > 0 && !k.full(); --i)  // newest request first
        if (mandatory[i - 1] < pages) k.keep_alone(mandatory[i - 1]);
    for (uint32_t i = 0; i < std::min(recent, pages) && !k.full(); ++i) k.keep_alone(pages - 1 - i);
    *n_out = k.emit(out);
    return KVR_OK;
}

kvr_status kvr_media_fixed_pages(uint32_t pages, uint32_t budget, uint32_t sink, const kvr_media *media,
                                 const uint32_t *mandatory, uint32_t n_mandatory, uint32_t *out, uint32_t *n_out) {
    if (!out || !n_out || (n_mandatory && !mandatory)) return fail(KVR_ERR_INVALID, "missing fixed-page arguments");
    *n_out = 0;
    if (kvr_status s = check_media(media)) return s;
    const std::vector<Span> groups = group_spans(media, pages, KVR_MEDIA_IN_ORDER);
    std::vector<Span> clipped;
    for (const Span &g : groups)
        if (g.begin < std::min(g.end, pages)) clipped.push_back({g.begin, std::min(g.end, pages)});
    Keeper k(pages, budget, clipped);
    for (uint32_t p = 0; p < std::min(pages, sink); ++p)
        if (!k.keep(p)) return fail(KVR_ERR_BUDGET, "sink page %u exceeds the selection budget %u", p, budget);
    if (!groups.empty() && groups.back().begin < pages && !k.keep(groups.back().begin))
        return fail(KVR_ERR_BUDGET, "the last media group exceeds the selection budget %u", budget);
    std::vector<uint32_t> newest(mandatory, mandatory + n_mandatory);
    std::sort(newest.begin(), newest.end(), [](uint32_t a, uint32_t b) { return a > b; });
    for (uint32_t p : newest)
        if (p < pages) k.keep(p);  // best effort
    *n_out = k.emit(out);
    return KVR_OK;
}

}  // extern "C"
