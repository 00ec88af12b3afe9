/*
 * kvr_oracle.c -- CPU restatement of KVMem's recall hot path.
 *
 * TEST INFRASTRUCTURE ONLY: imported by tests/, by the smoke entry point and
 * by the benchmark's CPU-baseline leg, never by the product library.
 *
 * Build with plain `gcc -O2 -std=c99` for x86-64 WITHOUT -mfma / -march=native:
 * the reference is compiled the same way, so `a*b + c` stays two roundings.
 * Reference citations are relative to the KVMem 0.19.0 source tree.
 */
#include "kvr_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------------- */
/* IEEE binary32 <-> binary16, round to nearest even.                       */
/* Restates f32_to_f16 / f16_to_f32 (kvmem/src/host/raw_kv_store.cpp:43-104) */
/* ---------------------------------------------------------------------- */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t biased = (x >> 23) & 0xffu;
    uint32_t mant = x & 0x7fffffu;
    if (biased == 0xffu) /* inf stays inf, NaN becomes a quiet NaN */
        return (uint16_t)(sign | 0x7c00u | (mant ? 0x200u : 0u));
    if ((x & 0x7fffffffu) == 0) return sign;
    const int e = (int)biased - 127 + 15; /* binary16 biased exponent */
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        /* binary16 subnormal: value / 2^-24 rounded to an integer */
        if (e < -10) return sign;
        mant |= 0x800000u;
        const uint32_t shift = (uint32_t)(14 - e);
        uint32_t q = mant >> shift;
        const uint32_t rest = mant & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1);
        if (rest > half || (rest == half && (q & 1u))) q += 1;
        return (uint16_t)(sign | q);
    }
    uint32_t h = ((uint32_t)e << 10) | (mant >> 13);
    const uint32_t rest = mant & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1; /* may carry into inf */
    return (uint16_t)(sign | h);
}

float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0x1f) {
        bits = sign | 0x7f800000u | (m << 13);
    } else if (e != 0) {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    } else if (m == 0) {
        bits = sign;
    } else {
        /* subnormal: m * 2^-24 is exact in binary32 */
        float v = (float)m * 5.9604644775390625e-08f;
        memcpy(&bits, &v, 4);
        bits |= sign;
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

/* The fp16 operand boundary: graph_recall.cpp:295-320 (recall_fp16).
 * Non-finite input and values that round to fp16 infinity are rejected. */
int orc_recall_fp16(float value, float *out) {
    if (!isfinite(value)) return ORC_ERR_NONFINITE;
    const uint16_t h = orc_f32_to_f16(value);
    if ((h & 0x7fffu) == 0x7c00u) return ORC_ERR_RANGE;
    *out = orc_f16_to_f32(h);
    return ORC_OK;
}

/* ---------------------------------------------------------------------- */
/* Score frame: graph_recall.cpp:269-293 (query_score_frame).               */
/* ---------------------------------------------------------------------- */
uint32_t orc_page_count(uint64_t accepted, uint32_t block_tokens) {
    if (!block_tokens) return 0;
    return (uint32_t)(accepted / block_tokens + (accepted % block_tokens != 0));
}

int orc_query_score_frame(uint64_t accepted, uint32_t block_tokens, uint32_t budget,
                          uint32_t sink, uint32_t recent, const uint32_t *fixed,
                          uint32_t n_fixed, uint64_t *starts, uint32_t *counts,
                          uint8_t *score_mask, uint8_t *transport_mask) {
    if (!block_tokens || !budget) return ORC_ERR_ARG;
    const uint64_t n64 = accepted / block_tokens + (accepted % block_tokens != 0);
    if (n64 > 0xffffffffull) return ORC_ERR_ARG;
    const uint32_t n = (uint32_t)n64;
    for (uint32_t i = 0; i < n; ++i) {
        const uint64_t start = (uint64_t)i * block_tokens;
        const uint64_t left = accepted - start;
        starts[i] = start;
        counts[i] = (uint32_t)(left < block_tokens ? left : block_tokens);
        score_mask[i] = 1;
        transport_mask[i] = n > budget;
    }
    if (n > budget && (uint64_t)sink + recent < n) {
        const uint32_t s = sink < n ? sink : n, r = recent < n ? recent : n;
        for (uint32_t i = 0; i < s; ++i) score_mask[i] = 0;
        for (uint32_t i = n - r; i < n; ++i) score_mask[i] = 0;
    }
    for (uint32_t i = 0; i < n_fixed; ++i) {
        if (fixed[i] >= n) return ORC_ERR_ARG;
        transport_mask[fixed[i]] = 0;
    }
    return ORC_OK;
}

/* ---------------------------------------------------------------------- */
/* Block formats.                                                           */
/* q8_0 dequant/quant: src/adapter/llama-kvmem-stagein.cu:19-29, 133-143,   */
/* 181-199.  q4_1 ({d, m, 16 nibble bytes}; low nibble -> j, high -> j+16)  */
/* is ggml's layout (third party, un-vendored); the nibble order matches    */
/* the reference's q4_0 kernel (stagein.cu:145-158).                        */
/* ---------------------------------------------------------------------- */
static uint16_t load_u16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static void store_u16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

void orc_dequant_q8_0(const uint8_t *block, float *y) {
    const float d = orc_f16_to_f32(load_u16(block));
    const int8_t *qs = (const int8_t *)(block + 2);
    for (int j = 0; j < ORC_QK; ++j) y[j] = (float)qs[j] * d;
}

void orc_dequant_q4_1(const uint8_t *block, float *y) {
    const float d = orc_f16_to_f32(load_u16(block));
    const float m = orc_f16_to_f32(load_u16(block + 2));
    const uint8_t *qs = block + 4;
    for (int j = 0; j < ORC_QK / 2; ++j) {
        const float lo = (float)(qs[j] & 15) * d;
        const float hi = (float)(qs[j] >> 4) * d;
        y[j] = lo + m;
        y[j + ORC_QK / 2] = hi + m;
    }
}

void orc_quant_q8_0(const float *x, uint8_t *block) {
    float amax = 0.0f;
    for (int j = 0; j < ORC_QK; ++j) amax = fmaxf(amax, fabsf(x[j]));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    store_u16(block, orc_f32_to_f16(d));
    int8_t *qs = (int8_t *)(block + 2);
    for (int j = 0; j < ORC_QK; ++j) qs[j] = (int8_t)roundf(x[j] * id);
}

size_t orc_row_bytes(int fmt, uint32_t width) {
    switch (fmt) {
    case ORC_FMT_F16: return (size_t)width * 2;
    case ORC_FMT_Q8_0: return width % ORC_QK ? 0 : (size_t)width / ORC_QK * ORC_Q8_0_BYTES;
    case ORC_FMT_Q4_1: return width % ORC_QK ? 0 : (size_t)width / ORC_QK * ORC_Q4_1_BYTES;
    default: return 0;
    }
}

/* Decode one token row of `width` channels to binary32. */
static void decode_row(const uint8_t *row, int fmt, uint32_t width, float *out) {
    if (fmt == ORC_FMT_F16) {
        for (uint32_t c = 0; c < width; ++c) out[c] = orc_f16_to_f32(load_u16(row + 2 * c));
    } else if (fmt == ORC_FMT_Q8_0) {
        for (uint32_t b = 0; b < width / ORC_QK; ++b)
            orc_dequant_q8_0(row + (size_t)b * ORC_Q8_0_BYTES, out + (size_t)b * ORC_QK);
    } else {
        for (uint32_t b = 0; b < width / ORC_QK; ++b)
            orc_dequant_q4_1(row + (size_t)b * ORC_Q4_1_BYTES, out + (size_t)b * ORC_QK);
    }
}

/* ---------------------------------------------------------------------- */
/* Page summaries: per channel a binary32 running sum over the page's      */
/* tokens in token order starting from zero, then sum * (1.0f / n).        */
/* RawKvStore::capture_mean_f16 / add_mean_f32 (raw_kv_store.cpp:158-197)  */
/* and RawKvStore::mean_k (raw_kv_store.cpp:606-625).                      */
/* ---------------------------------------------------------------------- */
int orc_page_summaries(const void *keys, int fmt, uint64_t tokens, uint32_t width,
                       uint32_t page_tokens, float *sums, float *means) {
    const size_t row = orc_row_bytes(fmt, width);
    if (!row || !page_tokens || !width) return ORC_ERR_ARG;
    const uint32_t pages = orc_page_count(tokens, page_tokens);
    float *value = (float *)malloc(sizeof(float) * width);
    float *sum = (float *)malloc(sizeof(float) * width);
    if (!value || !sum) { free(value); free(sum); return ORC_ERR_ARG; }
    for (uint32_t p = 0; p < pages; ++p) {
        const uint64_t start = (uint64_t)p * page_tokens;
        const uint32_t n = (uint32_t)(tokens - start < page_tokens ? tokens - start : page_tokens);
        for (uint32_t c = 0; c < width; ++c) sum[c] = 0.0f;
        for (uint32_t t = 0; t < n; ++t) {
            decode_row((const uint8_t *)keys + (start + t) * row, fmt, width, value);
            for (uint32_t c = 0; c < width; ++c) sum[c] += value[c];
        }
        const float inv = 1.0f / (float)n;
        for (uint32_t c = 0; c < width; ++c) {
            if (sums) sums[(size_t)p * width + c] = sum[c];
            if (means) means[(size_t)p * width + c] = sum[c] * inv;
        }
    }
    free(value);
    free(sum);
    return ORC_OK;
}

/* ---------------------------------------------------------------------- */
/* Page softmax scoring: graph_recall.cpp:322-394 (page_softmax_scores).    */
/*   logit_j = scale * sum_d fp16(q_d) * fp16(mean_{j,d})  (double, d order) */
/*   Mean: out_j += p_j / (A * Hq)                                          */
/*   Max:  out_j += gmax_j / sum_j gmax_j / (A * Hkv), gmax = max over the   */
/*         group's head probabilities                                       */
/*   MaxLogit (literal "max of logits, then softmax" variant):               */
/*         out_j += softmax_j(max_{h in g} logit_{h,j}) / (A * Hkv)          */
/* Rows of all active layers are summed.  Pages outside score_mask get 0 and */
/* stay out of every denominator.                                           */
/* ---------------------------------------------------------------------- */
static double page_scale(float attention_scale, uint32_t head_dim) {
    return attention_scale > 0 ? (double)attention_scale : 1 / sqrt((double)head_dim);
}

int orc_page_softmax_scores(const float *means, const float *query,
                            const uint32_t *layer_rows, uint32_t layers, uint32_t rows,
                            uint32_t query_heads, uint32_t kv_heads, uint32_t head_dim,
                            uint32_t pages, const uint8_t *score_mask,
                            float attention_scale, int aggregation, double *out) {
    if (!means || !query || !layer_rows || !layers || !rows || !query_heads || !kv_heads ||
        !head_dim || query_heads % kv_heads || !out ||
        (aggregation != ORC_AGG_MEAN && aggregation != ORC_AGG_MAX &&
         aggregation != ORC_AGG_MAX_LOGIT))
        return ORC_ERR_ARG;
    for (uint32_t j = 0; j < pages; ++j) out[j] = 0;
    uint32_t active = 0;
    for (uint32_t l = 0; l < layers; ++l) {
        if (layer_rows[l] > rows) return ORC_ERR_ARG;
        active += layer_rows[l] != 0;
    }
    uint32_t n = 0;
    uint32_t *enabled = (uint32_t *)malloc(sizeof(uint32_t) * (pages ? pages : 1));
    for (uint32_t j = 0; j < pages; ++j)
        if (!score_mask || score_mask[j]) enabled[n++] = j;
    if (!n || !active) { free(enabled); return ORC_OK; }

    const size_t kw = (size_t)kv_heads * head_dim, qw = (size_t)query_heads * head_dim;
    const uint32_t group = query_heads / kv_heads;
    float *m16 = (float *)malloc(sizeof(float) * n * kw);
    float *q16 = (float *)malloc(sizeof(float) * head_dim);
    double *logit = (double *)malloc(sizeof(double) * n);
    double *gmax = (double *)malloc(sizeof(double) * n);
    const double scale = page_scale(attention_scale, head_dim);
    int status = ORC_OK;

    for (uint32_t l = 0; l < layers && status == ORC_OK; ++l) {
        if (!layer_rows[l]) continue;
        for (uint32_t j = 0; j < n && status == ORC_OK; ++j)
            for (size_t d = 0; d < kw && status == ORC_OK; ++d)
                status = orc_recall_fp16(means[((size_t)l * pages + enabled[j]) * kw + d],
                                         &m16[(size_t)j * kw + d]);
        for (uint32_t t = 0; t < layer_rows[l] && status == ORC_OK; ++t) {
            for (uint32_t h = 0; h < query_heads && status == ORC_OK; ++h) {
                const uint32_t g = h / group;
                const float *qrow = query + ((size_t)l * rows + t) * qw + (size_t)h * head_dim;
                for (uint32_t d = 0; d < head_dim && status == ORC_OK; ++d)
                    status = orc_recall_fp16(qrow[d], &q16[d]);
                if (status != ORC_OK) break;
                double maximum = -INFINITY;
                for (uint32_t j = 0; j < n; ++j) {
                    double dot = 0;
                    const float *mrow = m16 + (size_t)j * kw + (size_t)g * head_dim;
                    for (uint32_t d = 0; d < head_dim; ++d) dot += (double)q16[d] * mrow[d];
                    logit[j] = dot * scale;
                    if (logit[j] > maximum) maximum = logit[j];
                }
                if (aggregation == ORC_AGG_MAX_LOGIT) {
                    /* running max of logits across the group's heads */
                    for (uint32_t j = 0; j < n; ++j)
                        gmax[j] = (h % group == 0 || logit[j] > gmax[j]) ? logit[j] : gmax[j];
                    if (h % group != group - 1) continue;
                    double gm = -INFINITY, denom = 0;
                    for (uint32_t j = 0; j < n; ++j) gm = gmax[j] > gm ? gmax[j] : gm;
                    for (uint32_t j = 0; j < n; ++j) denom += gmax[j] = exp(gmax[j] - gm);
                    for (uint32_t j = 0; j < n; ++j)
                        out[enabled[j]] += gmax[j] / denom / ((double)active * kv_heads);
                    continue;
                }
                double denom = 0;
                for (uint32_t j = 0; j < n; ++j) denom += logit[j] = exp(logit[j] - maximum);
                if (aggregation == ORC_AGG_MEAN) {
                    for (uint32_t j = 0; j < n; ++j)
                        out[enabled[j]] += logit[j] / denom / ((double)active * query_heads);
                } else {
                    if (h % group == 0)
                        for (uint32_t j = 0; j < n; ++j) gmax[j] = 0.0;
                    for (uint32_t j = 0; j < n; ++j) {
                        const double p = logit[j] / denom;
                        gmax[j] = p > gmax[j] ? p : gmax[j];
                    }
                    if (h % group == group - 1) {
                        double mass = 0;
                        for (uint32_t j = 0; j < n; ++j) mass += gmax[j];
                        for (uint32_t j = 0; j < n; ++j)
                            out[enabled[j]] += gmax[j] / mass / ((double)active * kv_heads);
                    }
                }
            }
        }
    }
    free(enabled); free(m16); free(q16); free(logit); free(gmax);
    if (status != ORC_OK)
        for (uint32_t j = 0; j < pages; ++j) out[j] = 0;
    return status;
}

/* Single-layer logits of every page (no mask, no softmax), double, with the
 * same operand rounding and dot order as orc_page_softmax_scores.
 * logits[(r * Hq + h) * pages + j]. */
int orc_page_logits(const float *means, const float *query, uint32_t rows,
                    uint32_t query_heads, uint32_t kv_heads, uint32_t head_dim,
                    uint32_t pages, float attention_scale, double *logits) {
    if (!means || !query || !rows || !query_heads || !kv_heads || !head_dim ||
        query_heads % kv_heads || !logits)
        return ORC_ERR_ARG;
    const size_t kw = (size_t)kv_heads * head_dim;
    const uint32_t group = query_heads / kv_heads;
    const double scale = page_scale(attention_scale, head_dim);
    for (uint32_t r = 0; r < rows; ++r)
        for (uint32_t h = 0; h < query_heads; ++h)
            for (uint32_t j = 0; j < pages; ++j) {
                double dot = 0;
                for (uint32_t d = 0; d < head_dim; ++d) {
                    float qv, mv;
                    int s = orc_recall_fp16(query[((size_t)r * query_heads + h) * head_dim + d], &qv);
                    if (s) return s;
                    s = orc_recall_fp16(means[(size_t)j * kw + (size_t)(h / group) * head_dim + d], &mv);
                    if (s) return s;
                    dot += (double)qv * mv;
                }
                logits[((size_t)r * query_heads + h) * pages + j] = dot * scale;
            }
    return ORC_OK;
}

/* ---------------------------------------------------------------------- */
/* Top-k: KvMemStore::pick_scored_blocks (kvmem_store.cpp:418-451) with     */
/* every page a candidate and no media groups.  Mandatory pages are kept    */
/* first; the rest ranked by (score desc, page id by tie rule) fill the     */
/* budget.  The reference's rule is HIGHER_FIRST (kvmem_store.cpp:444-446). */
/* Output ascending ids.                                                    */
/* ---------------------------------------------------------------------- */
static int ranks_before(const double *s, uint32_t a, uint32_t b, int tie_rule) {
    if (s[a] != s[b]) return s[a] > s[b];
    return tie_rule == ORC_TIE_HIGHER_FIRST ? a > b : a < b;
}

static void rank_sort(uint32_t *ids, uint32_t *tmp, uint32_t n, const double *s, int tie) {
    if (n < 2) return;
    const uint32_t h = n / 2;
    rank_sort(ids, tmp, h, s, tie);
    rank_sort(ids + h, tmp, n - h, s, tie);
    uint32_t i = 0, j = h, o = 0;
    while (i < h && j < n) tmp[o++] = ranks_before(s, ids[j], ids[i], tie) ? ids[j++] : ids[i++];
    while (i < h) tmp[o++] = ids[i++];
    while (j < n) tmp[o++] = ids[j++];
    memcpy(ids, tmp, sizeof(uint32_t) * n);
}

int orc_pick_scored_blocks(const double *scores, uint32_t n, const uint32_t *mandatory,
                           uint32_t n_mandatory, uint32_t budget, int tie_rule,
                           int signed_scores, uint32_t *out, uint32_t *n_out) {
    *n_out = 0;
    if (!budget || (n && !scores)) return ORC_ERR_ARG;
    for (uint32_t i = 0; i < n; ++i)
        if (!isfinite(scores[i]) || (!signed_scores && scores[i] < 0)) return ORC_ERR_ARG;
    uint8_t *kept = (uint8_t *)calloc(n ? n : 1, 1);
    uint32_t count = 0;
    for (uint32_t i = 0; i < n_mandatory; ++i) {
        const uint32_t id = mandatory[i];
        if (id >= n) { free(kept); return ORC_ERR_ARG; }
        if (kept[id]) continue;
        if (count + 1 > budget) { free(kept); return ORC_ERR_BUDGET; }
        kept[id] = 1;
        ++count;
    }
    uint32_t *ids = (uint32_t *)malloc(sizeof(uint32_t) * (n ? n : 1));
    uint32_t *tmp = (uint32_t *)malloc(sizeof(uint32_t) * (n ? n : 1));
    for (uint32_t i = 0; i < n; ++i) ids[i] = i;
    rank_sort(ids, tmp, n, scores, tie_rule);
    for (uint32_t i = 0; i < n && count < budget; ++i)
        if (!kept[ids[i]]) { kept[ids[i]] = 1; ++count; }
    uint32_t o = 0;
    for (uint32_t i = 0; i < n; ++i)
        if (kept[i]) out[o++] = i;
    *n_out = o;
    free(kept); free(ids); free(tmp);
    return ORC_OK;
}

/* ---------------------------------------------------------------------- */
/* Half-page layerwise scores: layerwise_tile_scores' fold                  */
/* (layerwise_selection.cpp:60-72) and layerwise_max_page_scores (:24-30).  */
/* mass holds 2*count half-page masses in page order (the softmax over the  */
/* halves frame); a negative half, a non-finite pair sum or mass on a page  */
/* outside score_mask is invalid.  keep_halves 0: out[i] = left + right;    */
/* 1: out[i] = std::max(left, right), i.e. right when left < right.         */
/* ---------------------------------------------------------------------- */
int orc_layerwise_fold(const double *mass, uint32_t count, const uint8_t *score_mask, int keep_halves,
                       double *out) {
    for (uint32_t i = 0; i < count; ++i) {
        const double left = mass[2 * i], right = mass[2 * i + 1], sum = left + right;
        if (left < 0 || right < 0 || !isfinite(sum) || (score_mask && !score_mask[i] && sum != 0))
            return ORC_ERR_ARG;
    }
    for (uint32_t i = 0; i < count; ++i) {
        const double left = mass[2 * i], right = mass[2 * i + 1];
        out[i] = keep_halves ? (left < right ? right : left) : left + right;
    }
    return ORC_OK;
}

/* ---------------------------------------------------------------------- */
/* Page policies around the scored pick (kvmem_store.cpp).  Media ranges    */
/* are token ranges [first, end), ranges[2*i], ranges[2*i+1].               */
/* ---------------------------------------------------------------------- */

/* scored_media_group (kvmem_store.cpp:18-32): the pages kept together with */
/* page id -- every range sharing a page with the group joins it, until     */
/* nothing changes; a page in no range is alone.                            */
void orc_media_group(uint32_t id, uint32_t n, uint32_t page_tokens, const uint32_t *ranges,
                     uint32_t n_ranges, uint32_t *begin_out, uint32_t *end_out) {
    uint32_t begin = id, end = id + 1;
    int changed;
    do {
        const uint32_t old_begin = begin, old_end = end;
        for (uint32_t r = 0; r < n_ranges; ++r) {
            const uint32_t lo = ranges[2 * r] / page_tokens;
            const uint64_t up = ((uint64_t)ranges[2 * r + 1] + page_tokens - 1) / page_tokens;
            const uint32_t hi = up < n ? (uint32_t)up : n;
            if (lo < end && begin < hi) {
                if (lo < begin) begin = lo;
                if (hi > end) end = hi;
            }
        }
        changed = old_begin != begin || old_end != end;
    } while (changed);
    *begin_out = begin;
    *end_out = end;
}

/* keep() of query_fixed_blocks / pick_scored_blocks: the page's whole media */
/* group, or nothing when it does not fit (an error when required).         */
static int keep_group(uint8_t *kept, uint32_t *count, uint32_t id, int required, uint32_t n, uint32_t budget,
                      uint32_t page_tokens, const uint32_t *ranges, uint32_t n_ranges) {
    if (id >= n) return ORC_ERR_ARG;
    uint32_t begin, end;
    orc_media_group(id, n, page_tokens, ranges, n_ranges, &begin, &end);
    uint32_t need = 0;
    for (uint32_t b = begin; b < end; ++b) need += !kept[b];
    if (*count + need > budget) return required ? ORC_ERR_BUDGET : ORC_OK;
    for (uint32_t b = begin; b < end; ++b)
        if (!kept[b]) { kept[b] = 1; ++*count; }
    return ORC_OK;
}

static uint32_t emit_kept(const uint8_t *kept, uint32_t n, uint32_t *out) {
    uint32_t o = 0;
    for (uint32_t i = 0; i < n; ++i)
        if (kept[i]) out[o++] = i;
    return o;
}

/* KvMemStore::query_fixed_blocks (kvmem_store.cpp:381-408): every page when */
/* the budget is 0 or covers them all; else the sink pages, the page where  */
/* the last media range starts (when it starts before total_tokens) and the */
/* mandatory pages, each with its whole media group and required to fit,    */
/* then the newest `recent` pages newest first, each kept only if it fits.  */
int orc_query_fixed_blocks(uint32_t n, uint32_t budget, uint32_t sink, uint32_t recent, const uint32_t *ranges,
                           uint32_t n_ranges, uint64_t total_tokens, uint32_t page_tokens,
                           const uint32_t *mandatory, uint32_t n_mandatory, uint32_t *out, uint32_t *n_out) {
    *n_out = 0;
    if (!page_tokens) return ORC_ERR_ARG;
    if (!budget || n <= budget) {
        for (uint32_t i = 0; i < n; ++i) out[i] = i;
        *n_out = n;
        return ORC_OK;
    }
    uint8_t *kept = (uint8_t *)calloc(n, 1);
    uint32_t count = 0;
    int st = ORC_OK;
    for (uint32_t i = 0; st == ORC_OK && i < (n < sink ? n : sink); ++i)
        st = keep_group(kept, &count, i, 1, n, budget, page_tokens, ranges, n_ranges);
    if (st == ORC_OK && n_ranges && ranges[2 * (n_ranges - 1)] < total_tokens)
        st = keep_group(kept, &count, ranges[2 * (n_ranges - 1)] / page_tokens, 1, n, budget, page_tokens, ranges,
                        n_ranges);
    for (uint32_t i = 0; st == ORC_OK && i < n_mandatory; ++i)
        st = keep_group(kept, &count, mandatory[i], 1, n, budget, page_tokens, ranges, n_ranges);
    for (uint32_t i = 0; st == ORC_OK && i < (n < recent ? n : recent); ++i)
        st = keep_group(kept, &count, n - 1 - i, 0, n, budget, page_tokens, ranges, n_ranges);
    if (st == ORC_OK) *n_out = emit_kept(kept, n, out);
    free(kept);
    return st;
}

/* KvMemStore::pick_scored_blocks (kvmem_store.cpp:418-451) with media      */
/* groups and every page a candidate (so every group is complete): the      */
/* mandatory pages' groups are required, then pages in (score desc, id by   */
/* tie rule) order each keep their whole group when it fits, else nothing.  */
int orc_pick_scored_grouped(const double *scores, uint32_t n, const uint32_t *mandatory, uint32_t n_mandatory,
                            uint32_t budget, int tie_rule, int signed_scores, const uint32_t *ranges,
                            uint32_t n_ranges, uint32_t page_tokens, uint32_t *out, uint32_t *n_out) {
    *n_out = 0;
    if (!budget || !page_tokens || (n && !scores)) return ORC_ERR_ARG;
    for (uint32_t i = 0; i < n; ++i)
        if (!isfinite(scores[i]) || (!signed_scores && scores[i] < 0)) return ORC_ERR_ARG;
    uint8_t *kept = (uint8_t *)calloc(n ? n : 1, 1);
    uint32_t count = 0;
    int st = ORC_OK;
    for (uint32_t i = 0; st == ORC_OK && i < n_mandatory; ++i)
        st = keep_group(kept, &count, mandatory[i], 1, n, budget, page_tokens, ranges, n_ranges);
    uint32_t *ids = (uint32_t *)malloc(sizeof(uint32_t) * (n ? n : 1));
    uint32_t *tmp = (uint32_t *)malloc(sizeof(uint32_t) * (n ? n : 1));
    for (uint32_t i = 0; i < n; ++i) ids[i] = i;
    rank_sort(ids, tmp, n, scores, tie_rule);
    for (uint32_t i = 0; st == ORC_OK && i < n; ++i)
        st = keep_group(kept, &count, ids[i], 0, n, budget, page_tokens, ranges, n_ranges);
    if (st == ORC_OK) *n_out = emit_kept(kept, n, out);
    free(kept); free(ids); free(tmp);
    return st;
}

/* KvMemStore::pick_topk_ungrouped (kvmem_store.cpp:578-723), TopK policy:  */
/* every page when the budget is 0 or covers them all; else, while pages    */
/* remain in the budget, the sink pages, the mandatory pages last to first  */
/* and the newest `recent` pages newest first; then the best remaining      */
/* pages by (score desc, higher id first) fill the budget.                  */
int orc_pick_topk_ungrouped(const double *scores, uint32_t n, uint32_t budget, uint32_t sink, uint32_t recent,
                            const uint32_t *mandatory, uint32_t n_mandatory, uint32_t *out, uint32_t *n_out) {
    *n_out = 0;
    if (!n) return ORC_OK;
    if (!budget || n <= budget) {
        for (uint32_t i = 0; i < n; ++i) out[i] = i;
        *n_out = n;
        return ORC_OK;
    }
    uint8_t *kept = (uint8_t *)calloc(n, 1);
    uint32_t count = 0;
#define ORC_KEEP(id) do { const uint32_t k_ = (id); if (k_ < n && !kept[k_]) { kept[k_] = 1; ++count; } } while (0)
    for (uint32_t i = 0; i < (sink < n ? sink : n) && count < budget; ++i) ORC_KEEP(i);
    for (uint32_t i = n_mandatory; i > 0 && count < budget; --i) ORC_KEEP(mandatory[i - 1]);
    for (uint32_t i = 0; i < (recent < n ? recent : n) && count < budget; ++i) ORC_KEEP(n - 1 - i);
    if (count < budget) {
        uint32_t *ids = (uint32_t *)malloc(sizeof(uint32_t) * n);
        uint32_t *tmp = (uint32_t *)malloc(sizeof(uint32_t) * n);
        uint32_t m = 0;
        for (uint32_t i = 0; i < n; ++i)
            if (!kept[i]) ids[m++] = i;
        rank_sort(ids, tmp, m, scores, ORC_TIE_HIGHER_FIRST);
        const uint32_t need = budget - count;
        for (uint32_t i = 0; i < m && i < need; ++i) ORC_KEEP(ids[i]);
        free(ids); free(tmp);
    }
#undef ORC_KEEP
    *n_out = emit_kept(kept, n, out);
    free(kept);
    return ORC_OK;
}

/* KvMemStore::constrain_media (kvmem_store.cpp:453-502) with recency off   */
/* (the pick_topk_blocks pass, :377-379): media ranges merge in list order  */
/* into page groups (a range starting before the last group's end extends   */
/* it); the sink pages and the last group are required, the mandatory pages */
/* newest first, then `selected` and then every other page, each in (score  */
/* desc, higher id first) order, keep their whole group when it fits.       */
int orc_constrain_media(const uint32_t *selected, uint32_t n_selected, const double *scores, uint32_t n,
                        uint32_t budget, uint32_t sink, const uint32_t *ranges, uint32_t n_ranges,
                        uint64_t total_tokens, uint32_t page_tokens, const uint32_t *mandatory,
                        uint32_t n_mandatory, uint32_t *out, uint32_t *n_out) {
    *n_out = 0;
    if (!page_tokens) return ORC_ERR_ARG;
    if (!n_ranges || n <= budget || budget == 0) {
        memcpy(out, selected, sizeof(uint32_t) * n_selected);
        *n_out = n_selected;
        return ORC_OK;
    }
    uint32_t *gb = (uint32_t *)malloc(sizeof(uint32_t) * (n_ranges + 1));
    uint32_t *ge = (uint32_t *)malloc(sizeof(uint32_t) * (n_ranges + 1));
    uint32_t ng = 0;
    for (uint32_t r = 0; r < n_ranges; ++r) {
        const uint32_t first_tok = ranges[2 * r], end_tok = ranges[2 * r + 1];
        if (first_tok >= total_tokens || end_tok <= first_tok) continue;
        const uint32_t first = first_tok / page_tokens;
        const uint32_t up = (end_tok + page_tokens - 1) / page_tokens;
        const uint32_t end = up < n ? up : n;
        if (ng && first < ge[ng - 1]) { if (end > ge[ng - 1]) ge[ng - 1] = end; }
        else { gb[ng] = first; ge[ng] = end; ++ng; }
    }
    uint32_t *lo = (uint32_t *)malloc(sizeof(uint32_t) * n), *hi = (uint32_t *)malloc(sizeof(uint32_t) * n);
    for (uint32_t i = 0; i < n; ++i) { lo[i] = i; hi[i] = i + 1; }
    for (uint32_t g = 0; g < ng; ++g)
        for (uint32_t i = gb[g]; i < ge[g]; ++i) { lo[i] = gb[g]; hi[i] = ge[g]; }
    uint8_t *kept = (uint8_t *)calloc(n, 1);
    uint32_t count = 0;
    int st = ORC_OK;
#define ORC_KEEP(id, required) do { const uint32_t k_ = (id); if (st == ORC_OK && k_ < n) { uint32_t need_ = 0; \
        for (uint32_t i_ = lo[k_]; i_ < hi[k_]; ++i_) need_ += !kept[i_]; \
        if (count + need_ > budget) { if (required) st = ORC_ERR_BUDGET; } \
        else { for (uint32_t i_ = lo[k_]; i_ < hi[k_]; ++i_) kept[i_] = 1; count += need_; } } } while (0)
    for (uint32_t i = 0; i < (n < sink ? n : sink); ++i) ORC_KEEP(i, 1);
    if (ng) ORC_KEEP(gb[ng - 1], 1);
    uint32_t *newest = (uint32_t *)malloc(sizeof(uint32_t) * (n_mandatory ? n_mandatory : 1));
    memcpy(newest, mandatory, sizeof(uint32_t) * n_mandatory);
    for (uint32_t i = 1; i < n_mandatory; ++i)  /* sort descending */
        for (uint32_t j = i; j > 0 && newest[j - 1] < newest[j]; --j) {
            const uint32_t t = newest[j]; newest[j] = newest[j - 1]; newest[j - 1] = t;
        }
    for (uint32_t i = 0; i < n_mandatory; ++i) ORC_KEEP(newest[i], 0);
    uint32_t *ids = (uint32_t *)malloc(sizeof(uint32_t) * (n + n_selected + 1));
    uint32_t *tmp = (uint32_t *)malloc(sizeof(uint32_t) * (n + n_selected + 1));
    memcpy(ids, selected, sizeof(uint32_t) * n_selected);
    rank_sort(ids, tmp, n_selected, scores, ORC_TIE_HIGHER_FIRST);
    for (uint32_t i = 0; i < n_selected; ++i) ORC_KEEP(ids[i], 0);
    uint32_t m = 0;
    for (uint32_t i = 0; i < n; ++i)
        if (!kept[i]) ids[m++] = i;
    rank_sort(ids, tmp, m, scores, ORC_TIE_HIGHER_FIRST);
    for (uint32_t i = 0; i < m; ++i) ORC_KEEP(ids[i], 0);
#undef ORC_KEEP
    if (st == ORC_OK) *n_out = emit_kept(kept, n, out);
    free(gb); free(ge); free(lo); free(hi); free(kept); free(newest); free(ids); free(tmp);
    return st;
}

/* ---------------------------------------------------------------------- */
/* Gather: the selected pages' token rows, ascending page order, into       */
/* consecutive slot rows: slot i holds page selected[i] at rows             */
/* [i*page_tokens, i*page_tokens + valid).  Rows past a short last page are */
/* left untouched.  write_block_to_gpu (llama-memory-kvmem.cpp:4464-4520)   */
/* addresses cell0 = slot * block_tokens and copies valid rows per plane.   */
/*   COPY          bytes unchanged (the reference product path)              */
/*   DEQUANT_F16   decode to binary32, then RNE to binary16                  */
/*   REQUANT_Q8_0  q8_0 -> binary32 -> q8_0 (quant_q8_0, stagein.cu:181-199) */
/* ---------------------------------------------------------------------- */
size_t orc_gather_row_bytes(int src_fmt, int mode, uint32_t width) {
    if (mode == ORC_GATHER_COPY) return orc_row_bytes(src_fmt, width);
    if (mode == ORC_GATHER_DEQUANT_F16) return orc_row_bytes(src_fmt, width) ? (size_t)width * 2 : 0;
    if (mode == ORC_GATHER_REQUANT_Q8_0 && src_fmt == ORC_FMT_Q8_0)
        return orc_row_bytes(ORC_FMT_Q8_0, width);
    return 0;
}

int orc_gather(const uint8_t *history, int src_fmt, uint32_t width, uint64_t tokens,
               uint32_t page_tokens, const uint32_t *selected, uint32_t k, int mode,
               uint8_t *slots) {
    const size_t srow = orc_row_bytes(src_fmt, width);
    const size_t drow = orc_gather_row_bytes(src_fmt, mode, width);
    if (!srow || !drow || !page_tokens) return ORC_ERR_ARG;
    const uint32_t pages = orc_page_count(tokens, page_tokens);
    for (uint32_t i = 0; i < k; ++i)
        if (selected[i] >= pages || (i && selected[i] <= selected[i - 1])) return ORC_ERR_ARG;
    float *row = (float *)malloc(sizeof(float) * width);
    for (uint32_t i = 0; i < k; ++i) {
        const uint64_t start = (uint64_t)selected[i] * page_tokens;
        const uint32_t n = (uint32_t)(tokens - start < page_tokens ? tokens - start : page_tokens);
        for (uint32_t t = 0; t < n; ++t) {
            const uint8_t *src = history + (start + t) * srow;
            uint8_t *dst = slots + ((size_t)i * page_tokens + t) * drow;
            if (mode == ORC_GATHER_COPY) {
                memcpy(dst, src, srow);
                continue;
            }
            decode_row(src, src_fmt, width, row);
            if (mode == ORC_GATHER_DEQUANT_F16) {
                for (uint32_t c = 0; c < width; ++c) store_u16(dst + 2 * c, orc_f32_to_f16(row[c]));
            } else {
                for (uint32_t b = 0; b < width / ORC_QK; ++b)
                    orc_quant_q8_0(row + (size_t)b * ORC_QK, dst + (size_t)b * ORC_Q8_0_BYTES);
            }
        }
    }
    free(row);
    return ORC_OK;
}

/* ---------------------------------------------------------------------- */
/* Seeded synthetic inputs.  Not a reference algorithm: the generator the   */
/* device side reproduces bit for bit (integer hashing plus correctly       */
/* rounded single operations only, no library transcendental functions).    */
/*   bits(seed, stream, c) = fmix(base(seed, stream) + (c + 1) * G)          */
/*   normal(2j), normal(2j+1): Box-Muller R cos(2 pi u2), R sin(2 pi u2),  */
/*              R = sqrt(-2 ln u1), draws 2j, 2j+1 giving u1 in (0, 1] and  */
/*              u2 in [0, 1) with 53 bits each; double from +, -, *, / only */
/*              (ln: atanh series after an exact exponent split; sqrt: six  */
/*              Newton steps; sin, cos: Taylor series after an exact        */
/*              eighth-turn reduction), rounded once to fp32.               */
/*   uniform(i): lo + u * (hi - lo) in fp32, three separate roundings.       */
/* ---------------------------------------------------------------------- */
#define SYN_G 0x9E3779B97F4A7C15ull
static uint64_t fmix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
static uint64_t synth_base(uint64_t seed, uint64_t stream) {
    return fmix64(fmix64(seed + SYN_G) ^ ((stream + 1) * 0xD1B54A32D192ED03ull));
}
uint64_t orc_synth_bits(uint64_t seed, uint64_t stream, uint64_t counter) {
    return fmix64(synth_base(seed, stream) + (counter + 1) * SYN_G);
}
static double syn_ln(double x) {  /* x in [2^-53, 1] */
    uint64_t b;
    memcpy(&b, &x, 8);
    int e = (int)((b >> 52) & 0x7ffu) - 1023;
    b = (b & 0x000fffffffffffffull) | 0x3ff0000000000000ull;
    double m;
    memcpy(&m, &b, 8);
    if (m > 1.4142135623730951) { m = m * 0.5; e += 1; }
    const double s = (m - 1.0) / (m + 1.0), s2 = s * s;
    static const double inv_odd[] = {1.0 / 21.0, 1.0 / 19.0, 1.0 / 17.0, 1.0 / 15.0, 1.0 / 13.0,
                                     1.0 / 11.0, 1.0 / 9.0,  1.0 / 7.0,  1.0 / 5.0,  1.0 / 3.0};
    double p = 1.0 / 23.0;
    for (int k = 0; k < 10; ++k) p = inv_odd[k] + s2 * p;
    const double t = s2 * p;
    return (double)e * 0.69314718055994530942 + 2.0 * (s + s * t);
}
static double syn_sqrt(double y) {  /* y >= 0 */
    if (y == 0.0) return 0.0;
    uint64_t b;
    memcpy(&b, &y, 8);
    const int e = (int)((b >> 52) & 0x7ffu) - 1023;
    /* e >> 1: arithmetic shift, floor(e / 2) for negative e as on the device */
    uint64_t rb = (uint64_t)((e >> 1) + 1023) << 52;
    double r;
    memcpy(&r, &rb, 8);
    for (int k = 0; k < 6; ++k) r = (r + y / r) * 0.5;
    return r;
}
static void syn_turn(double t, double *cs) {  /* cos and sin of 2 pi t, t in [0, 1) */
    const int q = (int)(t * 4.0);
    double r = t - (double)q * 0.25;
    const int swap = r > 0.125;
    if (swap) r = 0.25 - r;
    const double x = r * 6.28318530717958647692, x2 = x * x;
    static const double cc[] = {1.0 / 87178291200.0, 1.0 / 479001600.0, 1.0 / 3628800.0, 1.0 / 40320.0,
                                1.0 / 720.0,         1.0 / 24.0,         0.5,             1.0};
    static const double sc[] = {1.0 / 6227020800.0, 1.0 / 39916800.0, 1.0 / 362880.0, 1.0 / 5040.0,
                                1.0 / 120.0,        1.0 / 6.0,        1.0};
    double c = 1.0 / 20922789888000.0;
    for (int k = 0; k < 8; ++k) c = cc[k] - x2 * c;
    double sn = 1.0 / 1307674368000.0;
    for (int k = 0; k < 7; ++k) sn = sc[k] - x2 * sn;
    sn = x * sn;
    const double cr = swap ? sn : c, sr = swap ? c : sn;
    cs[0] = q == 0 ? cr : q == 1 ? -sr : q == 2 ? -cr : sr;
    cs[1] = q == 0 ? sr : q == 1 ? cr : q == 2 ? -sr : -cr;
}
/* normals 2j and 2j+1 */
static void normal_pair(uint64_t base, uint64_t j, double *z) {
    const uint64_t r1 = fmix64(base + (2 * j + 1) * SYN_G), r2 = fmix64(base + (2 * j + 2) * SYN_G);
    const double u1 = (double)((r1 >> 11) + 1) * 1.1102230246251565404e-16; /* 2^-53 */
    const double u2 = (double)(r2 >> 11) * 1.1102230246251565404e-16;
    const double radius = syn_sqrt(-2.0 * syn_ln(u1));
    double cs[2];
    syn_turn(u2, cs);
    z[0] = radius * cs[0];
    z[1] = radius * cs[1];
}
static double normal_from_base(uint64_t base, uint64_t index) {
    double z[2];
    normal_pair(base, index >> 1, z);
    return z[index & 1];
}
/* normals first..first+count-1 into out as binary32, a pair at a time */
static void normals_f32(uint64_t base, uint64_t first, uint64_t count, float *out) {
    double z[2];
    for (uint64_t i = 0; i < count; ++i) {
        const uint64_t k = first + i;
        if (i == 0 || (k & 1) == 0) normal_pair(base, k >> 1, z);
        out[i] = (float)z[k & 1];
    }
}
static float unit24(uint64_t r) { return (float)(r >> 40) * 5.9604644775390625e-08f; }
static float lerp_rn(float lo, float hi, float u) {
    volatile float span = hi - lo;  /* volatile: three separate roundings */
    volatile float prod = u * span;
    return lo + prod;
}
double orc_synth_normal(uint64_t seed, uint64_t stream, uint64_t index) {
    return normal_from_base(synth_base(seed, stream), index);
}
float orc_synth_uniform(uint64_t seed, uint64_t stream, uint64_t index, float lo, float hi) {
    return lerp_rn(lo, hi, unit24(orc_synth_bits(seed, stream, index)));
}
void orc_synth_normal_f16(uint64_t seed, uint64_t stream, uint64_t count, uint16_t *out) {
    const uint64_t base = synth_base(seed, stream);
    float v[256];
    for (uint64_t i0 = 0; i0 < count; i0 += 256) {
        const uint64_t n = count - i0 < 256 ? count - i0 : 256;
        normals_f32(base, i0, n, v);
        for (uint64_t i = 0; i < n; ++i) out[i0 + i] = orc_f32_to_f16(v[i]);
    }
}
void orc_synth_scaled_normal_f16(uint64_t seed, uint64_t stream, uint64_t rows,
                                 uint32_t width, const float *channel_scale, uint16_t *out) {
    const uint64_t base = synth_base(seed, stream);
    float v[256];
    const uint64_t count = rows * width;
    for (uint64_t i0 = 0; i0 < count; i0 += 256) {
        const uint64_t n = count - i0 < 256 ? count - i0 : 256;
        normals_f32(base, i0, n, v);
        for (uint64_t i = 0; i < n; ++i) {
            volatile float scaled = v[i] * channel_scale[(i0 + i) % width];
            out[i0 + i] = orc_f32_to_f16(scaled);
        }
    }
}
void orc_synth_normal_f32(uint64_t seed, uint64_t stream, uint64_t count, float *out) {
    const uint64_t base = synth_base(seed, stream);
    normals_f32(base, 0, count, out);
}
void orc_synth_uniform_f32(uint64_t seed, uint64_t stream, uint64_t count, float lo,
                           float hi, float *out) {
    for (uint64_t i = 0; i < count; ++i) out[i] = orc_synth_uniform(seed, stream, i, lo, hi);
}
/* q8_0 block b: draws 9b..9b+7 give 32 codes (16-bit chunk % 255 - 127),   */
/* draw 9b+8 gives the scale d ~ U(d_lo, d_hi) rounded to fp16.             */
void orc_synth_q8_0(uint64_t seed, uint64_t stream, uint64_t blocks, float d_lo,
                    float d_hi, uint8_t *out) {
    const uint64_t base = synth_base(seed, stream);
    for (uint64_t b = 0; b < blocks; ++b) {
        uint8_t *blk = out + b * ORC_Q8_0_BYTES;
        for (int w = 0; w < 8; ++w) {
            const uint64_t r = fmix64(base + (b * 9 + (uint64_t)w + 1) * SYN_G);
            for (int c = 0; c < 4; ++c)
                blk[2 + w * 4 + c] = (uint8_t)(int8_t)((int)((r >> (16 * c)) & 0xffffu) % 255 - 127);
        }
        const uint64_t r = fmix64(base + (b * 9 + 8 + 1) * SYN_G);
        store_u16(blk, orc_f32_to_f16(lerp_rn(d_lo, d_hi, unit24(r))));
    }
}
/* q4_1 block b: draws 4b, 4b+1 give the 16 nibble bytes, 4b+2 the scale d, */
/* 4b+3 the minimum m, each rounded to fp16.                                */
void orc_synth_q4_1(uint64_t seed, uint64_t stream, uint64_t blocks, float d_lo,
                    float d_hi, float m_lo, float m_hi, uint8_t *out) {
    const uint64_t base = synth_base(seed, stream);
    for (uint64_t b = 0; b < blocks; ++b) {
        uint8_t *blk = out + b * ORC_Q4_1_BYTES;
        for (int w = 0; w < 2; ++w) {
            const uint64_t r = fmix64(base + (b * 4 + (uint64_t)w + 1) * SYN_G);
            for (int c = 0; c < 8; ++c) blk[4 + w * 8 + c] = (uint8_t)(r >> (8 * c));
        }
        const uint64_t rd = fmix64(base + (b * 4 + 2 + 1) * SYN_G);
        const uint64_t rm = fmix64(base + (b * 4 + 3 + 1) * SYN_G);
        store_u16(blk, orc_f32_to_f16(lerp_rn(d_lo, d_hi, unit24(rd))));
        store_u16(blk + 2, orc_f32_to_f16(lerp_rn(m_lo, m_hi, unit24(rm))));
    }
}
/* q8_0 of N(0,1): values normal(32b + j) quantized with orc_quant_q8_0. */
void orc_synth_normal_q8_0(uint64_t seed, uint64_t stream, uint64_t blocks, uint8_t *out) {
    const uint64_t base = synth_base(seed, stream);
    float x[ORC_QK];
    for (uint64_t b = 0; b < blocks; ++b) {
        normals_f32(base, b * ORC_QK, ORC_QK, x);
        orc_quant_q8_0(x, out + b * ORC_Q8_0_BYTES);
    }
}

/* ---------------------------------------------------------------------- */
/* Sampled attention page masses: the dense FP64 statement the reference  */
/* checks its GPU sampler against (src/adapter/llama-kvmem-attention.cpp:  */
/* 44-96, KVMEM_ATTENTION_VERIFY): per sampled row and query head, logits  */
/* of every token with a finite mask value, scale*dot in double, optional  */
/* softcap*tanh(x/softcap), plus the mask; softmax over all tokens; the     */
/* probabilities summed per page and divided by the head count.  Key       */
/* decoding follows llama-kvmem-attention-cuda.cu:31-56 (q8_0, q4_0, q5_0   */
/* blocks; f32/f16/bf16 scalars), element products exact in binary32.      */
/* ---------------------------------------------------------------------- */
void orc_dequant_q4_0(const uint8_t *block, float *y) {
    const float d = orc_f16_to_f32(load_u16(block));
    const uint8_t *qs = block + 2;
    for (int j = 0; j < ORC_QK; ++j) {
        const int code = (qs[j % 16] >> (j < 16 ? 0 : 4)) & 15;
        y[j] = (float)(code - 8) * d;
    }
}

void orc_dequant_q5_0(const uint8_t *block, float *y) {
    const float d = orc_f16_to_f32(load_u16(block));
    const uint8_t *qh = block + 2, *qs = block + 6;
    for (int j = 0; j < ORC_QK; ++j) {
        const int low = (qs[j % 16] >> (j < 16 ? 0 : 4)) & 15;
        const int high = (qh[j / 8] >> (j % 8)) & 1;
        y[j] = (float)((low | (high << 4)) - 16) * d;
    }
}

static float attn_scalar(const uint8_t *p, int fmt, size_t i) {
    if (fmt == ORC_FMT_F32) {
        float v;
        memcpy(&v, p + 4 * i, 4);
        return v;
    }
    const uint16_t h = load_u16(p + 2 * i);
    if (fmt == ORC_FMT_F16) return orc_f16_to_f32(h);
    const uint32_t bits = (uint32_t)h << 16;
    float v;
    memcpy(&v, &bits, 4);
    return v;
}

static int attn_scalar_fmt(int fmt) { return fmt == ORC_FMT_F32 || fmt == ORC_FMT_F16 || fmt == ORC_FMT_BF16; }

static void attn_key(const uint8_t *row, int fmt, uint32_t dim, float *out) {
    for (uint32_t b = 0; b < dim / ORC_QK; ++b) {
        float *y = out + (size_t)b * ORC_QK;
        if (fmt == ORC_FMT_Q8_0) orc_dequant_q8_0(row + (size_t)b * ORC_Q8_0_BYTES, y);
        else if (fmt == ORC_FMT_Q4_0) orc_dequant_q4_0(row + (size_t)b * ORC_Q4_0_BYTES, y);
        else if (fmt == ORC_FMT_Q5_0) orc_dequant_q5_0(row + (size_t)b * ORC_Q5_0_BYTES, y);
        else
            for (uint32_t j = 0; j < ORC_QK; ++j) y[j] = attn_scalar(row, fmt, (size_t)b * ORC_QK + j);
    }
}

int orc_attention_page_mass(const uint8_t *q, int q_fmt, size_t q_row_stride, size_t q_head_stride,
                            const uint8_t *k, int k_fmt, size_t k_row_stride, size_t k_head_stride,
                            const uint8_t *mask, int mask_fmt, size_t mask_row_stride,
                            uint32_t head_dim, uint32_t query_heads, uint32_t kv_heads,
                            uint32_t tokens, uint32_t page_tokens, float scale, float softcap,
                            const uint32_t *rows, uint32_t n_rows, double *out) {
    const int key_ok = attn_scalar_fmt(k_fmt) || k_fmt == ORC_FMT_Q8_0 || k_fmt == ORC_FMT_Q4_0 ||
                       k_fmt == ORC_FMT_Q5_0;
    if (!q || !k || !mask || !rows || !out || !attn_scalar_fmt(q_fmt) || !attn_scalar_fmt(mask_fmt) || !key_ok ||
        !head_dim || head_dim % ORC_QK || !query_heads || !kv_heads || query_heads % kv_heads || !tokens ||
        !page_tokens)
        return ORC_ERR_ARG;
    const uint32_t pages = (uint32_t)(((uint64_t)tokens + page_tokens - 1) / page_tokens);
    const uint32_t group = query_heads / kv_heads;
    float *query = (float *)malloc(sizeof(float) * head_dim);
    float *key = (float *)malloc(sizeof(float) * head_dim);
    float *bias = (float *)malloc(sizeof(float) * tokens);
    double *logits = (double *)malloc(sizeof(double) * tokens);
    if (!query || !key || !bias || !logits) {
        free(query), free(key), free(bias), free(logits);
        return ORC_ERR_ARG;
    }
    for (uint32_t s = 0; s < n_rows; ++s) {
        double *expected = out + (size_t)s * pages;
        for (uint32_t p = 0; p < pages; ++p) expected[p] = 0.0;
        const uint8_t *mrow = mask + (size_t)rows[s] * mask_row_stride;
        for (uint32_t t = 0; t < tokens; ++t) bias[t] = attn_scalar(mrow, mask_fmt, t);
        for (uint32_t h = 0; h < query_heads; ++h) {
            const uint8_t *qrow = q + (size_t)rows[s] * q_row_stride + (size_t)h * q_head_stride;
            for (uint32_t d = 0; d < head_dim; ++d) query[d] = attn_scalar(qrow, q_fmt, d);
            double maximum = -INFINITY;
            for (uint32_t t = 0; t < tokens; ++t) {
                if (!isfinite(bias[t])) {
                    logits[t] = -INFINITY;
                    continue;
                }
                attn_key(k + (size_t)t * k_row_stride + (size_t)(h / group) * k_head_stride, k_fmt, head_dim, key);
                double dot = 0.0;
                for (uint32_t d = 0; d < head_dim; ++d) dot += (double)query[d] * key[d];
                dot *= scale;
                if (softcap > 0) dot = softcap * tanh(dot / softcap);
                logits[t] = dot + bias[t];
                if (logits[t] > maximum) maximum = logits[t];
            }
            double denominator = 0.0;
            for (uint32_t t = 0; t < tokens; ++t) denominator += logits[t] = exp(logits[t] - maximum);
            for (uint32_t t = 0; t < tokens; ++t) expected[t / page_tokens] += logits[t] / denominator / query_heads;
        }
    }
    free(query), free(key), free(bias), free(logits);
    return ORC_OK;
}

/* ---------------------------------------------------------------------- */
/* Raw-K stage-in transform (kvmem_stagein_enqueue_k + flush,              */
/* src/adapter/llama-kvmem-stagein.cu:105-234, 746-783, 817-858): decode   */
/* q8_0/q4_0, NeoX RoPE at each token's position, Walsh-Hadamard over runs */
/* of `fwht` values (scaled by 1/sqrt(fwht) first, butterflies in the      */
/* reference's loop order), requantize to the source format.               */
/* ---------------------------------------------------------------------- */

/* sin and cos of a binary32 angle, each rounded once from a binary64
 * evaluation: reduction by the nearest multiple k of pi/2 (Cody-Waite, two
 * binary64 parts, fused), Taylor polynomials of degree 21 / 20 on
 * |r| <= pi/4, quadrant k mod 4.  The device runs the same operations
 * (within 1 ulp of the reference's sincosf, which is not reproducible on
 * another machine). */
void orc_rope_sincos(float angle, float *s, float *c) {
    const double x = angle;
    const double k = rint(x * 0.6366197723675814);
    double r = fma(-k, 1.5707963267948966, x);
    r = fma(-k, 6.123233995736766e-17, r);
    const double r2 = r * r;
    double ps = 1.9572941063391263e-20;
    ps = fma(ps, r2, -8.22063524662433e-18);
    ps = fma(ps, r2, 2.8114572543455206e-15);
    ps = fma(ps, r2, -7.647163731819816e-13);
    ps = fma(ps, r2, 1.6059043836821613e-10);
    ps = fma(ps, r2, -2.505210838544172e-08);
    ps = fma(ps, r2, 2.7557319223985893e-06);
    ps = fma(ps, r2, -0.0001984126984126984);
    ps = fma(ps, r2, 0.008333333333333333);
    ps = fma(ps, r2, -0.16666666666666666);
    const double sr = fma(r * r2, ps, r);
    double pc = 4.110317623312165e-19;
    pc = fma(pc, r2, -1.5619206968586225e-16);
    pc = fma(pc, r2, 4.779477332387385e-14);
    pc = fma(pc, r2, -1.1470745597729725e-11);
    pc = fma(pc, r2, 2.08767569878681e-09);
    pc = fma(pc, r2, -2.755731922398589e-07);
    pc = fma(pc, r2, 2.48015873015873e-05);
    pc = fma(pc, r2, -0.001388888888888889);
    pc = fma(pc, r2, 0.041666666666666664);
    pc = fma(pc, r2, -0.5);
    const double cr = fma(r2, pc, 1.0);
    const unsigned q = (unsigned)((int64_t)k) & 3u;
    *s = (float)(q == 0 ? sr : q == 1 ? cr : q == 2 ? -sr : -cr);
    *c = (float)(q == 0 ? cr : q == 1 ? -sr : q == 2 ? -cr : sr);
}

/* quant_q4_0 (stagein.cu:201-234); the reference's x*id + 8.5 is taken as
 * one fused multiply-add (a CUDA compiler contracts it by default). */
void orc_quant_q4_0(const float *x, uint8_t *block) {
    float amax = 0.0f, vmax = 0.0f;
    for (int j = 0; j < ORC_QK; ++j)
        if (amax < fabsf(x[j])) {
            amax = fabsf(x[j]);
            vmax = x[j];
        }
    const float d = vmax / -8.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    store_u16(block, orc_f32_to_f16(d));
    for (int j = 0; j < ORC_QK / 2; ++j) {
        int x0 = (int)fmaf(x[j], id, 8.5f), x1 = (int)fmaf(x[j + ORC_QK / 2], id, 8.5f);
        if (x0 > 15) x0 = 15;
        if (x1 > 15) x1 = 15;
        block[2 + j] = (uint8_t)((x0 & 15) | ((x1 & 15) << 4));
    }
}

/* NeoX rotation of one token row (rope_neox_kernel, stagein.cu:160-178):
 * in each head, (i, i + n_rot/2) by pos*theta[i]; x0*c - x1*s and
 * x0*s + x1*c with the first product fused. */
void orc_rope_neox_row(float *row, uint32_t width, uint32_t head_dim, uint32_t n_rot, const float *theta,
                       float pos) {
    const uint32_t half = n_rot / 2;
    for (uint32_t h = 0; h < width / head_dim; ++h) {
        float *x = row + (size_t)h * head_dim;
        for (uint32_t i = 0; i < half; ++i) {
            float s, c;
            orc_rope_sincos(pos * theta[i], &s, &c);
            const float x0 = x[i], x1 = x[i + half];
            x[i] = fmaf(x0, c, -(x1 * s));
            x[i + half] = fmaf(x0, s, x1 * c);
        }
    }
}

/* fwht_kernel (stagein.cu:105-130) on each run of n values of a row. */
void orc_fwht_row(float *row, uint32_t width, uint32_t n) {
    const float scale = 1.0f / sqrtf((float)n);
    for (uint32_t g = 0; g < width / n; ++g) {
        float *t = row + (size_t)g * n;
        for (uint32_t i = 0; i < n; ++i) t[i] = t[i] * scale;
        for (uint32_t h = 1; h < n; h *= 2)
            for (uint32_t i = 0; i < n; i += 2 * h)
                for (uint32_t j = 0; j < h; ++j) {
                    const float a = t[i + j], b = t[i + j + h];
                    t[i + j] = a + b;
                    t[i + j + h] = a - b;
                }
    }
}

/* Variants of the transform's floating-point choices, for the sensitivity
 * tests only (variant 0 is the transform itself):
 *   ORC_VAR_UNFUSED_ROT   x0*c - x1*s and x0*s + x1*c with every product
 *                         and the sum rounded separately
 *   ORC_VAR_UNFUSED_Q4    q4_0's x*id + 8.5 rounded twice
 *   ORC_VAR_SIN_UP/_DOWN, ORC_VAR_COS_UP/_DOWN
 *                         sin or cos one binary32 ulp away (toward +/-inf)
 *   ORC_VAR_RNE           q8_0 codes rint(x*id), q4_0 codes rint(x*id) + 8:
 *                         ties to even instead of the reference's rules */
static void quant_q8_0_var(const float *x, uint8_t *block, int variant) {
    if (!(variant & ORC_VAR_RNE)) {
        orc_quant_q8_0(x, block);
        return;
    }
    float amax = 0.0f;
    for (int j = 0; j < ORC_QK; ++j) amax = fmaxf(amax, fabsf(x[j]));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    store_u16(block, orc_f32_to_f16(d));
    int8_t *qs = (int8_t *)(block + 2);
    for (int j = 0; j < ORC_QK; ++j) qs[j] = (int8_t)rintf(x[j] * id);
}

static void quant_q4_0_var(const float *x, uint8_t *block, int variant) {
    if (!(variant & (ORC_VAR_UNFUSED_Q4 | ORC_VAR_RNE))) {
        orc_quant_q4_0(x, block);
        return;
    }
    float amax = 0.0f, vmax = 0.0f;
    for (int j = 0; j < ORC_QK; ++j)
        if (amax < fabsf(x[j])) {
            amax = fabsf(x[j]);
            vmax = x[j];
        }
    const float d = vmax / -8.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    store_u16(block, orc_f32_to_f16(d));
    for (int j = 0; j < ORC_QK / 2; ++j) {
        int q[2];
        for (int h = 0; h < 2; ++h) {
            const float p = x[j + h * ORC_QK / 2] * id;
            q[h] = variant & ORC_VAR_RNE ? (int)rintf(p) + 8 : (int)(p + 8.5f);
            if (q[h] > 15) q[h] = 15;
        }
        block[2 + j] = (uint8_t)((q[0] & 15) | ((q[1] & 15) << 4));
    }
}

static void rope_row_var(float *row, uint32_t width, uint32_t head_dim, uint32_t n_rot, const float *theta,
                         float pos, int variant) {
    if (!(variant & (ORC_VAR_UNFUSED_ROT | ORC_VAR_SIN_UP | ORC_VAR_SIN_DOWN | ORC_VAR_COS_UP | ORC_VAR_COS_DOWN))) {
        orc_rope_neox_row(row, width, head_dim, n_rot, theta, pos);
        return;
    }
    const uint32_t half = n_rot / 2;
    for (uint32_t h = 0; h < width / head_dim; ++h) {
        float *x = row + (size_t)h * head_dim;
        for (uint32_t i = 0; i < half; ++i) {
            float s, c;
            orc_rope_sincos(pos * theta[i], &s, &c);
            if (variant & ORC_VAR_SIN_UP) s = nextafterf(s, INFINITY);
            if (variant & ORC_VAR_SIN_DOWN) s = nextafterf(s, -INFINITY);
            if (variant & ORC_VAR_COS_UP) c = nextafterf(c, INFINITY);
            if (variant & ORC_VAR_COS_DOWN) c = nextafterf(c, -INFINITY);
            const float x0 = x[i], x1 = x[i + half];
            if (variant & ORC_VAR_UNFUSED_ROT) {
                const float a = x0 * c, b = x1 * s, e = x0 * s, f = x1 * c;
                x[i] = a - b;
                x[i + half] = e + f;
            } else {
                x[i] = fmaf(x0, c, -(x1 * s));
                x[i + half] = fmaf(x0, s, x1 * c);
            }
        }
    }
}

int orc_rope_fwht_rows_variant(const uint8_t *rows, int fmt, uint32_t width, uint32_t n, int64_t pos0,
                               uint32_t head_dim, uint32_t n_rot, const float *theta, uint32_t fwht, int variant,
                               uint8_t *out) {
    if ((fmt != ORC_FMT_Q8_0 && fmt != ORC_FMT_Q4_0) || !width || width % ORC_QK || !head_dim ||
        width % head_dim || n_rot % 2 || n_rot > head_dim || (n_rot && !theta) ||
        (fwht && (width % fwht || (fwht != 64 && fwht != 128 && fwht != 256 && fwht != 512))))
        return ORC_ERR_ARG;
    const uint32_t bb = fmt == ORC_FMT_Q8_0 ? ORC_Q8_0_BYTES : ORC_Q4_0_BYTES, bpr = width / ORC_QK;
    float *row = (float *)malloc(sizeof(float) * width);
    if (!row) return ORC_ERR_ARG;
    for (uint32_t t = 0; t < n; ++t) {
        const uint8_t *in = rows + (size_t)t * bpr * bb;
        uint8_t *o = out + (size_t)t * bpr * bb;
        for (uint32_t b = 0; b < bpr; ++b) {
            if (fmt == ORC_FMT_Q8_0) orc_dequant_q8_0(in + (size_t)b * bb, row + (size_t)b * ORC_QK);
            else orc_dequant_q4_0(in + (size_t)b * bb, row + (size_t)b * ORC_QK);
        }
        rope_row_var(row, width, head_dim, n_rot, theta, (float)(pos0 + t), variant);
        if (fwht) orc_fwht_row(row, width, fwht);
        for (uint32_t b = 0; b < bpr; ++b) {
            if (fmt == ORC_FMT_Q8_0) quant_q8_0_var(row + (size_t)b * ORC_QK, o + (size_t)b * bb, variant);
            else quant_q4_0_var(row + (size_t)b * ORC_QK, o + (size_t)b * bb, variant);
        }
    }
    free(row);
    return ORC_OK;
}

int orc_rope_fwht_rows(const uint8_t *rows, int fmt, uint32_t width, uint32_t n, int64_t pos0,
                       uint32_t head_dim, uint32_t n_rot, const float *theta, uint32_t fwht, uint8_t *out) {
    return orc_rope_fwht_rows_variant(rows, fmt, width, n, pos0, head_dim, n_rot, theta, fwht, 0, out);
}

/* The gather with the raw-K transform: slot s of the selection holds page
 * selected[s]'s rows transformed at their positions pos_base + t. */
int orc_gather_rope(const uint8_t *history, int fmt, uint32_t width, uint64_t tokens, uint32_t page_tokens,
                    const uint32_t *selected, uint32_t k, uint32_t head_dim, uint32_t n_rot,
                    const float *theta, uint32_t fwht, int64_t pos_base, uint8_t *slots) {
    const uint32_t bb = fmt == ORC_FMT_Q8_0 ? ORC_Q8_0_BYTES : ORC_Q4_0_BYTES;
    const size_t row = (size_t)width / ORC_QK * bb;
    for (uint32_t s = 0; s < k; ++s) {
        const uint64_t first = (uint64_t)selected[s] * page_tokens;
        if (first >= tokens) continue;
        const uint32_t valid = (uint32_t)(tokens - first < page_tokens ? tokens - first : page_tokens);
        const int rc = orc_rope_fwht_rows(history + first * row, fmt, width, valid, pos_base + (int64_t)first,
                                          head_dim, n_rot, theta, fwht, slots + (size_t)s * page_tokens * row);
        if (rc) return rc;
    }
    return ORC_OK;
}

/* ---------------------------------------------------------------------- */
/* Graph propagation and LRFU                                              */
/* ---------------------------------------------------------------------- */
/* span_coefficient (graph_recall.cpp:234-247) of pages i and i+1: 1 when one
 * span holds both, the cross weight when a span boundary falls inside the
 * pair, else 1. */
int orc_span_coefficients(const uint64_t *span_begin, const uint64_t *span_end,
                          const uint8_t *end_known, uint32_t n_spans, uint32_t block_tokens,
                          uint32_t pages, double cross, double *out) {
    if (!block_tokens || !(cross >= 0 && cross <= 1)) return ORC_ERR_ARG;
    for (uint32_t i = 0; i + 1 < pages; ++i) {
        const uint64_t begin = (uint64_t)i * block_tokens;
        const uint64_t end = (uint64_t)(i + 1) * block_tokens + block_tokens;
        double c = 1;
        int inside = 0;
        for (uint32_t s = 0; s < n_spans && !inside; ++s)
            inside = span_begin[s] <= begin && end <= span_end[s];
        if (!inside)
            for (uint32_t s = 0; s < n_spans; ++s)
                if ((begin < span_begin[s] && span_begin[s] < end) ||
                    (end_known[s] && begin < span_end[s] && span_end[s] < end)) {
                    c = cross;
                    break;
                }
        out[i] = c;
    }
    return ORC_OK;
}

/* propagate_query_scores (graph_recall.cpp:494-552): positive evidence moves
 * one hop, alpha/4 to each adjacent node (:522-531) and alpha/2 over the
 * source's graph row in proportion to its edge masses among nodes (:532-545);
 * negative scores stay at their page (:547-551). */
int orc_propagate_scores(const double *raw, const uint8_t *mask, uint32_t n, uint32_t n_rows,
                         const uint32_t *row_source, const uint32_t *row_begin,
                         const uint32_t *edge_target, const double *edge_mass,
                         const double *neighbor_weight, double alpha, double *out) {
#define NODE(j) ((j) < n && (!mask || mask[j]))
    if (!(alpha >= 0 && alpha <= 1)) return ORC_ERR_ARG;
    double total = 0;
    uint32_t nodes = 0;
    for (uint32_t i = 0; i < n; ++i) {
        if (!isfinite(raw[i])) return ORC_ERR_NONFINITE;
        if (NODE(i)) {
            ++nodes;
            total += 0. < raw[i] ? raw[i] : 0.;
        }
    }
    if (!isfinite(total)) return ORC_ERR_NONFINITE;
    memcpy(out, raw, sizeof(double) * n);
    if (nodes <= 1 || total == 0 || alpha == 0) return ORC_OK;
    double *seed = (double *)calloc(n, sizeof(double));
    for (uint32_t i = 0; i < n; ++i)
        if (NODE(i)) seed[i] = (0. < raw[i] ? raw[i] : 0.) / total;
    int rc = ORC_OK;
    for (uint32_t i = 0; i < n && rc == ORC_OK; ++i) {
        if (!NODE(i)) continue;
        for (int dir = -1; dir <= 1; dir += 2) {
            if (dir < 0 && i == 0) continue;
            const uint32_t j = dir < 0 ? i - 1 : i + 1;
            if (!NODE(j)) continue;
            const double c = neighbor_weight ? neighbor_weight[dir < 0 ? j : i] : 1.;
            if (!(c >= 0 && c <= 1)) { rc = ORC_ERR_ARG; break; }
            const double delta = total * seed[i] * (alpha * .25 * c);
            out[i] -= delta;
            out[j] += delta;
        }
    }
    for (uint32_t r = 0; r < n_rows && rc == ORC_OK; ++r) {
        const uint32_t src = row_source[r], e0 = row_begin[r], e1 = row_begin[r + 1];
        if (e0 > e1) { rc = ORC_ERR_ARG; break; }
        if (!NODE(src)) continue;
        double den = 0;
        for (uint32_t e = e0; e < e1; ++e) {
            if (!(isfinite(edge_mass[e]) && edge_mass[e] >= 0)) { rc = ORC_ERR_ARG; break; }
            if (edge_target[e] != src && NODE(edge_target[e])) den += edge_mass[e];
        }
        if (rc != ORC_OK || !den) continue;
        for (uint32_t e = e0; e < e1; ++e) {
            const uint32_t t = edge_target[e];
            if (t == src || !NODE(t)) continue;
            const double delta = total * seed[src] * (alpha * .5 * edge_mass[e] / den);
            out[src] -= delta;
            out[t] += delta;
        }
    }
    free(seed);
    if (rc != ORC_OK) return rc;
    const double slack = 1e-12 * (1. < total ? total : 1.);
    for (uint32_t i = 0; i < n; ++i) {
        const double resid = raw[i] < 0. ? raw[i] : 0.;
        if (!(isfinite(out[i]) && out[i] >= resid - slack)) return ORC_ERR_ARG;
        out[i] = resid < out[i] ? out[i] : resid;
    }
    return ORC_OK;
#undef NODE
}

static int cmp_double(const void *a, const void *b) {
    const double x = *(const double *)a, y = *(const double *)b;
    return x < y ? -1 : (y < x ? 1 : 0);
}

/* LrfuHistory::preview (lrfu.hpp:57-79): the threshold is the score of
 * ascending rank min(n-1, floor((1-fraction)*n)) (nth_element); scores below
 * it keep only their negative part. */
int orc_lrfu_preview(const double *scores, uint32_t n, const double *history, uint32_t n_history,
                     double lambda, double top_fraction, double *out) {
    if (!(lambda >= 0 && lambda <= 1) || !(top_fraction > 0 && top_fraction <= 1)) return ORC_ERR_ARG;
    for (uint32_t i = 0; i < n; ++i)
        if (!isfinite(scores[i])) return ORC_ERR_NONFINITE;
    if (!n) return ORC_OK;
    double threshold = -INFINITY;
    if (top_fraction < 1) {
        double *ranked = (double *)malloc(sizeof(double) * n);
        memcpy(ranked, scores, sizeof(double) * n);
        qsort(ranked, n, sizeof(double), cmp_double);
        const double r = (1 - top_fraction) * (double)n;
        const size_t rank = (size_t)r < n - 1 ? (size_t)r : n - 1;
        threshold = ranked[rank];
        free(ranked);
    }
    for (uint32_t i = 0; i < n; ++i) {
        const double h = i < n_history ? history[i] : 0;
        const double s = scores[i];
        out[i] = lambda * h + (s >= threshold ? s : (0. < s ? 0. : s));
    }
    return ORC_OK;
}
