/*
 * kvr_oracle.h -- CPU restatement of KVMem's recall hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links, loads or
 * calls this code.  It is the checker that tests/, the smoke entry point and
 * the CPU-baseline leg of the benchmark compare the HIP path against.
 *
 * Plain C99, single-threaded, double accumulation exactly where the reference
 * uses double.  Every function names the reference file:line it restates
 * (paths relative to the KVMem 0.19.0 source tree).
 *
 * Parity pinning (what checks each function, besides the reference build in
 * oracle/_ref when that is present):
 *   orc_f32_to_f16 / orc_f16_to_f32  exhaustive fp16 round trip + RNE midpoints
 *   orc_recall_fp16                  graph_recall_test.cpp:57-61 known answers
 *   orc_query_score_frame            graph_recall_test.cpp:23-31 known answers
 *   orc_page_summary_*               sequential-sum closed form (integers, exact)
 *   orc_page_softmax_scores (Mean)   graph_recall_test.cpp:22-56, 63-84 closed forms
 *   orc_page_softmax_scores (Max)    graph_recall_test.cpp:85-96 closed form
 *   orc_page_softmax_scores (MaxLogit, the literal max-of-logits variant)
 *                                    closed form on a two-page example
 *   orc_pick_scored_blocks           brute force on tiny inputs +
 *                                    layerwise_selection_test.cpp:184-194 ties
 *   orc_layerwise_fold               layerwise_selection_test.cpp:104-160
 *                                    known answers (short evidence kept by
 *                                    half pages; strongest half after the
 *                                    whole Query); the reference's own
 *                                    layerwise_tile_scores in oracle/_ref
 *   orc_media_group / orc_query_fixed_blocks / orc_pick_scored_grouped /
 *   orc_pick_topk_ungrouped / orc_constrain_media
 *                                    the reference's own KvMemStore
 *                                    (query_fixed_blocks, pick_scored_blocks,
 *                                    pick_topk_blocks) in oracle/_ref on random
 *                                    stores with media ranges; kvmem_store_test
 *                                    known answers; brute-force subset search
 *                                    on tiny grouped inputs
 *   orc_dequant_q8_0 / orc_quant_q8_0 exact-product closed form, stagein.cu formulas
 *   orc_dequant_q4_1                 closed form y = nib*d + m (ggml q4_1 layout;
 *                                    no reference test holds q4_1 bytes)
 *   orc_dequant_q4_0 / q5_0          hand-built blocks with known codes (the
 *                                    layouts of llama-kvmem-attention-cuda.cu:31-56)
 *   orc_rope_sincos                  numpy sin/cos of the binary32 angle (within
 *                                    1 ulp; the device runs the same operations)
 *   orc_rope_neox_row / orc_fwht_row the rotation's closed form (pair norms,
 *                                    angle 0 is the identity, a rotation and its
 *                                    inverse); Walsh-Hadamard applied twice is
 *                                    the identity, a unit vector gives a
 *                                    Hadamard row
 *   orc_quant_q4_0 / orc_rope_fwht_rows  hand-built blocks; the transform with
 *                                    no rotation and no Walsh-Hadamard returns
 *                                    blocks whose extreme code is full scale
 *   orc_attention_page_mass          closed forms (uniform logits -> token
 *                                    shares, two-token logistic, softcap tanh,
 *                                    masked tokens and pages, mass sums to 1)
 *                                    and a per-page log-sum-exp restatement
 *                                    computed independently in the tests
 *   orc_span_coefficients /          graph_recall_test.cpp:109-131 (graph
 *   orc_propagate_scores             lifecycle), :167-188 (explicit transport
 *                                    matrix, alpha 0, negative scores, masked
 *                                    node, NaN/inf rejected), :311-322
 *                                    (message locality) known answers; mass
 *                                    conservation; a dense transport-matrix
 *                                    restatement in the tests
 *   orc_lrfu_preview                 kvmem_store_test.cpp:1176-1206 known
 *                                    answers; the gate by a sorted rank
 *   orc_synth_*                      not a reference algorithm: the shared
 *                                    seeded input generator (moments checked)
 */
#ifndef KVR_ORACLE_H
#define KVR_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    ORC_OK = 0,
    ORC_ERR_ARG = 1,       /* invalid geometry or argument            */
    ORC_ERR_NONFINITE = 2, /* recall operand is NaN or infinite        */
    ORC_ERR_RANGE = 3,     /* recall operand rounds to fp16 infinity   */
    ORC_ERR_BUDGET = 4     /* mandatory pages exceed the budget        */
};

enum { ORC_AGG_MEAN = 0, ORC_AGG_MAX = 1, ORC_AGG_MAX_LOGIT = 2 };
enum { ORC_TIE_LOWER_FIRST = 0, ORC_TIE_HIGHER_FIRST = 1 };

/* History formats: token-major rows of `width` channels.  F32 and BF16 are
 * query/mask scalars and attention key formats; Q4_0 and Q5_0 attention key
 * formats only (same values as the library's kvr_format). */
enum { ORC_FMT_F16 = 0, ORC_FMT_Q8_0 = 1, ORC_FMT_Q4_1 = 2, ORC_FMT_F32 = 3, ORC_FMT_BF16 = 4,
       ORC_FMT_Q4_0 = 5, ORC_FMT_Q5_0 = 6 };
/* Gather modes. */
enum { ORC_GATHER_COPY = 0, ORC_GATHER_DEQUANT_F16 = 1, ORC_GATHER_REQUANT_Q8_0 = 2 };

#define ORC_QK 32
#define ORC_Q8_0_BYTES 34 /* {fp16 d; int8 qs[32]}            */
#define ORC_Q4_1_BYTES 20 /* {fp16 d; fp16 m; uint8 qs[16]}   */
#define ORC_Q4_0_BYTES 18 /* {fp16 d; uint8 qs[16]}           */
#define ORC_Q5_0_BYTES 22 /* {fp16 d; uint8 qh[4]; uint8 qs[16]} */

/* ---- scalar conversions ------------------------------------------------ */
uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);
int orc_recall_fp16(float value, float *out);

/* ---- frame -------------------------------------------------------------- */
uint32_t orc_page_count(uint64_t accepted, uint32_t block_tokens);
int orc_query_score_frame(uint64_t accepted, uint32_t block_tokens, uint32_t budget,
                          uint32_t sink, uint32_t recent, const uint32_t *fixed,
                          uint32_t n_fixed, uint64_t *starts, uint32_t *counts,
                          uint8_t *score_mask, uint8_t *transport_mask);

/* ---- page summaries (mean-K) ------------------------------------------- */
size_t orc_row_bytes(int fmt, uint32_t width);
int orc_page_summaries(const void *keys, int fmt, uint64_t tokens, uint32_t width,
                       uint32_t page_tokens, float *sums, float *means);

/* ---- scoring ----------------------------------------------------------- */
int orc_page_softmax_scores(const float *means, const float *query,
                            const uint32_t *layer_rows, uint32_t layers, uint32_t rows,
                            uint32_t query_heads, uint32_t kv_heads, uint32_t head_dim,
                            uint32_t pages, const uint8_t *score_mask,
                            float attention_scale, int aggregation, double *out);
int orc_page_logits(const float *means, const float *query, uint32_t rows,
                    uint32_t query_heads, uint32_t kv_heads, uint32_t head_dim,
                    uint32_t pages, float attention_scale, double *logits);

/* ---- selection ---------------------------------------------------------- */
int orc_pick_scored_blocks(const double *scores, uint32_t n, const uint32_t *mandatory,
                           uint32_t n_mandatory, uint32_t budget, int tie_rule,
                           int signed_scores, uint32_t *out, uint32_t *n_out);

int orc_layerwise_fold(const double *mass, uint32_t count, const uint8_t *score_mask, int keep_halves,
                       double *out);
void orc_media_group(uint32_t id, uint32_t n, uint32_t page_tokens, const uint32_t *ranges,
                     uint32_t n_ranges, uint32_t *begin, uint32_t *end);
int orc_query_fixed_blocks(uint32_t n, uint32_t budget, uint32_t sink, uint32_t recent, const uint32_t *ranges,
                           uint32_t n_ranges, uint64_t total_tokens, uint32_t page_tokens,
                           const uint32_t *mandatory, uint32_t n_mandatory, uint32_t *out, uint32_t *n_out);
int orc_pick_scored_grouped(const double *scores, uint32_t n, const uint32_t *mandatory, uint32_t n_mandatory,
                            uint32_t budget, int tie_rule, int signed_scores, const uint32_t *ranges,
                            uint32_t n_ranges, uint32_t page_tokens, uint32_t *out, uint32_t *n_out);
int orc_pick_topk_ungrouped(const double *scores, uint32_t n, uint32_t budget, uint32_t sink, uint32_t recent,
                            const uint32_t *mandatory, uint32_t n_mandatory, uint32_t *out, uint32_t *n_out);
int orc_constrain_media(const uint32_t *selected, uint32_t n_selected, const double *scores, uint32_t n,
                        uint32_t budget, uint32_t sink, const uint32_t *ranges, uint32_t n_ranges,
                        uint64_t total_tokens, uint32_t page_tokens, const uint32_t *mandatory,
                        uint32_t n_mandatory, uint32_t *out, uint32_t *n_out);

/* ---- block formats ------------------------------------------------------ */
void orc_dequant_q8_0(const uint8_t *block, float *y);
void orc_dequant_q4_1(const uint8_t *block, float *y);
void orc_quant_q8_0(const float *x, uint8_t *block);
void orc_dequant_q4_0(const uint8_t *block, float *y);
void orc_dequant_q5_0(const uint8_t *block, float *y);
void orc_quant_q4_0(const float *x, uint8_t *block);

/* ---- raw-K stage-in transform ------------------------------------------- */
void orc_rope_sincos(float angle, float *s, float *c);
void orc_rope_neox_row(float *row, uint32_t width, uint32_t head_dim, uint32_t n_rot, const float *theta,
                       float pos);
void orc_fwht_row(float *row, uint32_t width, uint32_t n);
int orc_rope_fwht_rows(const uint8_t *rows, int fmt, uint32_t width, uint32_t n, int64_t pos0,
                       uint32_t head_dim, uint32_t n_rot, const float *theta, uint32_t fwht, uint8_t *out);
/* The same with other floating-point choices (sensitivity tests only; a
 * bit set of ORC_VAR_*; 0 is orc_rope_fwht_rows). */
enum {
    ORC_VAR_UNFUSED_ROT = 1, ORC_VAR_UNFUSED_Q4 = 2, ORC_VAR_SIN_UP = 4, ORC_VAR_SIN_DOWN = 8,
    ORC_VAR_COS_UP = 16, ORC_VAR_COS_DOWN = 32, ORC_VAR_RNE = 64
};
int orc_rope_fwht_rows_variant(const uint8_t *rows, int fmt, uint32_t width, uint32_t n, int64_t pos0,
                               uint32_t head_dim, uint32_t n_rot, const float *theta, uint32_t fwht, int variant,
                               uint8_t *out);
int orc_gather_rope(const uint8_t *history, int fmt, uint32_t width, uint64_t tokens, uint32_t page_tokens,
                    const uint32_t *selected, uint32_t k, uint32_t head_dim, uint32_t n_rot,
                    const float *theta, uint32_t fwht, int64_t pos_base, uint8_t *slots);

/* ---- sampled attention (attention-feedback observer) ------------------ */
/* out: double [n_rows][ceil(tokens/page_tokens)].  Operands are host copies
 * of the device layouts (byte strides as in kvr_attention_sample). */
int orc_attention_page_mass(const uint8_t *q, int q_fmt, size_t q_row_stride, size_t q_head_stride,
                            const uint8_t *k, int k_fmt, size_t k_row_stride, size_t k_head_stride,
                            const uint8_t *mask, int mask_fmt, size_t mask_row_stride,
                            uint32_t head_dim, uint32_t query_heads, uint32_t kv_heads,
                            uint32_t tokens, uint32_t page_tokens, float scale, float softcap,
                            const uint32_t *rows, uint32_t n_rows, double *out);

/* ---- gather ------------------------------------------------------------- */
size_t orc_gather_row_bytes(int src_fmt, int mode, uint32_t width);
int orc_gather(const uint8_t *history, int src_fmt, uint32_t width, uint64_t tokens,
               uint32_t page_tokens, const uint32_t *selected, uint32_t k, int mode,
               uint8_t *slots);

/* ---- graph propagation and LRFU ------------------------------------------ */
/* Span coefficient of each adjacent page pair (i, i+1), i < pages-1, for
 * message spans [begin, end) (end_known[s] 0: an open span); no spans: 1.
 * span_coefficient, graph_recall.cpp:234-247. */
int orc_span_coefficients(const uint64_t *span_begin, const uint64_t *span_end,
                          const uint8_t *end_known, uint32_t n_spans, uint32_t block_tokens,
                          uint32_t pages, double cross, double *out);
/* propagate_query_scores (graph_recall.cpp:494-552) for a frame whose page i
 * starts at token i*block_tokens: mask = transport_mask (NULL: all), graph
 * rows flattened by page (row_source, row_begin, edge_target, edge_mass),
 * neighbor_weight[i] the coefficient of pages (i, i+1) (NULL: 1).  The
 * transfers run in ascending page order (the reference's follow its hash
 * map's iteration order). */
int orc_propagate_scores(const double *raw, const uint8_t *mask, uint32_t n, uint32_t n_rows,
                         const uint32_t *row_source, const uint32_t *row_begin,
                         const uint32_t *edge_target, const double *edge_mass,
                         const double *neighbor_weight, double alpha, double *out);
/* LrfuHistory::preview (kvmem/include/kvmem/lrfu.hpp:57-79): the candidate
 * lambda*history + gated scores. */
int orc_lrfu_preview(const double *scores, uint32_t n, const double *history, uint32_t n_history,
                     double lambda, double top_fraction, double *out);

/* ---- seeded synthetic inputs (shared with the device generator) ------- */
uint64_t orc_synth_bits(uint64_t seed, uint64_t stream, uint64_t counter);
double orc_synth_normal(uint64_t seed, uint64_t stream, uint64_t index);
float orc_synth_uniform(uint64_t seed, uint64_t stream, uint64_t index, float lo, float hi);
void orc_synth_normal_f16(uint64_t seed, uint64_t stream, uint64_t count, uint16_t *out);
void orc_synth_scaled_normal_f16(uint64_t seed, uint64_t stream, uint64_t rows,
                                 uint32_t width, const float *channel_scale, uint16_t *out);
void orc_synth_normal_f32(uint64_t seed, uint64_t stream, uint64_t count, float *out);
void orc_synth_uniform_f32(uint64_t seed, uint64_t stream, uint64_t count, float lo,
                           float hi, float *out);
void orc_synth_q8_0(uint64_t seed, uint64_t stream, uint64_t blocks, float d_lo,
                    float d_hi, uint8_t *out);
void orc_synth_q4_1(uint64_t seed, uint64_t stream, uint64_t blocks, float d_lo,
                    float d_hi, float m_lo, float m_hi, uint8_t *out);
void orc_synth_normal_q8_0(uint64_t seed, uint64_t stream, uint64_t blocks, uint8_t *out);

#ifdef __cplusplus
}
#endif
#endif
