// kvr_attention.hip -- sampled attention page masses for gfx950: the
// attention-feedback observer of src/adapter/llama-kvmem-attention-cuda.cu.
//
// For each sampled query row r and query head h the reference takes the
// softmax of scale*q.k (soft-capped, plus the additive mask) over all key
// tokens, sums it per page and averages over heads (the dense FP64 check at
// src/adapter/llama-kvmem-attention.cpp:44-96 states the same result).  It
// gets there through per-page log-sum-exps (page_lse, .cu:59-98), a
// per-(row, head) max and 1/sum over pages (normalize, .cu:99-115) and the
// head average (average, .cu:116-126).
//
// Here the first step reads every key once: a workgroup owns a group of up
// to 16 pages of one kv-head and every (sampled row, query head of the
// group) pair of a 16-pair tile.  Its four waves stream the pages' 16-token
// tiles through a two-slot ring of loads and multiply them with the pair
// tile's queries on the matrix cores (fp16 keys and, staged through a
// per-wave LDS tile, q8_0 keys on v_mfma_f32_16x16x32_f16 with split
// hi/lo queries; the other formats decoded to binary32 on
// v_mfma_f32_16x16x4f32), keep each tile's logits and reduce them to
// per-page log-sum-exps.  The second kernel does the normalization and the
// head average of one sampled row per workgroup row.  Arithmetic is
// binary32 with binary32 accumulation, as in the reference.
#include "kvr_device.hpp"
#include "kvr_internal.hpp"

namespace kvr {
namespace {

constexpr int kAttnThreads = 256;
constexpr int kAttnWaves = kAttnThreads / kWave;

typedef uint32_t u32x4a __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Element i of a row of binary32, binary16 or bfloat16 scalars is read
// through the dword that holds it (one load instruction whatever the
// format; a per-format branch would wait for each load where it joins):
// scalar_word gives that dword and the element's bit offset in it,
// scalar_value converts.  Loads are issued first and converted after.
__device__ __forceinline__ const uint32_t *scalar_word(const uint8_t *p, uint32_t scalar, uint32_t i,
                                                       uint32_t &shift) {
    const uint32_t lead = uint32_t(reinterpret_cast<uintptr_t>(p) & 3u);
    const uint32_t at = lead + (scalar == kScalarF32 ? 4u : 2u) * i;  // bytes past the dword below p
    shift = (at & 2u) * 8u;
    return reinterpret_cast<const uint32_t *>(p - lead) + (at >> 2);
}
// Straight-line (masks, not selects: a uniform select can become a branch,
// which would split the block the loads are scheduled in).
__device__ __forceinline__ float scalar_value(uint32_t w, uint32_t shift, uint32_t scalar) {
    const uint32_t h = (w >> shift) & 0xffffu;
    const uint32_t m32 = 0u - uint32_t(scalar == kScalarF32), m16 = 0u - uint32_t(scalar == kScalarF16);
    const uint32_t bits = (w & m32) | (__float_as_uint(h2f(uint16_t(h))) & m16) | ((h << 16) & ~(m32 | m16));
    return __uint_as_float(bits);
}

// Bytes of one 32-value block and the dword-aligned words that hold it.
template <int KF> struct KeyBlock;
template <> struct KeyBlock<kKeyF16> { static constexpr uint32_t kBytes = 64; };
template <> struct KeyBlock<kKeyBF16> { static constexpr uint32_t kBytes = 64; };
template <> struct KeyBlock<kKeyF32> { static constexpr uint32_t kBytes = 128; };
template <> struct KeyBlock<kKeyQ8> { static constexpr uint32_t kBytes = 34; };
template <> struct KeyBlock<kKeyQ4> { static constexpr uint32_t kBytes = 18; };
template <> struct KeyBlock<kKeyQ5> { static constexpr uint32_t kBytes = 22; };

template <int KF> constexpr bool kQuantized = KF == kKeyQ8 || KF == kKeyQ4 || KF == kKeyQ5;

// Raw words of one block.  Scalar formats: the block's 16-byte vectors.
// Quantized formats (blocks start on 2-byte boundaries): n = (bytes-2)/4
// dwords from the dword boundary at or below the block, then the block's
// last two 16-bit halves, so every load stays inside the block's own dword
// span and never reads past its last byte.
template <int KF> struct RawBlock {
    static constexpr uint32_t kVec = kQuantized<KF> ? 1 : KeyBlock<KF>::kBytes / 16;
    static constexpr uint32_t kWords = kQuantized<KF> ? (KeyBlock<KF>::kBytes - 2) / 4 : 0;
    u32x4 v[kVec > 0 ? kVec : 1];
    uint32_t w[kWords > 0 ? kWords : 1];
    uint32_t t0, t1, odd;
};

template <int KF>
__device__ __forceinline__ RawBlock<KF> load_block(const uint8_t *row, uint32_t b) {
    RawBlock<KF> r;
    const uint8_t *p = row + b * KeyBlock<KF>::kBytes;
    if constexpr (!kQuantized<KF>) {
#pragma unroll
        for (uint32_t i = 0; i < RawBlock<KF>::kVec; ++i) r.v[i] = reinterpret_cast<const u32x4 *>(p)[i];
    } else {
        constexpr uint32_t B = KeyBlock<KF>::kBytes, n = RawBlock<KF>::kWords;
        r.odd = uint32_t(reinterpret_cast<uintptr_t>(p) & 2u);
        const uint32_t *base = reinterpret_cast<const uint32_t *>(p - r.odd);  // keeps the global address space
        const u32x4a lo = *reinterpret_cast<const u32x4a *>(base);
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) r.w[i] = lo[i];
        if constexpr (n == 8) {
            const u32x4a hi = *reinterpret_cast<const u32x4a *>(base + 4);
#pragma unroll
            for (uint32_t i = 0; i < 4; ++i) r.w[4 + i] = hi[i];
        } else if constexpr (n == 5) {
            r.w[4] = base[4];
        }
        r.t0 = *reinterpret_cast<const uint16_t *>(p + B - 4);
        r.t1 = *reinterpret_cast<const uint16_t *>(p + B - 2);
    }
    return r;
}

// The block's values in order, as the reference decodes them
// (llama-kvmem-attention-cuda.cu:37-56): element i of a quantized block is
// its integer code times the fp16 scale, a product exact in binary32.
template <int KF>
__device__ __forceinline__ void decode_block(const RawBlock<KF> &r, float *out) {
    if constexpr (KF == kKeyF32) {
#pragma unroll
        for (int i = 0; i < 32; ++i) out[i] = __uint_as_float(r.v[i / 4][i % 4]);
    } else if constexpr (KF == kKeyF16 || KF == kKeyBF16) {
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            const uint16_t h = uint16_t(r.v[i / 8][(i % 8) / 2] >> (16 * (i % 2)));
            out[i] = KF == kKeyF16 ? h2f(h) : bf2f(h);
        }
    } else {
        // v[j] = block bytes [4j, 4j+4)
        constexpr uint32_t n = RawBlock<KF>::kWords;
        uint32_t v[n + 1];
#pragma unroll
        for (uint32_t j = 0; j + 1 < n; ++j) v[j] = r.odd ? __builtin_amdgcn_alignbyte(r.w[j + 1], r.w[j], 2) : r.w[j];
        v[n - 1] = r.odd ? (r.w[n - 1] >> 16) | (r.t0 << 16) : r.w[n - 1];
        v[n] = r.t1;
        const float d = h2f(uint16_t(v[0]));
        if constexpr (KF == kKeyQ8) {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const uint32_t c = __builtin_amdgcn_alignbyte(v[k + 1], v[k], 2);  // codes 4k..4k+3
#pragma unroll
                for (int m = 0; m < 4; ++m) out[4 * k + m] = float(int8_t(c >> (8 * m))) * d;
            }
        } else if constexpr (KF == kKeyQ4) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t c = __builtin_amdgcn_alignbyte(v[k + 1], v[k], 2);  // qs[4k..4k+3]
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const uint32_t byte = (c >> (8 * m)) & 0xffu;
                    out[4 * k + m] = float(int(byte & 15u) - 8) * d;
                    out[16 + 4 * k + m] = float(int(byte >> 4) - 8) * d;
                }
            }
        } else {
            const uint32_t qh = __builtin_amdgcn_alignbyte(v[1], v[0], 2);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t c = __builtin_amdgcn_alignbyte(v[k + 2], v[k + 1], 2);  // qs[4k..4k+3]
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const uint32_t byte = (c >> (8 * m)) & 0xffu;
                    const int i = 4 * k + m;
                    out[i] = float(int((byte & 15u) | (((qh >> i) & 1u) << 4)) - 16) * d;
                    out[16 + i] = float(int((byte >> 4) | (((qh >> (16 + i)) & 1u) << 4)) - 16) * d;
                }
            }
        }
    }
}

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
constexpr uint32_t kPairTile = 16;   // (row, query head) pairs per workgroup: the MFMA's M
constexpr uint32_t kTokenTile = 16;  // tokens per MFMA: its N
constexpr float kLog2e = 1.44269504088896340736f, kLn2 = 0.693147180559945309417f;

// A group of pages of one kv-head for a tile of 16 (row, query head) pairs
// on the matrix cores: v_mfma_f32_16x16x4f32 multiplies 16 pairs' queries
// (16 x 4 dims) by 16 tokens' keys (4 dims x 16 tokens) and accumulates
// over the head dim.  Lane l supplies A[pair l%16][k = l/16] and B[k =
// l/16][token l%16]; in round r the k index g = l/16 walks the 32 dims of
// key block 4r+g, so each lane decodes whole blocks of its own token (the
// same dot product, summed in another order).  The lane receives D[pair
// 4*(l/16)+i][token l%16], i = 0..3.  Pair p0+m is sampled row (p0+m)/group
// and query head kv*group + (p0+m)%group.
//
// fp16 keys take v_mfma_f32_16x16x32_f16 instead: one MFMA per 32-dim key
// block, lane l supplying 8 dims of block b (its k slots; A and B use the
// same slots, so the dot product is the same) straight from its 16-byte key
// load, with no decode.  The binary32 query is split into fp16 high and low
// parts (q = hi + lo to about 2^-22 relative) after scaling each pair by a
// power of two that keeps its largest element below 2^15; the products of
// fp16 parts are exact, accumulation is binary32 in the matrix core, and
// the power of two comes back with the logit scale.  Two MFMAs (hi, lo) per
// block: 8 per 16-token tile at head dim 128, against 32 of the f32 form.
//
// q8_0 keys (head dims that are multiples of 128) take the fp16 matrix
// cores too: a wave's 16-token tile is staged through its own LDS slot with
// coalesced 16-byte loads (the tile's rows are 34-byte blocks, not 16-byte
// aligned), and each lane then reads its 8 codes of each block and the
// block's fp16 scale from LDS.  Codes become fp16 exactly (0x64 high byte
// over code + 128, less 1152); per block a hi and a lo MFMA from zero give
// the pair's dot product with the codes, which the lane multiplies by its
// token's block scale before adding it up.
//
// The workgroup's 16-token tiles, page after page, are dealt to its waves
// in turn (flat tile f goes to wave f%4), and each wave streams its tiles
// through one ring of loads across the pages.  When a page is 16, 32, 64,
// 128 or 256 tokens (BATCH), a wave's tiles of one page come in one run of
// n = 1, 1, 1, 2 or 4 consecutive tiles of its own: the lanes keep the
// run's logits, and at the run's end one max over the run (16 lanes by DPP)
// and one exponential per token give the page's partial -- one exponential
// per token and pair.  Otherwise lanes keep a running max and rescaled sum
// per pair in base 2 (two exponentials per token and pair) and fold their
// 16 lanes where a wave's next tile is on another page.  Either way the
// page's partial of each wave goes to LDS; one barrier at the end, then the
// four waves' partials of each (page, pair) give its log-sum-exp.
enum AttnPath : int { kPathF32 = 0, kPathF16 = 1, kPathQ8 = 2 };
constexpr uint32_t kMaxPageGroup = 16;
// G4: the query-head group is a multiple of 4, so a lane's four output
// pairs 4*kg+i (i = 0..3, from a multiple of 16) are heads of one sampled
// row and share its mask word: one load and one decode per tile, not four.
template <int KF, int R, bool G4, int PATH, bool BATCH>
__global__ __launch_bounds__(kAttnThreads) void k_attn_lse(AttnArgs a) {
    constexpr bool kHalf = PATH != kPathF32;  // fp16 matrix-core forms
    constexpr bool kQ8 = PATH == kPathQ8;
    // q8_0 staging: a token's kv-head row is RB bytes (4R blocks of 34),
    // read as CPR 16-byte chunks (the last one ends at the row's end),
    // NL chunks per lane for a 16-row tile
    constexpr uint32_t RB = 136 * R, CPR = (RB + 15) / 16, CH = kTokenTile * CPR, NL = (CH + kWave - 1) / kWave;
    __shared__ float part[2][kMaxPageGroup][kAttnWaves][kPairTile];  // max, sum
    __shared__ float glse[kMaxPageGroup][kPairTile];                 // the group's log-sum-exps
    // q8_0: one LDS tile per wave (a tile is staged and consumed within one
    // step, and a wave's LDS operations complete in order)
    __shared__ __align__(16) uint8_t q8_tiles[kQ8 ? kAttnWaves * kTokenTile * RB : 16];
    const uint32_t groups = (a.pages + a.page_group - 1) / a.page_group;
    const uint32_t kv = blockIdx.x / groups, pg0 = (blockIdx.x % groups) * a.page_group;
    const uint32_t npg = min(a.page_group, a.pages - pg0);
    const uint32_t p0 = blockIdx.y * kPairTile, npairs = a.n_rows * a.group;
    const uint32_t tid = threadIdx.x, lane = tid % kWave;
    // the wave index as a scalar: tile and page arithmetic stays on the
    // scalar unit
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid / kWave);
    const uint32_t col = lane % 16, kg = lane / 16;
    const uint32_t nb = a.dim / 32;
    const uint32_t T = (a.page_tokens + kTokenTile - 1) / kTokenTile;  // tiles per page
    const uint32_t nflat = npg * T;
    // a run: the wave's consecutive tiles of one page (BATCH)
    const uint32_t run = T <= 2 ? 1u : T / 4;
    for (uint32_t i = tid; i < npg * kAttnWaves * kPairTile; i += kAttnThreads) {
        (&part[0][0][0][0])[i] = -__builtin_inff();
        (&part[1][0][0][0])[i] = 0.0f;
    }
    auto pair_row = [&](uint32_t p) { return a.rows[p / a.group]; };
    auto block_of = [&](uint32_t r) { return min(4 * r + kg, nb - 1); };
    // wave-local tile k is flat tile w + 4k: page pg0 + flat/T, tile flat%T;
    // tokens past the page or the sequence are clamped to the last token
    // (in bounds) and not counted
    // flat tile -> (page, tile of the page); BATCH pages are a power of two
    // of tiles, so a shift (the division otherwise: dozens of scalar
    // instructions per tile)
    const uint32_t tsh = uint32_t(__builtin_ctz(T));
    auto tdiv = [&](uint32_t f) { return BATCH ? f >> tsh : f / T; };
    auto tmod = [&](uint32_t f) { return BATCH ? f & (T - 1) : f % T; };
    auto tile_page = [&](uint32_t k) { return tdiv(min(w + kAttnWaves * k, nflat - 1)); };
    auto tile_first = [&](uint32_t k, uint32_t &end) {
        const uint32_t fc = min(w + kAttnWaves * k, nflat - 1);
        const uint32_t pg = pg0 + tdiv(fc);
        end = min(pg * a.page_tokens + a.page_tokens, a.tokens);
        return pg * a.page_tokens + tmod(fc) * kTokenTile;
    };
    auto tile_token = [&](uint32_t k, bool &live) {
        uint32_t end;
        const uint32_t t = tile_first(k, end) + col;
        live = w + kAttnWaves * k < nflat && t < end;
        return min(t, end - 1);
    };
    const uint8_t *mrow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        mrow[i] = a.mask + uint64_t(a.mask_rows[min(p0 + 4 * kg + i, npairs - 1) / a.group]) * a.mask_row_stride;

    // ring of two slots: a tile's slot is consumed and refilled with the
    // wave's tile two on before its MFMAs run (four slots were measured
    // slower: the registers cost a wave per SIMD)
    constexpr int RING = 2;
    RawBlock<KF> ring[RING][kQ8 ? 1 : R];
    u32x4 qraw[RING][kQ8 ? NL : 1];  // q8_0: the slot's staged chunks
    u32x4 bw[RING];                  // mask words (one register tuple per slot)
    uint32_t bsh[RING][4];
    // chunk j of this lane in a q8_0 tile: row rr, byte offset off in the row
    auto chunk = [&](uint32_t j, uint32_t &rr, uint32_t &off) {
        const uint32_t c = min(lane + kWave * j, CH - 1);  // lanes past the tile repeat its last chunk
        rr = c / CPR;
        off = min(16 * (c - rr * CPR), RB - 16);
    };
    // Matrix-core forms: a tile's keys through a buffer resource from its
    // first token's row of this kv-head, so each lane's offsets are the same
    // in every tile (no address arithmetic per tile) and rows past the
    // sequence read as zeros (they are never counted).  Offsets are 32-bit:
    // the host keeps key rows under 128 MiB.  The default cache policy: the
    // streaming (nontemporal) one was measured 30% slower for fp16 keys.
    const uint32_t krs = uint32_t(a.k_row_stride), head_bytes = nb * KeyBlock<KF>::kBytes;
    auto key_rsrc = [&](uint32_t first) {
        const uint32_t rows = min(a.tokens - first, kTokenTile);
        return buffer_rsrc(a.k + uint64_t(first) * a.k_row_stride + uint64_t(kv) * a.k_head_stride,
                           (rows - 1) * krs + head_bytes);
    };
    const uint32_t f16_off = col * krs + 16 * kg;  // fp16: the lane's token row, its 16 bytes of a block
    uint32_t q8_off[kQ8 ? NL : 1];                 // q8_0: the lane's staged chunks
#pragma unroll
    for (uint32_t j = 0; j < (kQ8 ? NL : 1); ++j) {
        uint32_t rr, off;
        chunk(j, rr, off);
        q8_off[j] = rr * krs + off;
    }
    auto issue = [&](int slot, uint32_t k) {
        bool live;
        const uint32_t t = tile_token(k, live);
        if constexpr (kQ8) {
            uint32_t end;
            const auto rs = key_rsrc(tile_first(k, end));
#pragma unroll
            for (uint32_t j = 0; j < NL; ++j)
                qraw[slot][j] = __builtin_bit_cast(
                    u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, int(q8_off[j]), 0, 0));
        } else if constexpr (PATH == kPathF16) {
            // 16 bytes (8 dims) of each of blocks 4r..4r+3 (clamped to the
            // head's last block; blocks past it meet zero queries)
            uint32_t end;
            const auto rs = key_rsrc(tile_first(k, end));
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    ring[slot][r].v[i] = __builtin_bit_cast(
                        u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                   rs, int(f16_off + min(4u * r + i, nb - 1) * KeyBlock<KF>::kBytes), 0, 0));
        } else {
            const uint8_t *row = a.k + uint64_t(t) * a.k_row_stride + uint64_t(kv) * a.k_head_stride;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if constexpr (kHalf) {
                    // 16 bytes (8 dims) of each of blocks 4r..4r+3 (clamped to
                    // the head's last block; blocks past it meet zero queries)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        ring[slot][r].v[i] = *reinterpret_cast<const u32x4 *>(
                            row + min(4u * r + i, nb - 1) * KeyBlock<KF>::kBytes + 16 * kg);
                } else {
                    ring[slot][r] = load_block<KF>(row, block_of(r));
                }
            }
        }
#pragma unroll
        for (int i = 0; i < (G4 ? 1 : 4); ++i) bw[slot][i] = *scalar_word(mrow[i], a.mask_scalar, t, bsh[slot][i]);
    };
    // A operand: pair p0+col, the 32 dims of block 4r+kg (zero past the
    // head dim or the pairs).  Its loads go first, then the ring's first
    // two tiles, then the conversion: the loop is entered with exactly the
    // two slots' loads outstanding, in slot order, as at its back edge.
    // f32 form: element s of round r is dim 32*(4r+kg) + s.  fp16 forms:
    // dim 32*(4r + s/8) + 8*kg + s%8, kept as hi/lo fp16 parts (qh, ql).
    auto q_dim = [&](int r, int s) {
        return kHalf ? 32 * min(4u * r + s / 8, nb - 1) + 8 * kg + s % 8 : 32 * block_of(r) + s;
    };
    auto q_on = [&](int r, int s) { return 4 * r + (kHalf ? uint32_t(s) / 8 : kg) < nb; };
    float qa[R][32];
    f16x8 qh[R][4], ql[R][4];
    float lscale[4];   // logit scale of the lane's output pairs 4*kg + i
    float lscale2[4];  // the same times log2(e)
    {
        const uint32_t p = p0 + col;
        const uint32_t pc = min(p, npairs - 1);
        const uint8_t *qrow = a.q + uint64_t(pair_row(pc)) * a.q_row_stride +
                              uint64_t(kv * a.group + pc % a.group) * a.q_head_stride;
        uint32_t qw[R][32], qs[R][32];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int s = 0; s < 32; ++s) qw[r][s] = *scalar_word(qrow, a.q_scalar, q_dim(r, s), qs[r][s]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int r = 0; r < RING; ++r) issue(r, uint32_t(r));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int s = 0; s < 32; ++s)
                qa[r][s] = p < npairs && q_on(r, s) ? scalar_value(qw[r][s], qs[r][s], a.q_scalar) : 0.0f;
        }
        if constexpr (kHalf) {
            // the pair's largest |q| over its four lanes (col, col+16, ...)
            float mx = 0.0f;
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int s = 0; s < 32; ++s) mx = fmaxf(mx, fabsf(qa[r][s]));
            mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
            mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
            // 2^-e brings it into [2^13, 2^15) (exact), small queries scaled
            // up as large ones are scaled down, so the fp16 parts keep their
            // bits (binary exponent from the bits; e in [-100, 100], so a zero
            // or subnormal maximum stays tiny and the logit scale 2^e * scale
            // stays a normal number)
            const int e = min(max(int((__float_as_uint(mx) >> 23) & 0xffu) - 127 - 13, -100), 100);
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const float x = __builtin_ldexpf(qa[r][8 * i + j], -e);
                        const _Float16 hi = _Float16(x);
                        qh[r][i][j] = hi;
                        ql[r][i][j] = _Float16(x - float(hi));
                    }
            const float own = __builtin_ldexpf(a.scale, e);
#pragma unroll
            for (int i = 0; i < 4; ++i) lscale[i] = __shfl(own, 4 * kg + i, kWave);
#pragma unroll
            for (int i = 0; i < 4; ++i) lscale2[i] = lscale[i] * kLog2e;
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) lscale[i] = a.scale;
#pragma unroll
            for (int i = 0; i < 4; ++i) lscale2[i] = a.scale * kLog2e;
        }
    }
    lds_barrier();  // partials initialized

    float m[4], sm[4];   // online form: running max and sum per output pair
    float lb[4][4];      // BATCH: the run's logits, tile j of the run in lb[j]
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        m[i] = -__builtin_inff();
        sm[i] = 0.0f;
    }
    const uint32_t nk = nflat > w ? (nflat - w + kAttnWaves - 1) / kAttnWaves : 0;  // this wave's tiles
    // The page's partial of this wave from the run's logits lb[t0..t1]
    // (positions known where the call is inlined): per pair the max over
    // the run's tokens (its 16 lanes by DPP), then the sum of exp2(l - max).
    // A NaN logit is left out of both (fmaxf), as is a -inf one.  Stored
    // for tiles of this wave only (padding tiles past nk are dropped).
    auto flush = [&](uint32_t k, int t0, int t1) {
        const uint32_t pl = tile_page(k);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float bm = lb[t1][i];
#pragma unroll
            for (int t = 0; t < 4; ++t)
                if (t >= t0 && t < t1) bm = fmaxf(bm, lb[t][i]);
            const float rm = dpp::group_reduce(bm, 16, dpp::FMax());
            float sv = 0.0f;
#pragma unroll
            for (int t = 0; t < 4; ++t)
                if (t >= t0 && t <= t1) sv += __builtin_amdgcn_exp2f(fmaxf(lb[t][i] - rm, -__builtin_inff()));
            const float e = dpp::group_reduce(sv, 16, dpp::Add());
            if (col == 0 && k < nk) {
                part[0][pl][w][4 * kg + i] = rm;
                part[1][pl][w][4 * kg + i] = e;
            }
        }
    };
    // process(slot, k, j): tile k (position j of a four-tile loop step)
    auto process = [&](int slot, uint32_t k, int j) {
        float kv32[kHalf ? 1 : R][32];
#pragma unroll
        for (int r = 0; r < (kHalf ? 1 : R); ++r)
            if constexpr (!kHalf) decode_block<KF>(ring[slot][r], kv32[r]);
        float bias[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            bias[i] = G4 && i > 0 ? bias[0] : scalar_value(bw[slot][i], bsh[slot][i], a.mask_scalar);
            // pinned here: the slot's old words are consumed before its
            // refill is issued (a conversion sunk past it would keep both
            // live, and the refill would land in registers that the loop's
            // back edge copies, waiting for the loads)
            asm volatile("" : "+v"(bias[i]));
        }
        // two accumulation chains keep two MFMAs of the wave in flight
        f32x4 acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = acc0;
        if constexpr (PATH == kPathF16) {
            // (hi chain, lo chain) on the slot's raw key words, issued
            // before the slot's refill overwrites them
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const f16x8 kb = __builtin_bit_cast(f16x8, ring[slot][r].v[i]);
                    acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(qh[r][i], kb, acc0, 0, 0, 0);
                    acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ql[r][i], kb, acc1, 0, 0, 0);
                }
        }
        uint8_t *tile = q8_tiles + w * (kTokenTile * RB);
        if constexpr (kQ8) {
            // stage the slot's chunks in this wave's LDS tile; the slot's
            // registers are then free for the refill
#pragma unroll
            for (uint32_t jj = 0; jj < NL; ++jj) {
                uint32_t rr, off;
                chunk(jj, rr, off);
                uint64_t *d = reinterpret_cast<uint64_t *>(tile + rr * RB + off);
                d[0] = uint64_t(qraw[slot][jj][0]) | (uint64_t(qraw[slot][jj][1]) << 32);
                d[1] = uint64_t(qraw[slot][jj][2]) | (uint64_t(qraw[slot][jj][3]) << 32);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        issue(slot, k + RING);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (kQ8) {
            // this lane's token is tile row `col`: per block b its fp16 scale
            // and codes 8*kg..8*kg+7 (dword-aligned for odd blocks, two bytes
            // into a dword for even ones)
            const uint8_t *rowp = tile + col * RB;
            f32x4 t[4 * R];
            float db[4 * R];
#pragma unroll
            for (int b = 0; b < 4 * R; ++b) {
                db[b] = h2f(*reinterpret_cast<const uint16_t *>(rowp + 34 * b));
                uint32_t lo, hi;
                if (b & 1) {
                    const uint32_t *p = reinterpret_cast<const uint32_t *>(rowp + 34 * b + 2 + 8 * kg);
                    lo = p[0];
                    hi = p[1];
                } else {
                    const uint32_t *p = reinterpret_cast<const uint32_t *>(rowp + 34 * b + 8 * kg);
                    const uint32_t w0 = p[0], w1 = p[1], w2 = p[2];
                    lo = __builtin_amdgcn_alignbyte(w1, w0, 2);
                    hi = __builtin_amdgcn_alignbyte(w2, w1, 2);
                }
                // int8 codes as fp16 1024 + (code + 128), less 1152: exact
                const uint32_t xl = lo ^ 0x80808080u, xh = hi ^ 0x80808080u;
                const u32x4 hv = {__builtin_amdgcn_perm(0x64646464u, xl, 0x04010400u),
                                  __builtin_amdgcn_perm(0x64646464u, xl, 0x04030402u),
                                  __builtin_amdgcn_perm(0x64646464u, xh, 0x04010400u),
                                  __builtin_amdgcn_perm(0x64646464u, xh, 0x04030402u)};
                const f16x8 kb = __builtin_bit_cast(f16x8, hv) - f16x8(_Float16(1152.0f));
                const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
                t[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qh[b / 4][b % 4], kb, z, 0, 0, 0);
                t[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ql[b / 4][b % 4], kb, t[b], 0, 0, 0);
            }
#pragma unroll
            for (int b = 0; b < 4 * R; ++b)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc0[i] = fmaf(t[b][i], db[b], acc0[i]);
        }
        if constexpr (PATH == kPathF32) {
            // even and odd k-steps; k-steps past the head dim have zero
            // queries
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int s = 0; s < 32; s += 2) {
                    acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[r][s], kv32[r][s], acc0, 0, 0, 0);
                    acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[r][s + 1], kv32[r][s + 1], acc1, 0, 0, 0);
                }
        }
        bool live;
        (void)tile_token(k, live);
        // base-2 logits: (dot * scale + bias) * log2(e), one fma without a
        // softcap (scale and bias premultiplied by log2(e))
        float l[4];
        if (a.softcap > 0.0f) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const bool use = live && __builtin_isfinite(bias[i]);
                float x = (kQ8 ? acc0[i] : acc0[i] + acc1[i]) * lscale[i];
                x = a.softcap * tanhf(x / a.softcap);
                l[i] = use ? (x + bias[i]) * kLog2e : -__builtin_inff();
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const bool use = live && __builtin_isfinite(bias[i]);
                const float b2 = G4 && i > 0 ? bias[0] * kLog2e : bias[i] * kLog2e;
                l[i] = use ? fmaf(kQ8 ? acc0[i] : acc0[i] + acc1[i], lscale2[i], b2) : -__builtin_inff();
            }
        }
        if constexpr (BATCH) {
#pragma unroll
            for (int i = 0; i < 4; ++i) lb[j][i] = l[i];
            // the run ends here: its page's partial (uniform branches on the
            // run length, each holding temporaries and LDS stores only)
            if (run == 4) {
                if (j == 3) flush(k, 0, 3);
            } else if (run == 2) {
                if (j & 1) flush(k, j - 1, j);
            } else {
                flush(k, j, j);
            }
        } else {
            // running max and sum in base 2 (branch-free: a token left out
            // has l = -inf, so nm = m and the sum is kept as it is)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float nm = fmaxf(m[i], l[i]);
                const float keep = m[i] == nm ? 1.0f : __builtin_amdgcn_exp2f(m[i] - nm);
                sm[i] = sm[i] * keep + (l[i] > -__builtin_inff() ? __builtin_amdgcn_exp2f(l[i] - nm) : 0.0f);
                m[i] = nm;
            }
            // this wave's last tile of the page: fold the 16 lanes of each
            // row (same pairs, different tokens) into the page's partial
            // (the branch holds temporaries and LDS stores only: running
            // values changed inside it would need merging copies at the
            // loop's back edge, which wait for the ring's loads)
            const uint32_t pl = tile_page(k);
            const bool last = k < nk && (k + 1 == nk || tile_page(k + 1) != pl);  // (padding tiles never flush)
            if (last) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float rm = dpp::group_reduce(m[i], 16, dpp::FMax());
                    const float e = dpp::group_reduce(sm[i] > 0.0f ? sm[i] * __builtin_amdgcn_exp2f(m[i] - rm) : 0.0f,
                                                      16, dpp::Add());
                    if (col == 0) {
                        part[0][pl][w][4 * kg + i] = rm;
                        part[1][pl][w][4 * kg + i] = e;
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                m[i] = last ? -__builtin_inff() : m[i];
                sm[i] = last ? 0.0f : sm[i];
            }
        }
    };
    // straight-line body (a skipped call would make the ring slots' values
    // path-dependent, and the copies that merge them wait for the loads):
    // a tile past the wave's last is computed and not counted
    if constexpr (BATCH) {
        for (uint32_t k = 0; k < nk; k += 4) {
            process(0, k, 0);
            process(1, k + 1, 1);
            process(0, k + 2, 2);
            process(1, k + 3, 3);
        }
    } else {
        for (uint32_t k = 0; k < nk; k += 2) {
            process(0, k, 0);
            process(1, k + 1, 1);
        }
    }
    lds_barrier();
    for (uint32_t i = tid; i < npg * kPairTile; i += kAttnThreads) {
        const uint32_t pl = i / kPairTile, pr = i % kPairTile, p = p0 + pr;
        if (p >= npairs) continue;
        float mx = part[0][pl][0][pr];
#pragma unroll
        for (int v = 1; v < kAttnWaves; ++v) mx = fmaxf(mx, part[0][pl][v][pr]);
        float total = 0.0f;
#pragma unroll
        for (int v = 0; v < kAttnWaves; ++v) {
            const float sv = part[1][pl][v][pr];
            total += sv > 0.0f ? sv * __builtin_amdgcn_exp2f(part[0][pl][v][pr] - mx) : 0.0f;
        }
        // back to base e: lse = (max2 + log2(total)) * ln 2
        const uint32_t r = p / a.group, h = kv * a.group + p % a.group;
        const float v = total > 0.0f ? (mx + __builtin_amdgcn_logf(total)) * kLn2 : -__builtin_inff();
        a.lse[(uint64_t(r) * a.heads + h) * a.pages + pg0 + pl] = v;
        glse[pl][pr] = v;
    }
    lds_barrier();
    // Each pair's max m of the group's page log-sum-exps and sum of
    // exp(lse - m) (0 when every page is -inf): the normalization's max and
    // sum over pages, taken per page group here and combined over the
    // groups by the mass kernel.
    if (tid < kPairTile && p0 + tid < npairs) {
        float m = -__builtin_inff(), sum = 0.0f;
        for (uint32_t pl = 0; pl < npg; ++pl) m = fmaxf(m, glse[pl][tid]);
        if (m > -__builtin_inff())
            for (uint32_t pl = 0; pl < npg; ++pl) sum += expf(glse[pl][tid] - m);
        const uint32_t p = p0 + tid, r = p / a.group, h = kv * a.group + p % a.group;
        float *st = a.stats + ((uint64_t(r) * a.heads + h) * groups + pg0 / a.page_group) * 2;
        st[0] = m;
        st[1] = sum;
    }
}

// Masses of one sampled row over a chunk of 256 pages.  Every workgroup of
// the row first takes, for each head, the max M over pages of its page
// log-sum-exps and 1/S, S = sum of exp(lse - M), from the page groups'
// (max m, sum s) pairs: M = max of the m, S = sum of s * exp(m - M).  One
// head per 16-lane row at a time, two heads per row with their loads in
// flight, four groups per lane per pass (a running max and rescaled sum
// beyond).  Then, for each page of its chunk, the head average of
// exp(lse - M) * (1/S): the reference's normalize and average kernels.
// The row's tables are read through buffer resources with 32-bit offsets
// (the host keeps a row's under 4 GiB), and each batch of loads is issued
// before the first of them is used.
constexpr uint32_t kMassPages = 256;
__device__ __forceinline__ float lse_at(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, int(off), 0, 0));
}
__global__ __launch_bounds__(kAttnThreads) void k_attn_mass(AttnArgs a) {
    extern __shared__ float norm[];  // [heads][2]
    const uint32_t r = blockIdx.y, tid = threadIdx.x, lane = tid % kWave;
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid / kWave);
    const uint32_t groups = (a.pages + a.page_group - 1) / a.page_group;
    const auto rs = buffer_rsrc(a.lse + uint64_t(r) * a.heads * a.pages, a.heads * a.pages * uint32_t(sizeof(float)));
    const auto ss = buffer_rsrc(a.stats + uint64_t(r) * a.heads * groups * 2, a.heads * groups * 2 * uint32_t(sizeof(float)));
    const uint32_t row = w * 4 + lane / 16, c = lane % 16;  // 16 rows of 16 lanes
    for (uint32_t h0 = row; h0 < a.heads; h0 += 32) {
        float m[2], sum[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            m[j] = -__builtin_inff();
            sum[j] = 0.0f;
        }
        for (uint32_t g0 = 0; g0 < groups; g0 += 64) {
            float vm[2][4], vs[2][4];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint32_t h = min(h0 + 16 * j, a.heads - 1);
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const uint32_t off = (h * groups + min(g0 + 16 * u + c, groups - 1)) * 2 * uint32_t(sizeof(float));
                    vm[j][u] = lse_at(ss, off);
                    vs[j][u] = lse_at(ss, off + 4);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const bool on = g0 + 16 * u + c < groups && vs[j][u] > 0.0f;
                    const float x = on ? vm[j][u] : -__builtin_inff();
                    const float nm = fmaxf(m[j], x);
                    sum[j] = (sum[j] > 0.0f ? sum[j] * expf(m[j] - nm) : 0.0f) + (on ? vs[j][u] * expf(x - nm) : 0.0f);
                    m[j] = nm;
                }
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const float gm = dpp::group_reduce(m[j], 16, dpp::FMax());
            const float gs = dpp::group_reduce(sum[j] > 0.0f ? sum[j] * expf(m[j] - gm) : 0.0f, 16, dpp::Add());
            const uint32_t h = h0 + 16 * j;
            if (c == 0 && h < a.heads) {
                // a head whose every page is -inf: max -inf, 1/sum NaN (as
                // the reference's normalize gives)
                norm[2 * h] = gm;
                norm[2 * h + 1] = gm > -__builtin_inff() ? 1.0f / gs : __builtin_nanf("");
            }
        }
    }
    lds_barrier();
    const uint32_t p = blockIdx.x * kMassPages + tid;
    if (p >= a.pages) return;
    // 32 heads' values of this page in flight at a time, added in head order
    float acc = 0.0f;
    for (uint32_t h0 = 0; h0 < a.heads; h0 += 32) {
        float v[32];
#pragma unroll
        for (uint32_t j = 0; j < 32; ++j) v[j] = lse_at(rs, (min(h0 + j, a.heads - 1) * a.pages + p) * uint32_t(sizeof(float)));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (uint32_t j = 0; j < 32; ++j)
            if (h0 + j < a.heads) acc += expf(v[j] - norm[2 * (h0 + j)]) * norm[2 * (h0 + j) + 1];
    }
    a.mass[uint64_t(r) * a.pages + p] = acc / float(a.heads);
}

template <int KF, int PATH, bool BATCH>
hipError_t launch_lse_t(const AttnArgs &a, const dim3 &grid, hipStream_t s) {
    const bool g4 = a.group % 4 == 0;
    if (a.dim <= 128 && g4) hipLaunchKernelGGL((k_attn_lse<KF, 1, true, PATH, BATCH>), grid, dim3(kAttnThreads), 0, s, a);
    else if (a.dim <= 128) hipLaunchKernelGGL((k_attn_lse<KF, 1, false, PATH, BATCH>), grid, dim3(kAttnThreads), 0, s, a);
    else if (g4) hipLaunchKernelGGL((k_attn_lse<KF, 2, true, PATH, BATCH>), grid, dim3(kAttnThreads), 0, s, a);
    else hipLaunchKernelGGL((k_attn_lse<KF, 2, false, PATH, BATCH>), grid, dim3(kAttnThreads), 0, s, a);
    return hipGetLastError();
}

// The key path: fp16 keys on the fp16 matrix cores; q8_0 keys too when the
// head dim is a multiple of 128 and every row is dword-aligned (the staged
// 16-byte loads); others decoded to binary32.  BATCH when a page's tiles
// split into equal runs per wave (pages of 16, 32, 64, 128 or 256 tokens).
template <int KF>
hipError_t launch_lse(const AttnArgs &a, hipStream_t s) {
    const uint32_t npairs = a.n_rows * a.group;
    const dim3 grid(a.kvheads * ((a.pages + a.page_group - 1) / a.page_group), (npairs + kPairTile - 1) / kPairTile);
    const uint32_t T = (a.page_tokens + kTokenTile - 1) / kTokenTile;
    const bool batch = T == 1 || T == 2 || T == 4 || T == 8 || T == 16;
    constexpr int base = KF == kKeyF16 ? kPathF16 : kPathF32;
    if constexpr (KF == kKeyQ8) {
        const bool staged = a.dim % 128 == 0 && (reinterpret_cast<uintptr_t>(a.k) | a.k_row_stride | a.k_head_stride) % 4 == 0;
        if (staged) return batch ? launch_lse_t<KF, kPathQ8, true>(a, grid, s) : launch_lse_t<KF, kPathQ8, false>(a, grid, s);
    }
    return batch ? launch_lse_t<KF, base, true>(a, grid, s) : launch_lse_t<KF, base, false>(a, grid, s);
}

}  // namespace

hipError_t launch_attention(const AttnArgs &a, hipStream_t s) {
    // one row's log-sum-exps and group pairs are addressed with 32-bit byte
    // offsets
    if (uint64_t(a.heads) * a.pages * 2 * sizeof(float) > 0xffffffffull) return hipErrorInvalidValue;
    hipError_t e = hipErrorInvalidValue;
    switch (a.k_format) {
    case kKeyF16: e = launch_lse<kKeyF16>(a, s); break;
    case kKeyBF16: e = launch_lse<kKeyBF16>(a, s); break;
    case kKeyF32: e = launch_lse<kKeyF32>(a, s); break;
    case kKeyQ8: e = launch_lse<kKeyQ8>(a, s); break;
    case kKeyQ4: e = launch_lse<kKeyQ4>(a, s); break;
    case kKeyQ5: e = launch_lse<kKeyQ5>(a, s); break;
    default: break;
    }
    if (e != hipSuccess) return e;
    const dim3 grid((a.pages + kMassPages - 1) / kMassPages, a.n_rows);
    hipLaunchKernelGGL(k_attn_mass, grid, dim3(kAttnThreads), size_t(a.heads) * 2 * sizeof(float), s, a);
    return hipGetLastError();
}

}  // namespace kvr
