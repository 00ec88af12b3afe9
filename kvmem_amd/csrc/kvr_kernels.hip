// kvr_kernels.hip -- gfx950 kernels of the recall hot path.
//
// Summary kernel (HBM-bound, the dominant cost): one lane owns 8 channels of
// one page (2 or 4 for a lone small fp16 layer) and walks the page's token
// rows in order, so a wave reads contiguous spans of each row and every
// channel is summed in the reference's order (binary32, token order from
// zero).  Scoring operands
// cross the recall fp16 boundary; logits, softmax and aggregation run in
// binary64 (the reference's CPU precision) so selection flips only on true
// near-ties.  Reference citations are relative to the KVMem 0.19.0 tree.
#include "kvr_device.hpp"
#include "kvr_internal.hpp"

#include <hip/hip_ext.h>
#include <math.h>

#include <type_traits>

namespace kvr {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef double f64x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
// 12-byte loads need only dword alignment on gfx950 (global_load_dwordx3).
typedef u32x3 u32x3a __attribute__((aligned(4)));

constexpr uint32_t kFmtF16 = 0, kFmtQ8 = 1, kFmtQ41 = 2, kFmtQ40 = 5;
constexpr uint32_t kModeCopy = 0, kModeDequantF16 = 1, kModeRequantQ8 = 2, kModeRopeFwht = 3;
constexpr uint32_t kQ40Bytes = 18;  // {fp16 d; uint8 qs[16]}

__device__ __forceinline__ float load_scalar(const uint8_t *p, uint32_t scalar) {
    if (scalar == kScalarF32) return *reinterpret_cast<const float *>(p);
    const uint16_t bits = *reinterpret_cast<const uint16_t *>(p);
    return scalar == kScalarF16 ? h2f(bits) : bf2f(bits);
}

// Raw bits of one query element (f32, or f16/bf16 in the low half), so its
// load can issue long before the value is converted.
__device__ __forceinline__ uint32_t load_raw(const uint8_t *p, uint32_t scalar) {
    return scalar == kScalarF32 ? *reinterpret_cast<const uint32_t *>(p)
                                : uint32_t(*reinterpret_cast<const uint16_t *>(p));
}
__device__ __forceinline__ float raw_value(uint32_t raw, uint32_t scalar) {
    if (scalar == kScalarF32) return __uint_as_float(raw);
    return scalar == kScalarF16 ? h2f(uint16_t(raw)) : bf2f(uint16_t(raw));
}
// Element i of one lane's query rows in (row, head, dim) order.
__device__ __forceinline__ const uint8_t *query_elem(const QueryArgs &q, uint32_t lane, uint32_t i) {
    const uint8_t *base = q.data + lane * q.lane_stride;
    if (q.dense) return base + uint64_t(i) * (q.scalar == kScalarF32 ? 4 : 2);
    const uint32_t d = i % q.dim, h = (i / q.dim) % q.qheads, r = i / (q.dim * q.qheads);
    return base + r * q.row_stride + h * q.head_stride + d * q.dim_stride;
}

__device__ __forceinline__ void add_f16x8(float *acc, const u32x4 v) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        acc[2 * i] += h2f(uint16_t(v[i] & 0xffffu));
        acc[2 * i + 1] += h2f(uint16_t(v[i] >> 16));
    }
}

// The fp16 channels one summary lane owns (8, 4 or 2) as one load: 16, 8
// or 4 bytes, so a wave reads 1 KiB, 512 B or 256 B of a row.
template <int CPL> struct F16Lane;
template <> struct F16Lane<8> { typedef u32x4 type; };
template <> struct F16Lane<4> { typedef u32x2 type; };
template <> struct F16Lane<2> { typedef uint32_t type; };
template <int CPL> __device__ __forceinline__ uint32_t lane_word(const typename F16Lane<CPL>::type &v, int i) {
    if constexpr (CPL == 2) return v;
    else return v[i];
}

__device__ __forceinline__ void add_q8x8(float *acc, uint32_t lo, uint32_t hi, float d) {
    // (float)q * d is exact in binary32 (8 x 11 significant bits), so the
    // fused multiply-add below rounds exactly like "p = q*d; acc += p".
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        acc[i] += float(int8_t(lo >> (8 * i))) * d;
        acc[4 + i] += float(int8_t(hi >> (8 * i))) * d;
    }
}

// The summary launch's fp16 key rows take the default cache policy in its
// one-wave workgroups (a lone small layer: measured 1.4 us faster per 64
// MiB layer than the streaming one) and the streaming policy in 256-thread
// ones (716 against 670 us per 8 lanes of 262144 tokens); its q8_0 rows and
// the stack's take the streaming policy, which measured faster there (q8_0
// summary 42.0 against 46.9 us per 131072-token layer; stack 15.2 against
// 16.6 us per 32768-token fp16 layer, 26.8 against 29.7 per 131072-token
// q8_0 layer).

// Ring depths of the summary streams: 12 rows of 16-byte loads (fp16) and
// 32 rows of 12-byte loads (q8_0).  Deeper rings of 16-byte loads make the
// register allocator copy ring slots whose loads are still in flight;
// narrower fp16 lanes (one 8- or 4-byte load per row) afford 32 rows (for
// 4-channel stack lanes 16 rows measured 178 us per steady launch, 24 rows
// 167.4 us, 32 rows 166.7 us).  48 rows of q8_0 measured slower than 32
// (k8v4 stack 27.7 against 26.7 us per layer).
constexpr int kF16Rows = 12, kQ8Rows = 32;
template <int CPL> constexpr int kF16RingRows = CPL == 8 ? kF16Rows : 32;

// Consumes rows 0..n-1 (n >= 1) in order through a ring of D loads in
// flight: row t's load issues D rows before row t is used.  Loads past the
// end are clamped to row n-1 (in bounds, never used), so no load sits behind
// a branch and the loads issue back to back.
template <int D, class Load, class Use>
__device__ __forceinline__ void stream_rows(uint32_t n, Load load, Use use) {
    decltype(load(0u)) ring[D];
    // The prologue's loads must issue in ring order: the wait before each
    // use counts loads still outstanding, so a reordered prologue would make
    // the first use of every pass wait for all of them.
#pragma unroll
    for (int u = 0; u < D; ++u) {
        ring[u] = load(min(uint32_t(u), n - 1));
        __builtin_amdgcn_sched_barrier(0);
    }
    uint32_t t = 0;
    for (; t + D < n; t += D) {
#pragma unroll
        for (int u = 0; u < D; ++u) {
            use(ring[u]);
            ring[u] = load(min(t + D + u, n - 1));
            // keeps each use beside its refill: hoisting the conversions of
            // later rows would wait for their loads before any refill issues
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int u = 0; u < D; ++u)
        if (t + u < n) use(ring[u]);
}

// ---------------------------------------------------------------------------
// Page summaries (+ fused logits).
// Restates RawKvStore::capture_mean_f16 / add_mean_f32 + mean_k
// (kvmem/src/host/raw_kv_store.cpp:158-197, 606-625) and, when FUSE, the
// logit loop of page_softmax_scores (kvmem/src/host/graph_recall.cpp:355-368).
// ---------------------------------------------------------------------------
// FUSE with q_stage: the workgroup's first lane's query rows, already
// through the fp16 operand boundary, staged once in dynamic LDS.
extern __shared__ __align__(16) uint16_t q_lds_buf[];

// One BS-thread block of the summary grid (`block` = its index in it):
// 256 threads, or 64 where a launch has fewer 256-thread blocks than the GPU
// has CUs (a lone small layer), so its blocks spread over every CU.
// CPL: fp16 channels per lane.  8 by default; a lone small fp16 layer takes
// 4 or 2, so the same rows are read by two or four times as many waves
// (every channel is still summed by one lane, in token order).
template <int SRC, bool FUSE, int BS = 256, int CPL = 8>
__device__ __forceinline__ void summary_block(const SummaryArgs &a, uint32_t block, uint16_t *q_lds) {
    static_assert(CPL == 8 || (SRC == kSrcKeysF16 && (CPL == 4 || CPL == 2)), "narrow lanes read fp16 keys");
    // Above the stage-in gather's waves when both share a CU: this kernel
    // is on the select critical path, the gather is bound by the host link.
    __builtin_amdgcn_s_setprio(2);
    const uint32_t gpp = a.width / CPL;  // channel groups per page
    const uint64_t gid = uint64_t(block) * BS + threadIdx.x;
    const uint64_t total = uint64_t(a.lanes) * a.pages * gpp;
    // Threads past the end still take part in the query-staging barrier.
    const bool active = gid < total;
    const uint64_t gclamp = active ? gid : total - 1;
    const uint32_t cg = uint32_t(gclamp % gpp);
    const uint64_t rest = gclamp / gpp;
    const uint32_t page = uint32_t(rest % a.pages);
    const uint32_t lane = uint32_t(rest / a.pages);
    const uint32_t c0 = cg * CPL;
    uint16_t hb[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float mean[8];
    uint32_t sbad = kOperandOk;

    // FUSE with q_stage: the workgroup stages its first lane's query rows in
    // LDS.  The first kQueryPrefetch elements per thread are loaded here,
    // ahead of the key stream, and reach LDS after it, so neither the stream
    // nor the epilogue waits on a query round trip.
    // Packed fp16 rows of up to 4096 elements take two 16-byte loads per
    // thread (qvec); other queries kQueryPrefetch single elements (qraw).
    constexpr uint32_t kQueryPrefetch = 16, kQueryVec = 2 * (256 / BS);
    uint32_t qraw[kQueryPrefetch];
    u32x4 qvec[kQueryVec];
    uint32_t staged_lane = 0xffffffffu, nq = 0;
    bool qv = false;
    if (FUSE && a.q_stage) {
        staged_lane = uint32_t((uint64_t(block) * BS / gpp) / a.pages);
        nq = a.q.rows * a.q.qheads * a.q.dim;
        qv = a.q.packed16 && nq <= BS * 8 * kQueryVec;
        if (qv) {
            const u32x4 *qp = reinterpret_cast<const u32x4 *>(a.q.data + staged_lane * a.q.lane_stride);
#pragma unroll
            for (uint32_t j = 0; j < kQueryVec; ++j) qvec[j] = qp[min(threadIdx.x + BS * j, nq / 8 - 1)];
        } else {
#pragma unroll
            for (uint32_t j = 0; j < kQueryPrefetch; ++j) {
                const uint32_t i = min(threadIdx.x + BS * j, nq - 1);  // in bounds; extras unused
                qraw[j] = load_raw(query_elem(a.q, staged_lane, i), a.q.scalar);
            }
        }
    }

    if (!active) {
        // nothing to summarize; stays for the barrier below
    } else if constexpr (SRC == kSrcSummary) {
        const u32x4 v = *reinterpret_cast<const u32x4 *>(
            a.src + lane * a.src_lane_stride + (uint64_t(page) * a.width + c0) * 2);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            hb[2 * i] = uint16_t(v[i] & 0xffffu);
            hb[2 * i + 1] = uint16_t(v[i] >> 16);
        }
    } else {
        const uint64_t t0 = uint64_t(page) * a.page_tokens;
        const uint64_t left = a.tokens - t0;
        const uint32_t n = left < a.page_tokens ? uint32_t(left) : a.page_tokens;
        float acc[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
        if constexpr (SRC == kSrcKeysF16) {
            typedef typename F16Lane<CPL>::type V;
            // streaming loads for whole-CU workgroups (a large layer), the
            // default policy for the one-wave ones of a lone small layer
            constexpr int kF16Policy = BS == 256 ? kBufferNontemporal : 0;
            auto add_row = [&](const V v) {
#pragma unroll
                for (int i = 0; i < CPL / 2; ++i) {
                    const uint32_t w = lane_word<CPL>(v, i);
                    acc[2 * i] += h2f(uint16_t(w & 0xffffu));
                    acc[2 * i + 1] += h2f(uint16_t(w >> 16));
                }
            };
            const uint32_t row_bytes = a.width * 2;
            if (a.width % (kWave * CPL) == 0 && uint64_t(a.page_tokens) * row_bytes < (1ull << 32)) {
                // Every wave's lanes read one page (whole waves are active
                // or not): the page is one buffer resource, and a row's
                // offset is a scalar added to the lane's column, so a load
                // costs no vector address arithmetic.
                const uint32_t nu = __builtin_amdgcn_readfirstlane(n);
                const uint8_t *first = a.src + uint64_t(__builtin_amdgcn_readfirstlane(lane)) * a.src_lane_stride +
                                       uint64_t(__builtin_amdgcn_readfirstlane(page)) * a.page_tokens * row_bytes;
                const auto rs = buffer_rsrc(first, nu * row_bytes);
                const int col = int(c0 * 2);
                stream_rows<kF16RingRows<CPL>>(
                    nu,
                    [&](uint32_t t) {
                        const int soff = int(t * row_bytes);
                        if constexpr (CPL == 8)
                            return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b128(rs, col, soff, kF16Policy));
                        else if constexpr (CPL == 4)
                            return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b64(rs, col, soff, kF16Policy));
                        else
                            return V(__builtin_amdgcn_raw_buffer_load_b32(rs, col, soff, kF16Policy));
                    },
                    add_row);
            } else {
                const V *p = reinterpret_cast<const V *>(a.src + lane * a.src_lane_stride + (t0 * a.width + c0) * 2);
                const uint64_t stride = gpp;  // lane loads per token row
                stream_rows<kF16RingRows<CPL>>(
                    n, [&](uint32_t t) { return kF16Policy ? __builtin_nontemporal_load(p + t * stride) : p[t * stride]; },
                    add_row);
            }
        } else {
            // q8_0 rows: lane owns 8 codes (quarter s) of block b, and the
            // block's four lanes (one quad) read the dword-aligned 36 bytes
            // around its 34 with one 12-byte load each: lane s takes dwords
            // [2s, 2s+3) of the span.  Even blocks start on a dword (codes at
            // span byte 2+8s), odd blocks two bytes into one (span starts two
            // bytes early, codes at 4+8s).  The fp16 scale sits in lane 0's
            // first dword and reaches the others by a quad broadcast.
            const uint32_t row_bytes = (a.width >> 5) * kQ8Bytes;
            const uint8_t *base = a.src + lane * a.src_lane_stride + t0 * row_bytes;
            const uint32_t b = cg >> 2, s = cg & 3;
            const uint32_t span = ((b * kQ8Bytes) & ~3u) + 8 * s;
            const bool odd = (b & 1) != 0;
            auto load_row = [&](uint32_t t) {
                return __builtin_nontemporal_load(reinterpret_cast<const u32x3a *>(base + uint64_t(t) * row_bytes + span));
            };
            auto sum_row = [&](const u32x3 x) {
                const uint32_t lo = odd ? x[1] : __builtin_amdgcn_alignbyte(x[1], x[0], 2);
                const uint32_t hi = odd ? x[2] : __builtin_amdgcn_alignbyte(x[2], x[1], 2);
                const uint32_t dw = dpp::move<dpp::kQuadBcast0>(x[0]);
                add_q8x8(acc, lo, hi, h2f(uint16_t(odd ? dw >> 16 : dw & 0xffffu)));
            };
            stream_rows<kQ8Rows>(n, load_row, sum_row);
        }
        const float inv = 1.0f / float(n);
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            mean[i] = acc[i] * inv;
            const uint32_t e = recall16(mean[i], hb[i]);
            sbad = sbad ? sbad : e;
        }
    }

    // The staged query reaches LDS before this thread stores anything: a
    // wait for its loads placed after a store would also wait for the store.
    if (FUSE && a.q_stage && qv) {
        // a finite fp16 value passes the recall boundary unchanged
        uint32_t qbad = kOperandOk;
#pragma unroll
        for (uint32_t j = 0; j < kQueryVec; ++j) {
            const uint32_t i8 = threadIdx.x + BS * j;
            if (i8 < nq / 8) {
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const uint32_t e = qvec[j][w] & 0x7c007c00u;
                    if ((e & 0xffffu) == 0x7c00u || (e >> 16) == 0x7c00u) qbad = kOperandNonfinite;
                }
                *reinterpret_cast<u32x4 *>(q_lds + 8 * i8) = qvec[j];
            }
        }
        if (qbad) raise_operand(a.status, qbad, a.epoch);
    } else if (FUSE && a.q_stage) {
        const QueryArgs &q = a.q;
        {
            uint32_t qbad = kOperandOk;
#pragma unroll
            for (uint32_t j = 0; j < kQueryPrefetch; ++j) {
                const uint32_t i = threadIdx.x + BS * j;
                uint16_t qh = 0;
                const uint32_t e = recall16(raw_value(qraw[j], q.scalar), qh);
                if (i < nq) {
                    qbad = qbad ? qbad : e;
                    q_lds[i] = qh;
                }
            }
            // the rest, 16 loads in flight per pass
            for (uint32_t base = threadIdx.x + BS * kQueryPrefetch; base < nq; base += BS * kQueryPrefetch) {
#pragma unroll
                for (uint32_t j = 0; j < kQueryPrefetch; ++j)
                    qraw[j] = load_raw(query_elem(q, staged_lane, min(base + BS * j, nq - 1)), q.scalar);
#pragma unroll
                for (uint32_t j = 0; j < kQueryPrefetch; ++j) {
                    const uint32_t i = base + BS * j;
                    uint16_t qh = 0;
                    const uint32_t e = recall16(raw_value(qraw[j], q.scalar), qh);
                    if (i < nq) {
                        qbad = qbad ? qbad : e;
                        q_lds[i] = qh;
                    }
                }
            }
            if (qbad) raise_operand(a.status, qbad, a.epoch);
        }
    }

    if (FUSE && a.q_stage) lds_barrier();
    if (FUSE && active) {
        // Dot products over 8-channel groups, each summed in channel order,
        // then over the kv-head slice's groups by one pairwise tree whatever
        // CPL is: the logits are bit-identical to those of 8-channel lanes
        // and of the stack's softmax-side logits.  With narrower lanes the
        // G = 8/CPL lanes of a group each gather its 8 means by quad DPP
        // broadcasts and compute its sums.
        constexpr int G = 8 / CPL;
        const QueryArgs &q = a.q;
        const uint32_t c8 = c0 & ~7u;  // the group's first channel
        const uint32_t kvh = c8 / q.dim, d0 = c8 % q.dim;
        const uint32_t group = q.qheads / q.kvheads;
        const int lph = int(q.dim >> 3);  // 8-channel groups per kv-head slice
        uint32_t w8[4];
        {
            uint32_t mine[CPL / 2];
#pragma unroll
            for (int i = 0; i < CPL / 2; ++i) mine[i] = uint32_t(hb[2 * i]) | (uint32_t(hb[2 * i + 1]) << 16);
            if constexpr (G == 1) {
#pragma unroll
                for (int i = 0; i < 4; ++i) w8[i] = mine[i];
            } else if constexpr (G == 2) {
                // quad_perm [g, g, 2+g, 2+g]: every lane reads lane g of its pair
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    w8[i] = dpp::move<0xA0>(mine[i]);
                    w8[2 + i] = dpp::move<0xF5>(mine[i]);
                }
            } else {
                // quad_perm [g, g, g, g]
                w8[0] = dpp::move<0x00>(mine[0]);
                w8[1] = dpp::move<0x55>(mine[0]);
                w8[2] = dpp::move<0xAA>(mine[0]);
                w8[3] = dpp::move<0xFF>(mine[0]);
            }
        }
        double m[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            m[2 * i] = double(h2f(uint16_t(w8[i] & 0xffffu)));
            m[2 * i + 1] = double(h2f(uint16_t(w8[i] >> 16)));
        }
        uint32_t bad = kOperandOk;
        const bool from_lds = lane == staged_lane;
        const bool writer = (cg & uint32_t(G * lph - 1)) == 0;
        // Four heads of the kv-head's group at a time (the last pass repeats
        // the group's last head and does not store it), so their loads and
        // cross-lane sums overlap.
        for (uint32_t r = 0; r < q.rows; ++r) {
            for (uint32_t h0 = 0; h0 < group; h0 += 4) {
                double part[4];
#pragma unroll
                for (uint32_t u = 0; u < 4; ++u) {
                    const uint32_t h = kvh * group + min(h0 + u, group - 1);
                    part[u] = 0.0;
                    if (from_lds) {
                        const u32x4 v = *reinterpret_cast<const u32x4 *>(q_lds + (r * q.qheads + h) * q.dim + d0);
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            part[u] = fma(double(h2f(uint16_t(v[i] & 0xffffu))), m[2 * i], part[u]);
                            part[u] = fma(double(h2f(uint16_t(v[i] >> 16))), m[2 * i + 1], part[u]);
                        }
                    } else {
                        const uint8_t *qp = q.data + lane * q.lane_stride + r * q.row_stride +
                                            h * q.head_stride + d0 * q.dim_stride;
#pragma unroll
                        for (int i = 0; i < 8; ++i) {
                            uint16_t qb = 0;
                            const uint32_t e = recall16(load_scalar(qp + i * q.dim_stride, q.scalar), qb);
                            bad = bad ? bad : e;
                            // fp16 x fp16 is exact in binary64: fma == multiply-then-add.
                            part[u] = fma(double(h2f(qb)), m[i], part[u]);
                        }
                    }
                }
#pragma unroll
                for (uint32_t u = 0; u < 4; ++u) part[u] = spread_group_sum<G>(part[u], lph);
#pragma unroll
                for (uint32_t u = 0; u < 4; ++u)
                    if (writer && h0 + u < group)
                        a.logits[((uint64_t(lane) * q.rows + r) * q.qheads + kvh * group + h0 + u) * a.pages + page] =
                            part[u] * q.scale;
            }
        }
        if (bad) raise_operand(a.status, bad, a.epoch);
    }

    // Summary stores last: nothing after them reuses their registers, so no
    // wait for their completion lands inside the fused epilogue.
    if (active && SRC != kSrcSummary) {
        const uint64_t out = (uint64_t(lane) * a.pages + page) * a.width + c0;
        if (a.means) {
            if constexpr (CPL == 2) {
                *reinterpret_cast<float2 *>(a.means + out) = make_float2(mean[0], mean[1]);
            } else {
                float4 *m4 = reinterpret_cast<float4 *>(a.means + out);
                m4[0] = make_float4(mean[0], mean[1], mean[2], mean[3]);
                if constexpr (CPL == 8) m4[1] = make_float4(mean[4], mean[5], mean[6], mean[7]);
            }
        }
        if (sbad) raise_operand(a.status, sbad, a.epoch);
        if (a.summaries) {
            typedef typename F16Lane<CPL>::type V;
            V v;
            if constexpr (CPL == 2) {
                v = uint32_t(hb[0]) | (uint32_t(hb[1]) << 16);
            } else {
#pragma unroll
                for (int i = 0; i < CPL / 2; ++i) v[i] = uint32_t(hb[2 * i]) | (uint32_t(hb[2 * i + 1]) << 16);
            }
            *reinterpret_cast<V *>(a.summaries + out) = v;
        }
    }
}

template <int SRC, bool FUSE, int BS, int CPL = 8>
__global__ __launch_bounds__(BS) void k_summary(SummaryArgs a) {
    summary_block<SRC, FUSE, BS, CPL>(a, blockIdx.x, q_lds_buf);
}

// ---------------------------------------------------------------------------
// Query rows -> packed fp16 operands (pack_current_query, page_softmax.cu:137-153,
// with the recall_fp16 boundary of graph_recall.cpp:364).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_pack_query(PackQueryArgs a) {
    const QueryArgs &q = a.q;
    const uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x;
    const uint64_t per_lane = uint64_t(q.rows) * q.qheads * q.dim;
    if (i >= per_lane * a.lanes) return;
    const uint32_t lane = uint32_t(i / per_lane);
    const uint64_t j = i % per_lane;
    const uint32_t d = uint32_t(j % q.dim), h = uint32_t((j / q.dim) % q.qheads),
                   r = uint32_t(j / (uint64_t(q.dim) * q.qheads));
    uint16_t hb = 0;
    const uint32_t e = recall16(load_scalar(q.data + lane * q.lane_stride + r * q.row_stride +
                                                h * q.head_stride + d * q.dim_stride, q.scalar), hb);
    if (e) raise_operand(a.status, e, a.epoch);
    a.out[i] = hb;
}

// ---------------------------------------------------------------------------
// Batched multi-row scoring on the matrix cores: per (lane, kv-head) the
// logits block Q_g[M = rows*group][D] x S_g^T[D][pages] with
// v_mfma_f64_16x16x4f64 (binary64 operands, exact fp16 products).
// Operand lanes: A[m = l%16][k = l/16], B[k = l/16][n = l%16];
// output register i of lane l is C[l/16 + 4i][l%16].  Lane l feeds the
// contiguous k-range [(l/16)*D/4, (l/16+1)*D/4) of both operands.
// One wave per 16-page tile; workgroups of four waves.
// ---------------------------------------------------------------------------
// KS: the k-range per lane group (head_dim / 4) at compile time for
// head_dim 64, 128 and 256 (0: at run time).  Each lane's operand halves are
// loaded unconditionally (clamped rows and pages, zeroed after), the page
// operand once for all row tiles, so no load waits behind another.
template <int KS>
__device__ __forceinline__ void logits_mfma_wave(const MfmaLogitsArgs &a) {
    const uint32_t wave = threadIdx.x >> 6, l = threadIdx.x & 63;
    const uint32_t n0 = (blockIdx.x * 4 + wave) * 16;
    const uint32_t g = blockIdx.y, lane = blockIdx.z;
    if (n0 >= a.pages) return;  // wave-uniform
    const uint32_t group = a.qheads / a.kvheads;
    const uint32_t M = a.rows * group;
    const uint32_t ks = KS > 0 ? uint32_t(KS) : a.dim >> 2;
    const uint32_t col = l & 15, kq = l >> 4;
    const uint32_t page = n0 + col;
    const bool pvalid = page < a.pages;
    const uint32_t width = a.kvheads * a.dim;
    const uint16_t *brow = a.summaries + (uint64_t(lane) * a.pages + (pvalid ? page : 0)) * width +
                           g * a.dim + kq * ks;
    constexpr int R = KS > 0 ? KS : 1;
    uint16_t bh[R];
    if (KS > 0) {
#pragma unroll
        for (int s = 0; s < R; ++s) bh[s] = brow[s];
    }
    for (uint32_t m0 = 0; m0 < M; m0 += 16) {
        const uint32_t m = m0 + col;
        const bool mvalid = m < M;
        const uint32_t mr = mvalid ? m : M - 1;
        const uint32_t r = mr / group, hh = mr % group;
        const uint16_t *arow = a.qpack + ((uint64_t(lane) * a.rows + r) * a.qheads + g * group + hh) * a.dim +
                               kq * ks;
        f64x4 acc = {0.0, 0.0, 0.0, 0.0};
        if (KS > 0) {
            uint16_t ah[R];
#pragma unroll
            for (int s = 0; s < R; ++s) ah[s] = arow[s];
#pragma unroll
            for (int s = 0; s < R; ++s) {
                const double av = mvalid ? double(h2f(ah[s])) : 0.0;
                const double bv = pvalid ? double(h2f(bh[s])) : 0.0;
                acc = __builtin_amdgcn_mfma_f64_16x16x4f64(av, bv, acc, 0, 0, 0);
            }
        } else {
            for (uint32_t s = 0; s < ks; ++s) {
                const uint16_t ahs = arow[s], bhs = brow[s];
                const double av = mvalid ? double(h2f(ahs)) : 0.0;
                const double bv = pvalid ? double(h2f(bhs)) : 0.0;
                acc = __builtin_amdgcn_mfma_f64_16x16x4f64(av, bv, acc, 0, 0, 0);
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t mo = m0 + kq + 4 * i;
            if (mo < M && pvalid) {
                const uint32_t ro = mo / group, ho = mo % group;
                a.logits[((uint64_t(lane) * a.rows + ro) * a.qheads + g * group + ho) * a.pages + page] =
                    acc[i] * a.scale;
            }
        }
    }
}

__global__ __launch_bounds__(256) void k_logits_mfma(MfmaLogitsArgs a) {
    switch (a.dim) {
    case 64: logits_mfma_wave<16>(a); break;
    case 128: logits_mfma_wave<32>(a); break;
    case 256: logits_mfma_wave<64>(a); break;
    default: logits_mfma_wave<0>(a); break;
    }
}

// ---------------------------------------------------------------------------
// Page softmax + head aggregation + top-k in one launch
// (graph_recall.cpp:362-394, kvmem_store.cpp:418-451).
//
// One workgroup per softmax unit of a lane -- a (row, q-head) for Mean, a
// (row, kv-head group) for Max and MaxLogit -- turns its logits into the
// unit's aggregation terms, written over the unit's first logits row:
//   Mean      t_j = p_j / w,                   p = softmax_j(logit_j)
//   Max       t_j = (g_j / sum_j g_j) / w,     g_j = max_h p_{h,j}
//   MaxLogit  t_j = softmax_j(max_h logit_{h,j}) / w
// with w = active layers x q-heads (Mean) or x kv-heads (group rules), the
// two divisions in the reference's order.  Masked pages get probability 0.
// The lane's last unit to finish (a device-scope counter; no workgroup ever
// waits for another) adds the terms in the reference's row order,
// scores_j (+)= sum_i t_{i,j}, and selects.  Exponentials, sums and
// quotients are binary64.
// ---------------------------------------------------------------------------
// Wave-synchronous LDS: orders this wave's LDS accesses before the ones that
// follow (lanes of one wave read what other lanes of it wrote).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}


constexpr uint32_t kTailLdsPages = 7680;  // keys of up to this many pages stay in LDS (<= 64 KiB padded)

// Registers: value i of a lane is page j = l + 64*i.
template <int NPL>
__device__ __forceinline__ void wave_softmax_regs(double (&v)[NPL], const bool (&on)[NPL]) {
    double m = -INFINITY;
#pragma unroll
    for (int i = 0; i < NPL; ++i) m = on[i] ? fmax(m, v[i]) : m;
    m = wave_max(m);
    double s = 0.0;
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
        v[i] = on[i] ? exp(v[i] - m) : 0.0;
        s += v[i];
    }
    s = wave_sum(s);
#pragma unroll
    for (int i = 0; i < NPL; ++i) v[i] = s > 0.0 ? v[i] / s : 0.0;
}

// Logits rows of q-heads [h0, h0 + nh) (nh <= 4, one kv-head's) for query
// row r of `lane`, computed from the stored fp16 summaries into rows
// dst + hh*pages: LDS, or global memory at device scope.  The wave's lanes
// split like the fused summary epilogue's (dim/8 lanes per page, 8 dims
// each, the same cross-lane sum), so the values are bit-identical to the
// fused path's.  Pages are shared among `waves` waves (this one is `wave`).
template <bool LDS, int LPH>
__device__ __forceinline__ void logits_rows_t(const SelectArgs &a, uint32_t lane, uint32_t r, uint32_t h0, uint32_t nh,
                                              uint32_t wave, uint32_t waves, double *dst) {
    const QueryArgs &q = a.q;
    const uint32_t lph = LPH > 0 ? uint32_t(LPH) : q.dim >> 3;
    const uint32_t l = threadIdx.x & 63, ppw = kWave / lph;
    const uint32_t k = l % lph, sub = l / lph;
    const uint32_t group = q.qheads / q.kvheads, kvh = h0 / group, W = q.kvheads * q.dim, n = a.pages;
    const double scale = q.scale;
    // all four heads are computed (past nh: repeats of the last), nh stored.
    // The 32 query values are loaded together (one 16-byte load per head
    // for packed fp16), the format chosen once outside the loads, and only
    // then converted: a per-element format choice compiles to a wait per load.
    double qd[4][8];
    uint32_t raw[4][8];
    uint32_t bad = kOperandOk;
    const uint8_t *qrow = q.data + lane * q.lane_stride + r * q.row_stride + 8 * k * q.dim_stride;
    auto head_at = [&](uint32_t hh) { return qrow + (h0 + min(hh, nh - 1)) * q.head_stride; };
    if (q.packed16) {
#pragma unroll
        for (uint32_t hh = 0; hh < 4; ++hh) {
            const u32x4 v = *reinterpret_cast<const u32x4 *>(head_at(hh));
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                raw[hh][2 * i] = v[i] & 0xffffu;
                raw[hh][2 * i + 1] = v[i] >> 16;
            }
        }
    } else if (q.scalar == kScalarF32) {
#pragma unroll
        for (uint32_t hh = 0; hh < 4; ++hh)
#pragma unroll
            for (int i = 0; i < 8; ++i)
                raw[hh][i] = *reinterpret_cast<const uint32_t *>(head_at(hh) + i * q.dim_stride);
    } else {
#pragma unroll
        for (uint32_t hh = 0; hh < 4; ++hh)
#pragma unroll
            for (int i = 0; i < 8; ++i)
                raw[hh][i] = *reinterpret_cast<const uint16_t *>(head_at(hh) + i * q.dim_stride);
    }
#pragma unroll
    for (uint32_t hh = 0; hh < 4; ++hh) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            uint16_t qb = 0;
            const uint32_t e = recall16(raw_value(raw[hh][i], q.scalar), qb);
            bad = bad ? bad : e;
            qd[hh][i] = double(h2f(qb));
        }
    }
    if (bad) raise_operand(a.status, bad, a.epoch);
    const uint16_t *S = a.summaries + uint64_t(lane) * n * W + kvh * q.dim + 8 * k;
    constexpr uint32_t U = 8;
    const uint32_t step = ppw * waves;
    for (uint32_t base = wave * ppw + sub; base < n + sub; base += step * U) {
        u32x4 x[U];
#pragma unroll
        for (uint32_t u = 0; u < U; ++u)
            x[u] = *reinterpret_cast<const u32x4 *>(S + uint64_t(min(base + u * step, n - 1)) * W);
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) {
            const uint32_t j = base + u * step;
            double m[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                m[2 * i] = double(h2f(uint16_t(x[u][i] & 0xffffu)));
                m[2 * i + 1] = double(h2f(uint16_t(x[u][i] >> 16)));
            }
            double part[4];
#pragma unroll
            for (uint32_t hh = 0; hh < 4; ++hh) {
                part[hh] = 0.0;
#pragma unroll
                for (int i = 0; i < 8; ++i) part[hh] = fma(qd[hh][i], m[i], part[hh]);
            }
#pragma unroll
            for (uint32_t hh = 0; hh < 4; ++hh) part[hh] = group_sum(part[hh], int(lph));
            if (k == 0 && j < n) {
#pragma unroll
                for (uint32_t hh = 0; hh < 4; ++hh) {
                    if (hh < nh) {
                        if (LDS) dst[uint64_t(hh) * n + j] = part[hh] * scale;
                        else store_device(dst + uint64_t(hh) * n + j, part[hh] * scale);
                    }
                }
            }
        }
    }
}

// Lanes per page fixed at compile time for head_dim 64, 128 and 256, so the
// cross-lane sums are straight DPP sequences.
template <bool LDS>
__device__ __forceinline__ void logits_rows(const SelectArgs &a, uint32_t lane, uint32_t r, uint32_t h0, uint32_t nh,
                                            uint32_t wave, uint32_t waves, double *dst) {
    switch (a.q.dim) {
    case 64: logits_rows_t<LDS, 8>(a, lane, r, h0, nh, wave, waves, dst); break;
    case 128: logits_rows_t<LDS, 16>(a, lane, r, h0, nh, wave, waves, dst); break;
    case 256: logits_rows_t<LDS, 32>(a, lane, r, h0, nh, wave, waves, dst); break;
    default: logits_rows_t<LDS, 0>(a, lane, r, h0, nh, wave, waves, dst); break;
    }
}

template <bool LDS>
__device__ __forceinline__ void units_logits(const SelectArgs &a, uint32_t lane, uint32_t u0, uint32_t u1,
                                             double *rows) {
    const uint32_t wave = threadIdx.x >> 6, waves = blockDim.x >> 6, n = a.pages;
    const uint32_t group = a.qheads / a.kvheads;
    double *lane_rows = a.logits + uint64_t(lane) * a.rows * a.qheads * n;
    if (a.aggregation == kAggMean) {
        for (uint32_t u = u0; u < u1;) {
            const uint32_t r = u / a.qheads, h = u % a.qheads, kv_end = (h / group + 1) * group;
            const uint32_t nh = min(min(4u, u1 - u), kv_end - h);
            logits_rows<LDS>(a, lane, r, h, nh, wave, waves, LDS ? rows + uint64_t(u - u0) * n : lane_rows + uint64_t(u) * n);
            u += nh;
        }
        return;
    }
    for (uint32_t u = u0; u < u1; ++u) {
        const uint32_t r = u / a.kvheads, g = u % a.kvheads;
        for (uint32_t h0 = g * group; h0 < (g + 1) * group; h0 += 4)
            logits_rows<LDS>(a, lane, r, h0, min(4u, (g + 1) * group - h0), wave, waves,
                             LDS ? rows + (uint64_t(u - u0) * group + (h0 - g * group)) * n
                                 : lane_rows + (uint64_t(r) * a.qheads + h0) * n);
    }
}

// LDS logits rows of a softmax workgroup (layer stacks, up to 1024 pages):
// one row per unit for Mean, the group's rows per unit otherwise, if they fit.
constexpr uint32_t kProbsLdsBytes = 64 * 1024;
__host__ __device__ constexpr uint32_t probs_lds_rows(uint32_t aggregation, uint32_t group) {
    return kUnitsPerBlock * (aggregation == kAggMean ? 1 : group);
}
__host__ __device__ constexpr bool probs_lds_fits(uint32_t aggregation, uint32_t group, uint32_t pages) {
    return pages <= 1024 && uint64_t(probs_lds_rows(aggregation, group)) * pages * 8 <= kProbsLdsBytes;
}
extern __shared__ __align__(16) double probs_lds[];

// One unit by one wave, rows of up to 64*NPL pages held in registers.
// lout: the unit's terms go to this LDS row instead of over its logits.
template <int NPL>
__device__ __forceinline__ void unit_terms_regs(const SelectArgs &a, double *lane_base, uint32_t unit,
                                                const double *lrows, double *lout = nullptr) {
    // Loads are unconditional with indices clamped into the row (values past
    // the row are read, then dropped): a load behind a per-lane branch would
    // wait for itself before the next one issues.
    const uint32_t n = a.pages, l = threadIdx.x & 63;
    auto at = [&](uint32_t i) { return min(l + uint32_t(i) * kWave, n - 1); };
    bool on[NPL];
    uint8_t mv[NPL];
    if (a.mask) {
#pragma unroll
        for (int i = 0; i < NPL; ++i) mv[i] = a.mask[at(i) >> a.mask_shift];
    } else {
#pragma unroll
        for (int i = 0; i < NPL; ++i) mv[i] = 1;
    }
#pragma unroll
    for (int i = 0; i < NPL; ++i) on[i] = l + i * kWave < n && mv[i];
    double t[NPL];
    double *out;
    // logits computed in this launch: from this workgroup's LDS rows
    // (`lrows`: the unit's first row) or at device scope
    auto logit = [&](const double *row, uint32_t j) { return a.summaries ? load_device(row + j) : row[j]; };
    auto lds_row = [&](uint32_t hh) { return lrows + uint64_t(hh) * n; };
    // The group rules take the group's heads HP at a time (short rows), the
    // chunk's loads in flight together and its heads' reductions in one
    // straight run.  Past the group's end a chunk repeats its last head,
    // which changes neither a max nor a max of softmaxes.
    constexpr uint32_t HP = NPL <= 4 ? 4 : 1;
    auto load_heads = [&](const double *first, uint32_t h0, uint32_t group, double (&x)[HP][NPL]) {
#pragma unroll
        for (uint32_t k = 0; k < HP; ++k) {
            const uint32_t hh = min(h0 + k, group - 1);
#pragma unroll
            for (int i = 0; i < NPL; ++i) x[k][i] = lrows ? lds_row(hh)[at(i)] : logit(first + uint64_t(hh) * n, at(i));
        }
    };
    if (a.aggregation == kAggMean) {
        out = lane_base + uint64_t(unit) * n;
#pragma unroll
        for (int i = 0; i < NPL; ++i) {
            const double x = lrows ? lrows[at(i)] : logit(out, at(i));
            t[i] = on[i] ? x : 0.0;
        }
        wave_softmax_regs(t, on);
#pragma unroll
        for (int i = 0; i < NPL; ++i) t[i] = t[i] / a.weight;
    } else {
        const uint32_t group = a.qheads / a.kvheads;
        const uint32_t r = unit / a.kvheads, g = unit % a.kvheads;
        out = lane_base + (uint64_t(r) * a.qheads + uint64_t(g) * group) * n;
        if (a.aggregation == kAggMax) {
            double gm[NPL];
#pragma unroll
            for (int i = 0; i < NPL; ++i) gm[i] = 0.0;
            for (uint32_t h0 = 0; h0 < group; h0 += HP) {
                double x[HP][NPL];
                load_heads(out, h0, group, x);
#pragma unroll
                for (uint32_t k = 0; k < HP; ++k) {
#pragma unroll
                    for (int i = 0; i < NPL; ++i) x[k][i] = on[i] ? x[k][i] : 0.0;
                    wave_softmax_regs(x[k], on);
                }
#pragma unroll
                for (uint32_t k = 0; k < HP; ++k)
#pragma unroll
                    for (int i = 0; i < NPL; ++i) gm[i] = x[k][i] > gm[i] ? x[k][i] : gm[i];
            }
            double mass = 0.0;
#pragma unroll
            for (int i = 0; i < NPL; ++i) mass += gm[i];
            mass = wave_sum(mass);
#pragma unroll
            for (int i = 0; i < NPL; ++i) t[i] = (mass > 0.0 ? gm[i] / mass : 0.0) / a.weight;
        } else {
#pragma unroll
            for (int i = 0; i < NPL; ++i) t[i] = -INFINITY;
            for (uint32_t h0 = 0; h0 < group; h0 += HP) {
                double x[HP][NPL];
                load_heads(out, h0, group, x);
#pragma unroll
                for (uint32_t k = 0; k < HP; ++k)
#pragma unroll
                    for (int i = 0; i < NPL; ++i) t[i] = fmax(t[i], on[i] ? x[k][i] : -INFINITY);
            }
            wave_softmax_regs(t, on);
#pragma unroll
            for (int i = 0; i < NPL; ++i) t[i] = t[i] / a.weight;
        }
    }
    // every lane rewrites only pages it read itself
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
        const uint32_t j = l + i * kWave;
        if (j < n) {
            if (lout) lout[j] = t[i];
            else store_device(out + j, t[i]);
        }
    }
}

// Workgroup-wide max and sum (waves by DPP, then the four wave results in
// wave order through LDS).
__device__ __forceinline__ double block_max(double v) {
    __shared__ double part[4];
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
    lds_barrier();
    v = fmax(fmax(part[0], part[1]), fmax(part[2], part[3]));
    lds_barrier();
    return v;
}
__device__ __forceinline__ double block_sum(double v) {
    __shared__ double part[4];
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
    lds_barrier();
    v = ((part[0] + part[1]) + part[2]) + part[3];
    lds_barrier();
    return v;
}

// Rows longer than 1024 pages: one unit per 256-thread workgroup, passes
// over memory in tiles of 16 values per thread (4096 pages per tile), the
// tile's loads in flight together; per-head statistics first, then one pass
// per page.  Thread t touches only pages j == t (mod 256).  Values this
// thread stored are re-read at device scope.
// Tile `base` of a long `row` for thread l (256 threads, 16 values per
// thread, the tile's loads in flight together; indices clamped into the row).
// own: values this thread stored itself, re-read at device scope.
constexpr int kLongTile = 16;
constexpr uint32_t kLongThreads = 256;
__device__ __forceinline__ void long_row_load(const SelectArgs &a, const double *row, bool own, uint32_t base,
                                              double (&x)[kLongTile], bool (&on)[kLongTile]) {
    const uint32_t n = a.pages, l = threadIdx.x;
    if (a.mask) {
        uint8_t mk[kLongTile];
#pragma unroll
        for (int i = 0; i < kLongTile; ++i) {
            const uint32_t j = min(base + l + i * kLongThreads, n - 1);
            x[i] = own || a.summaries ? load_device(row + j) : row[j];
            mk[i] = a.mask[j >> a.mask_shift];
        }
#pragma unroll
        for (int i = 0; i < kLongTile; ++i) on[i] = mk[i] != 0;
    } else {
#pragma unroll
        for (int i = 0; i < kLongTile; ++i) {
            const uint32_t j = min(base + l + i * kLongThreads, n - 1);
            x[i] = own || a.summaries ? load_device(row + j) : row[j];
            on[i] = true;
        }
    }
}
// f(j, value, on) over thread l's pages j < n of a long `row`, tile by tile.
template <class F>
__device__ __forceinline__ void long_row_tiles(const SelectArgs &a, const double *row, bool own, F f) {
    const uint32_t n = a.pages, l = threadIdx.x;
    for (uint32_t base = 0; base < n; base += kLongThreads * kLongTile) {
        double x[kLongTile];
        bool on[kLongTile];
        long_row_load(a, row, own, base, x, on);
#pragma unroll
        for (int i = 0; i < kLongTile; ++i) {
            const uint32_t j = base + l + i * kLongThreads;
            if (j < n) f(j, x[i], on[i]);
        }
    }
}
// A long row's softmax statistics: its max m and sum s of exp(x - m) over
// unmasked pages (per-thread partials in tile order, then block_max/sum).
// KEEP: a row of one tile keeps its values in registers between the two
// passes instead of loading them again (same values, same results; the
// layer stack's softmax workgroups reload, which measured faster there).
template <bool KEEP = false>
__device__ __forceinline__ void long_row_stats(const SelectArgs &a, const double *row, bool own, double &m,
                                               double &s) {
    double mm = -INFINITY, ss = 0.0;
    if (KEEP && a.pages <= kLongThreads * kLongTile) {
        const uint32_t l = threadIdx.x;
        double x[kLongTile];
        bool on[kLongTile];
        long_row_load(a, row, own, 0, x, on);
#pragma unroll
        for (int i = 0; i < kLongTile; ++i)
            if (l + i * kLongThreads < a.pages) mm = on[i] ? fmax(mm, x[i]) : mm;
        m = block_max(mm);
#pragma unroll
        for (int i = 0; i < kLongTile; ++i)
            if (l + i * kLongThreads < a.pages) ss += on[i] ? exp(x[i] - m) : 0.0;
        s = block_sum(ss);
        return;
    }
    long_row_tiles(a, row, own, [&](uint32_t, double x, bool on) { mm = on ? fmax(mm, x) : mm; });
    m = block_max(mm);
    long_row_tiles(a, row, own, [&](uint32_t, double x, bool on) { ss += on ? exp(x - m) : 0.0; });
    s = block_sum(ss);
}
// A page's probability from its row's statistics.
__device__ __forceinline__ double row_prob(double x, double m, double s) { return s > 0.0 ? exp(x - m) / s : 0.0; }

__device__ __forceinline__ void unit_terms_loop(const SelectArgs &a, double *lane_base, uint32_t unit) {
    constexpr int T = 16;
    constexpr uint32_t S = 256;  // threads per unit
    const uint32_t n = a.pages, l = threadIdx.x;
    auto tiles = [&](const double *row, bool own, auto f) { long_row_tiles(a, row, own, f); };
    auto stats = [&](const double *row, bool own, double &m, double &s) { long_row_stats(a, row, own, m, s); };
    auto prob = [&](double x, double m, double s) { return row_prob(x, m, s); };
    if (a.aggregation == kAggMean) {
        double *row = lane_base + uint64_t(unit) * n;
        double m, s;
        stats(row, false, m, s);
        tiles(row, false, [&](uint32_t j, double x, bool on) {
            store_device(row + j, (on ? prob(x, m, s) : 0.0) / a.weight);
        });
        return;
    }
    const uint32_t group = a.qheads / a.kvheads;
    const uint32_t r = unit / a.kvheads, g = unit % a.kvheads;
    double *out = lane_base + (uint64_t(r) * a.qheads + uint64_t(g) * group) * n;
    // g_j = max over the group's rows of value(hh, j), into out[j]
    auto group_max = [&](bool own, double init, auto value) {
        double total = 0.0;
        for (uint32_t base = 0; base < n; base += S * T) {
            double gm[T];
#pragma unroll
            for (int i = 0; i < T; ++i) gm[i] = init;
            for (uint32_t hh = 0; hh < group; ++hh) {
                const double *row = out + uint64_t(hh) * n;
                double x[T];
#pragma unroll
                for (int i = 0; i < T; ++i) {
                    const uint32_t j = min(base + l + i * S, n - 1);
                    x[i] = own || a.summaries ? load_device(row + j) : row[j];
                }
#pragma unroll
                for (int i = 0; i < T; ++i) gm[i] = value(gm[i], x[i]);
            }
#pragma unroll
            for (int i = 0; i < T; ++i) {
                const uint32_t j = base + l + i * S;
                if (j < n) {
                    store_device(out + j, gm[i]);
                    total += gm[i];
                }
            }
        }
        return total;
    };
    if (a.aggregation == kAggMax) {
        // each head's probabilities over its own row, then g_j into the first
        for (uint32_t hh = 0; hh < group; ++hh) {
            double *row = out + uint64_t(hh) * n;
            double m, s;
            stats(row, false, m, s);
            tiles(row, false, [&](uint32_t j, double x, bool on) { store_device(row + j, on ? prob(x, m, s) : 0.0); });
        }
        // masked pages hold probability 0 in every row, so their g_j is 0
        const double mass = block_sum(group_max(true, 0.0, [](double gm, double p) { return p > gm ? p : gm; }));
        tiles(out, true, [&](uint32_t j, double x, bool) {
            store_device(out + j, (mass > 0.0 ? x / mass : 0.0) / a.weight);
        });
    } else {
        group_max(false, -INFINITY, [](double gm, double x) { return fmax(gm, x); });
        double m, s;
        stats(out, true, m, s);
        tiles(out, true, [&](uint32_t j, double x, bool on) {
            store_device(out + j, (on ? prob(x, m, s) : 0.0) / a.weight);
        });
    }
}

// ---------------------------------------------------------------------------
// Selection restates KvMemStore::pick_scored_blocks
// (kvmem/src/host/kvmem_store.cpp:418-451): mandatory pages first, then the
// best (score desc, id by tie rule) up to k, output in ascending id order.
// The k-th best of the order-preserving 64-bit keys is found by an MSB
// radix select (8-bit digits in an LDS histogram, the leading bits common to
// every candidate skipped, early exit once the boundary bucket is taken
// whole), then the pages are compacted in id order with scans; ties at the
// threshold are resolved by rank among equal keys in id order.  One wave
// does it for up to 1024 pages (no workgroup barriers), the whole
// workgroup for longer rows.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t order_key(double v) {
    uint64_t u = uint64_t(__double_as_longlong(v));
    if ((u << 1) == 0) u = 0;  // -0.0 ranks equal to +0.0
    return (u >> 63) ? ~u : (u | 0x8000000000000000ull);
}

// Pages kept before the ranking (mandatory / fixed pages): a bitmap of the
// lane's pages in LDS, bit j of word j/32 for page j; null when there are
// none.
struct FixedPages {
    const uint32_t *bits;
    __device__ __forceinline__ bool at(uint32_t j) const { return bits && (bits[j >> 5] >> (j & 31) & 1u); }
};

// Dynamic LDS of the selection kernels: the lane's keys (pages <= kTailLdsPages).
extern __shared__ __align__(16) uint64_t tail_keys[];
// LDS slot of page j's key: one pad slot after every 16 keys, so the 16-key
// chunks that consecutive threads walk start in different banks (unpadded,
// a wave's key reads fall on two banks).
__host__ __device__ constexpr uint32_t key_slot(uint32_t j) { return j + (j >> 4); }

// One wave finds, in a complete 256-bin digit histogram, the digit `d`
// holding the `remaining`-th best key, the rank `rem` within it and its
// count `cnt` (every lane gets them).
__device__ __forceinline__ void radix_find(const uint32_t *hist, uint32_t remaining, uint32_t &d, uint32_t &rem,
                                           uint32_t &cnt) {
    const uint32_t l = threadIdx.x & 63;
    // lane l covers digits 255-4l .. 252-4l, highest first
    const uint32_t c0 = hist[255 - 4 * l], c1 = hist[254 - 4 * l], c2 = hist[253 - 4 * l],
                   c3 = hist[252 - 4 * l];
    const uint32_t tot = c0 + c1 + c2 + c3;
    const uint32_t incl = wave_inclusive_scan(tot);
    const uint32_t excl = incl - tot;
    const uint64_t owner = __ballot(excl < remaining && remaining <= incl);
    const int b = __ffsll((long long)owner) - 1;  // the one lane holding the boundary
    rem = remaining - excl;
    if (rem <= c0) {
        d = 255 - 4 * l; cnt = c0;
    } else if (rem <= c0 + c1) {
        rem -= c0; d = 254 - 4 * l; cnt = c1;
    } else if (rem <= c0 + c1 + c2) {
        rem -= c0 + c1; d = 253 - 4 * l; cnt = c2;
    } else {
        rem -= c0 + c1 + c2; d = 252 - 4 * l; cnt = c3;
    }
    d = wave_bcast(d, b);
    rem = wave_bcast(rem, b);
    cnt = wave_bcast(cnt, b);
}

// Histogram pass of the radix select: counts keys matching `prefix` above
// bit pos+8 by their digit at `pos`, then finds the digit holding the
// `remaining`-th best.  `for_each_key(f)` calls f(key) for this lane's
// candidate keys.  Returns false when the whole boundary bucket is taken.
template <class ForEach>
__device__ __forceinline__ bool radix_pass(ForEach for_each_key, uint32_t *hist, int pos, uint64_t &prefix,
                                           uint32_t &remaining) {
    const uint32_t l = threadIdx.x & 63;
    const uint64_t hi_mask = pos + 8 >= 64 ? 0ull : ~0ull << (pos + 8);
#pragma unroll
    for (int q = 0; q < 4; ++q) hist[l + 64 * q] = 0;
    wave_lds_sync();
    const uint64_t want = prefix & hi_mask;
    for_each_key([&](uint64_t key) {
        if ((key & hi_mask) == want) atomicAdd(&hist[(key >> pos) & 255u], 1u);
    });
    wave_lds_sync();
    uint32_t d, rem, cnt;
    radix_find(hist, remaining, d, rem, cnt);
    wave_lds_sync();
    prefix |= uint64_t(d) << pos;
    remaining = rem;
    return rem != cnt;
}

// Threshold search.  After it, with HT = thresh >> shift:
//   (key >> shift) >  HT            selected
//   (key >> shift) == HT && bucket  selected (the boundary bucket holds
//                                   exactly the remaining count)
//   key == thresh && !bucket        the first/last `remaining` equal keys
//                                   by id (tie rule), shift == 0
struct Threshold {
    uint64_t thresh = 0;
    uint32_t remaining = 0, shift = 0;
    bool bucket = false;
    __device__ __forceinline__ int cls(uint64_t key) const {  // 2 taken, 1 tied at the threshold, 0 not
        const uint64_t hk = key >> shift, ht = thresh >> shift;
        return (hk > ht || (hk == ht && bucket)) ? 2 : (hk == ht ? 1 : 0);
    }
};

// Equal-key ranks [lo, hi) taken by the tie rule among eq_total keys tied at
// the threshold (in id order).
__device__ __forceinline__ void tie_window(const SelectArgs &a, uint32_t remaining, uint32_t eq_total, uint32_t &lo,
                                          uint32_t &hi) {
    if (a.tie_higher_first) {
        lo = remaining >= eq_total ? 0u : eq_total - remaining;
        hi = eq_total;
    } else {
        lo = 0;
        hi = remaining < eq_total ? remaining : eq_total;
    }
}

// Selection of one lane by one wave, for up to 16*64 pages.  Lane l owns the
// id chunk [l*C, l*C + C), C = ceil(pages/64) <= 16, and holds its keys in
// registers.
__device__ __forceinline__ void wave_select(const SelectArgs &a, uint32_t lane, uint32_t n, bool lds, const double *sc,
                                            uint32_t *hist, const FixedPages fx, uint32_t n_fixed) {
    constexpr int R = 16;
    const uint32_t l = threadIdx.x & 63;
    const uint32_t C = (n + kWave - 1) / kWave;
    const uint32_t j0 = min(n, l * C), j1 = min(n, j0 + C);
    auto load_key = [&](uint32_t j) -> uint64_t { return lds ? tail_keys[key_slot(j)] : order_key(sc[j]); };
    uint64_t kr[R];
    uint32_t cand_bits = 0;  // chunk entries that are candidates
#pragma unroll
    for (int c = 0; c < R; ++c) {
        const uint32_t j = j0 + c;
        const bool in = j < j1;
        kr[c] = in ? load_key(j) : 0;
        if (in && !fx.at(j)) cand_bits |= 1u << c;
    }
    auto for_each_key = [&](auto f) {
#pragma unroll
        for (int c = 0; c < R; ++c)
            if (cand_bits >> c & 1u) f(kr[c]);
    };
    const uint32_t n_cand = n - n_fixed;
    const uint32_t k_eff = a.k - n_fixed;  // the tail checked n_fixed <= k
    Threshold t;
    if (k_eff == 0) {
        t.thresh = ~0ull;  // nothing ranks
        t.bucket = true;
    } else if (k_eff >= n_cand) {
        t.bucket = true;   // every candidate
    } else {
        uint64_t and_all = ~0ull, or_all = 0;
        for_each_key([&](uint64_t key) {
            and_all &= key;
            or_all |= key;
        });
        and_all = wave_and(and_all);
        or_all = wave_or(or_all);
        const uint64_t diff = and_all ^ or_all;
        t.remaining = k_eff;
        if (diff == 0) {  // all candidates equal: the tie rule decides
            t.thresh = and_all;
        } else {
            const int top = 63 - __clzll(diff);
            uint64_t prefix = and_all & ~((2ull << top) - 1);  // the common high bits
            for (int pos = top / 8 * 8;; pos -= 8) {
                if (!radix_pass(for_each_key, hist, pos, prefix, t.remaining)) {
                    t.bucket = true;  // the whole boundary bucket is selected
                    t.shift = uint32_t(pos);
                    break;
                }
                if (pos == 0) break;  // full key: the tie rule picks among equals
            }
            t.thresh = prefix;
        }
    }

    // Compaction in id order.
    uint32_t n_take = 0, n_eq = 0;
#pragma unroll
    for (int c = 0; c < R; ++c) {
        if (j0 + c >= j1) continue;
        const int k = (cand_bits >> c & 1u) ? t.cls(kr[c]) : 2;
        n_take += k == 2;
        n_eq += k == 1;
    }
    const uint32_t eq_incl = wave_inclusive_scan(n_eq);
    const uint32_t eq_base = eq_incl - n_eq;
    const uint32_t eq_total = wave_bcast(eq_incl, kWave - 1);
    uint32_t lo, hi;
    tie_window(a, t.remaining, eq_total, lo, hi);
    const uint32_t eq_lo = max(lo, eq_base), eq_hi = min(hi, eq_base + n_eq);
    n_take += eq_hi > eq_lo ? eq_hi - eq_lo : 0u;
    const uint32_t take_incl = wave_inclusive_scan(n_take);
    const uint32_t total = wave_bcast(take_incl, kWave - 1);
    uint32_t o = take_incl - n_take;
    uint32_t rank = eq_base;
    uint32_t *out = a.selected + uint64_t(lane) * a.k;
    auto emit = [&](uint32_t j, int k) {
        bool take = k == 2;
        if (k == 1) {
            take = rank >= lo && rank < hi;
            ++rank;
        }
        if (take && o < a.k) out[o++] = j;
    };
#pragma unroll
    for (int c = 0; c < R; ++c)
        if (j0 + c < j1) emit(j0 + c, (cand_bits >> c & 1u) ? t.cls(kr[c]) : 2);
    if (l == 0) a.count[lane] = min(total, a.k);
}

// Selection of one lane by the whole workgroup (256 threads), for rows
// longer than 1024 pages: the same threshold search and compaction as
// wave_select, with thread t owning the id chunk [t*C, t*C + C),
// C = ceil(pages/256), keys read 8 at a time from LDS or the scores.
__device__ __forceinline__ void wg_select(const SelectArgs &a, uint32_t lane, uint32_t n, bool lds, const double *sc,
                                          uint32_t *hist, const FixedPages fx, uint32_t n_fixed) {
    constexpr uint32_t B = 256, W = B / kWave;
    __shared__ uint64_t s_red[2][W];
    __shared__ uint32_t s_ctl[3];
    __shared__ uint32_t s_scan[W];
    const uint32_t tid = threadIdx.x, w = tid / kWave, l = tid % kWave;
    const uint32_t C = (n + B - 1) / B;
    const uint32_t j0 = min(n, tid * C), j1 = min(n, j0 + C);
    auto load_key = [&](uint32_t j) -> uint64_t { return lds ? tail_keys[key_slot(j)] : order_key(sc[j]); };
    // chunks of up to 64 ids (rows up to 16384 pages) keep their fixed
    // pages in a register mask; longer chunks test the LDS bitmap per pass
    const bool masked = C <= 64;
    uint64_t mand_bits = 0;
    if (masked && fx.bits)
        for (uint32_t j = j0; j < j1; ++j)
            if (fx.at(j)) mand_bits |= 1ull << (j - j0);
    // chunks of up to RK keys in LDS (every row that keeps its keys there)
    // are read into registers once; the passes below walk the registers
    constexpr uint32_t RK = 32;
    const bool in_regs = lds && C <= RK;
    uint64_t kr[RK];
    if (in_regs) {
#pragma unroll
        for (uint32_t c = 0; c < RK; ++c) kr[c] = j0 + c < j1 ? tail_keys[key_slot(j0 + c)] : 0;
    }
    // f(j, key, candidate) over this thread's chunk in id order
    auto chunk = [&](auto f) {
        if (in_regs) {
#pragma unroll
            for (uint32_t c = 0; c < RK; ++c)
                if (j0 + c < j1) f(j0 + c, kr[c], !(mand_bits >> c & 1ull));
            return;
        }
        for (uint32_t b = j0; b < j1; b += 8) {
            uint64_t kk[8];
#pragma unroll
            for (uint32_t u = 0; u < 8; ++u) kk[u] = load_key(min(b + u, j1 - 1));
#pragma unroll
            for (uint32_t u = 0; u < 8; ++u) {
                const uint32_t j = b + u;
                if (j < j1) f(j, kk[u], masked ? !(mand_bits >> (j - j0) & 1ull) : !fx.at(j));
            }
        }
    };
    // exclusive prefix and total of v over the workgroup in thread order
    auto scan = [&](uint32_t v, uint32_t &excl, uint32_t &total) {
        const uint32_t incl = wave_inclusive_scan(v);
        if (l == kWave - 1) s_scan[w] = incl;
        lds_barrier();
        uint32_t before = 0, tot = 0;
#pragma unroll
        for (uint32_t i = 0; i < W; ++i) {
            const uint32_t x = s_scan[i];
            before += i < w ? x : 0u;
            tot += x;
        }
        lds_barrier();
        excl = before + incl - v;
        total = tot;
    };
    const uint32_t n_cand = n - n_fixed;
    const uint32_t k_eff = a.k - n_fixed;
    Threshold t;
    if (k_eff == 0) {
        t.thresh = ~0ull;
        t.bucket = true;
    } else if (k_eff >= n_cand) {
        t.bucket = true;
    } else {
        uint64_t and_all = ~0ull, or_all = 0;
        chunk([&](uint32_t, uint64_t key, bool cand) {
            if (cand) {
                and_all &= key;
                or_all |= key;
            }
        });
        and_all = wave_and(and_all);
        or_all = wave_or(or_all);
        if (l == 0) {
            s_red[0][w] = and_all;
            s_red[1][w] = or_all;
        }
        lds_barrier();
#pragma unroll
        for (uint32_t i = 0; i < W; ++i) {
            and_all &= s_red[0][i];
            or_all |= s_red[1][i];
        }
        const uint64_t diff = and_all ^ or_all;
        t.remaining = k_eff;
        if (diff == 0) {
            t.thresh = and_all;
        } else {
            const int top = 63 - __clzll(diff);
            uint64_t prefix = and_all & ~((2ull << top) - 1);
            for (int pos = top / 8 * 8;; pos -= 8) {
                const uint64_t hi_mask = pos + 8 >= 64 ? 0ull : ~0ull << (pos + 8);
                const uint64_t want = prefix & hi_mask;
                hist[tid] = 0;
                lds_barrier();
                chunk([&](uint32_t, uint64_t key, bool cand) {
                    if (cand && (key & hi_mask) == want) atomicAdd(&hist[(key >> pos) & 255u], 1u);
                });
                lds_barrier();
                if (w == 0) {
                    uint32_t d, rem, cnt;
                    radix_find(hist, t.remaining, d, rem, cnt);
                    if (l == 0) {
                        s_ctl[0] = d;
                        s_ctl[1] = rem;
                        s_ctl[2] = cnt;
                    }
                }
                lds_barrier();
                const uint32_t d = s_ctl[0], rem = s_ctl[1], cnt = s_ctl[2];
                lds_barrier();  // hist and s_ctl are rewritten by the next pass
                prefix |= uint64_t(d) << pos;
                t.remaining = rem;
                if (rem == cnt) {
                    t.bucket = true;
                    t.shift = uint32_t(pos);
                    break;
                }
                if (pos == 0) break;
            }
            t.thresh = prefix;
        }
    }

    uint32_t n_take = 0, n_eq = 0;
    chunk([&](uint32_t, uint64_t key, bool cand) {
        const int k = cand ? t.cls(key) : 2;
        n_take += k == 2;
        n_eq += k == 1;
    });
    uint32_t eq_base, eq_total;
    scan(n_eq, eq_base, eq_total);
    uint32_t lo, hi;
    tie_window(a, t.remaining, eq_total, lo, hi);
    const uint32_t eq_lo = max(lo, eq_base), eq_hi = min(hi, eq_base + n_eq);
    n_take += eq_hi > eq_lo ? eq_hi - eq_lo : 0u;
    uint32_t o, total;
    scan(n_take, o, total);
    uint32_t rank = eq_base;
    uint32_t *out = a.selected + uint64_t(lane) * a.k;
    chunk([&](uint32_t j, uint64_t key, bool cand) {
        const int k = cand ? t.cls(key) : 2;
        bool take = k == 2;
        if (k == 1) {
            take = rank >= lo && rank < hi;
            ++rank;
        }
        if (take && o < a.k) out[o++] = j;
    });
    if (tid == 0) a.count[lane] = min(total, a.k);
}

// ---------------------------------------------------------------------------
// Graph propagation (propagate_query_scores, kvmem/src/host/graph_recall.cpp:
// 494-552) and LRFU preview (LrfuHistory::preview, kvmem/include/kvmem/
// lrfu.hpp:57-79), one lane per 1024-thread workgroup.
//
// Propagation is a sum of transfers: node i gives (total * seed_i) * w to
// node j and loses as much, seed_i = max(0, raw_i) / total, w = alpha/4 times
// the span coefficient to each adjacent node and (alpha/2 * mass) / den over
// its graph row -- the reference's expressions, operand for operand.  The
// reference applies the transfers one by one in its hash map's order; here
// each is rounded to an integer count of 2^(e-62) units (2^e > total) and
// the counts are added (adjacent ones by the receiving page itself, graph
// edges by LDS integer atomics), so the result does not depend on the order
// and differs from the reference's by a few units of the total's last place.
// The LRFU threshold is the score of a given ascending rank, found by the
// same radix select as the page selection (order-preserving keys, ±0 equal).
// Contraction stays off: every product and sum is rounded on its own, as in
// the reference's host build.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int64_t graph_units(double delta, int shift) {
    return static_cast<int64_t>(rint(ldexp(delta, shift)));
}

// Thread t owns the pages [t*C, t*C + C), C = ceil(pages/1024) <= 8, and
// holds them with one page either side in registers; graph rows go one per
// thread with their first four edges loaded in one round trip.
constexpr uint32_t kGraphThreads = 1024, kGraphChunk = kGraphMaxPages / kGraphThreads;

__global__ __launch_bounds__(1024) void k_graph_lrfu(GraphLrfuArgs a) {
#pragma clang fp contract(off)
    constexpr uint32_t B = kGraphThreads, W = B / kWave, CH = kGraphChunk, EB = 4;
    __shared__ double s_sum[W];
    __shared__ uint32_t s_cnt[W], s_bad[W];
    __shared__ uint64_t s_red[2][W];
    __shared__ uint32_t hist[256];
    __shared__ uint32_t s_ctl[2];
    const uint32_t tid = threadIdx.x, w = tid / kWave, l = tid % kWave;
    const uint32_t lane = a.lane0 + blockIdx.x, n = a.pages;
    const GraphLane g = a.graph[blockIdx.x];
    double *sc = a.scores + uint64_t(lane) * n;
    const uint8_t *mk = a.mask ? a.mask + uint64_t(lane) * n : nullptr;
    int64_t *net = reinterpret_cast<int64_t *>(tail_keys);  // transfer units per page
    const uint32_t C = (n + B - 1) / B;
    const uint32_t j0 = min(n, tid * C), cnt = min(n, j0 + C) - j0;
    auto node = [&](uint32_t j) { return j < n && (!mk || mk[j]); };
    // workgroup OR of a flag (every thread gets it)
    auto any = [&](uint32_t flag) {
        flag = wave_max(flag);
        if (l == 0) s_bad[w] = flag;
        lds_barrier();
        uint32_t r = 0;
#pragma unroll
        for (uint32_t i = 0; i < W; ++i) r |= s_bad[i];
        lds_barrier();
        return r != 0;
    };
    // pages j0-1 .. j0+CH: ve[c] is page j0-1+c (0 outside the lane)
    double ve[CH + 2];
    bool ne[CH + 2];
#pragma unroll
    for (uint32_t c = 0; c < CH + 2; ++c) {
        const uint32_t p = j0 + c - 1;  // wraps to UINT32_MAX for j0 = 0, c = 0
        const bool in = (c >= 1 && c <= cnt) || ((c == 0 || c == cnt + 1) && a.propagate && cnt && p < n);
        ve[c] = in ? sc[p] : 0.;
        ne[c] = in && (!mk || mk[p]);
    }
    double v[CH];  // this thread's values: the scores, then the propagated ones
    uint32_t bad = 0;
#pragma unroll
    for (uint32_t c = 0; c < CH; ++c) {
        v[c] = ve[c + 1];
        if (c < cnt) bad |= !__builtin_isfinite(v[c]);
    }

    if (a.propagate) {
        double part = 0;
        uint32_t nodes = 0;
#pragma unroll
        for (uint32_t c = 0; c < CH; ++c)
            if (c < cnt && ne[c + 1]) {
                ++nodes;
                part += 0. < v[c] ? v[c] : 0.;
            }
        part = wave_sum(part);
        nodes = wave_sum(nodes);
        bad = wave_max(bad);
        if (l == 0) {
            s_sum[w] = part;
            s_cnt[w] = nodes;
            s_bad[w] = bad;
        }
        lds_barrier();
        double total = 0;
        nodes = 0;
        bad = 0;
#pragma unroll
        for (uint32_t i = 0; i < W; ++i) {
            total += s_sum[i];
            nodes += s_cnt[i];
            bad |= s_bad[i];
        }
        lds_barrier();
        if (bad || !__builtin_isfinite(total)) {
            if (tid == 0) raise_status(a.status, kStatusScores, a.epoch);
            return;
        }
        if (nodes > 1 && total != 0. && a.alpha != 0.) {
            int e;
            (void)frexp(total, &e);  // total < 2^e
            const int shift = 62 - e;
            const double wn = a.alpha * .25, wr = a.alpha * .5;
            auto base = [&](double r) {
                const double seed = (0. < r ? r : 0.) / total;
                return total * seed;
            };
            uint32_t gbad = 0;
            // span coefficient of the pair (j0-1+c, j0+c), c = 0..CH
            double pw[CH + 1];
#pragma unroll
            for (uint32_t c = 0; c < CH + 1; ++c) {
                const uint32_t i = j0 + c;
                const bool in = g.neighbor_weight && i >= 1 && i < n && c <= cnt;
                pw[c] = in ? g.neighbor_weight[i - 1] : 1.;
            }
            // adjacent pages: each page sums what it receives and gives
#pragma unroll
            for (uint32_t c = 0; c < CH; ++c) {
                if (c >= cnt) continue;
                int64_t q = 0;
                if (ne[c + 1]) {
                    const double bj = base(ve[c + 1]);
                    if (ne[c]) {
                        gbad |= !(pw[c] >= 0. && pw[c] <= 1.);
                        const double wt = wn * pw[c];
                        q += graph_units(base(ve[c]) * wt, shift) - graph_units(bj * wt, shift);
                    }
                    if (ne[c + 2]) {
                        gbad |= !(pw[c + 1] >= 0. && pw[c + 1] <= 1.);
                        const double wt = wn * pw[c + 1];
                        q += graph_units(base(ve[c + 2]) * wt, shift) - graph_units(bj * wt, shift);
                    }
                }
                net[j0 + c] = q;
            }
            lds_barrier();
            // graph rows: one thread per row, its edges in order
            for (uint32_t r = tid; r < g.n_rows; r += B) {
                const uint32_t src = g.row_source[r];
                const uint32_t e0 = g.row_begin[r], e1 = g.row_begin[r + 1];
                if (e0 > e1 || e1 > g.n_edges) {
                    gbad = 1;
                    continue;
                }
                if (!node(src)) continue;
                const double rs = sc[src];
                double m4[EB];
                uint32_t t4[EB];
#pragma unroll
                for (uint32_t u = 0; u < EB; ++u) {
                    const bool in = e0 + u < e1;
                    m4[u] = in ? g.edge_mass[e0 + u] : 0.;
                    t4[u] = in ? g.edge_target[e0 + u] : src;
                }
                bool n4[EB];
                double den = 0;
#pragma unroll
                for (uint32_t u = 0; u < EB; ++u) {
                    n4[u] = t4[u] != src && node(t4[u]);
                    if (e0 + u < e1) gbad |= !(m4[u] >= 0. && m4[u] <= __DBL_MAX__);
                    if (n4[u]) den += m4[u];
                }
                for (uint32_t e = e0 + EB; e < e1; ++e) {
                    const double m = g.edge_mass[e];
                    gbad |= !(m >= 0. && m <= __DBL_MAX__);
                    const uint32_t t = g.edge_target[e];
                    if (t != src && node(t)) den += m;
                }
                if (!(den != 0.)) continue;
                const double bs = base(rs);
                if (bs == 0.) continue;
                uint64_t given = 0;
                auto give = [&](uint32_t t, double m) {
                    const double wt = wr * m / den;
                    const uint64_t q = uint64_t(graph_units(bs * wt, shift));
                    atomicAdd(reinterpret_cast<unsigned long long *>(net + t), (unsigned long long)q);
                    given += q;
                };
#pragma unroll
                for (uint32_t u = 0; u < EB; ++u)
                    if (n4[u]) give(t4[u], m4[u]);
                for (uint32_t e = e0 + EB; e < e1; ++e) {
                    const uint32_t t = g.edge_target[e];
                    if (t != src && node(t)) give(t, g.edge_mass[e]);
                }
                atomicAdd(reinterpret_cast<unsigned long long *>(net + src), (unsigned long long)(0ull - given));
            }
            lds_barrier();
            const double slack = 1e-12 * (1. < total ? total : 1.);
#pragma unroll
            for (uint32_t c = 0; c < CH; ++c) {
                if (c >= cnt) continue;
                const double r = v[c];
                const int64_t q = net[j0 + c];
                double o = q ? r + ldexp(double(q), -shift) : r;
                const double resid = r < 0. ? r : 0.;
                gbad |= !(o >= resid - slack);
                v[c] = resid < o ? o : resid;
            }
            if (any(gbad)) {
                if (tid == 0) raise_status(a.status, kStatusGraph, a.epoch);
                return;
            }
#pragma unroll
            for (uint32_t c = 0; c < CH; ++c)
                if (c < cnt) sc[j0 + c] = v[c];
        }
    } else if (any(bad)) {
        if (tid == 0) raise_status(a.status, kStatusScores, a.epoch);
        return;
    }
    if (!a.lrfu) return;

    // LRFU: threshold key of ascending rank `rank`, i.e. the (n - rank)-th
    // largest, by a radix select over the registers
    uint64_t thr = 0;
    if (a.gate) {
        uint64_t and_all = ~0ull, or_all = 0;
#pragma unroll
        for (uint32_t c = 0; c < CH; ++c)
            if (c < cnt) {
                const uint64_t k = order_key(v[c]);
                and_all &= k;
                or_all |= k;
            }
        and_all = wave_and(and_all);
        or_all = wave_or(or_all);
        if (l == 0) {
            s_red[0][w] = and_all;
            s_red[1][w] = or_all;
        }
        lds_barrier();
#pragma unroll
        for (uint32_t i = 0; i < W; ++i) {
            and_all &= s_red[0][i];
            or_all |= s_red[1][i];
        }
        const uint64_t diff = and_all ^ or_all;
        uint64_t prefix = and_all;
        if (diff) {
            const int top = 63 - __clzll(diff);
            prefix = and_all & ~((2ull << top) - 1);
            uint32_t remaining = n - a.rank;
            for (int pos = top / 8 * 8;; pos -= 8) {
                const uint64_t hi_mask = pos + 8 >= 64 ? 0ull : ~0ull << (pos + 8);
                const uint64_t want = prefix & hi_mask;
                if (tid < 256) hist[tid] = 0;
                lds_barrier();
#pragma unroll
                for (uint32_t c = 0; c < CH; ++c)
                    if (c < cnt) {
                        const uint64_t k = order_key(v[c]);
                        if ((k & hi_mask) == want) atomicAdd(&hist[(k >> pos) & 255u], 1u);
                    }
                lds_barrier();
                if (w == 0) {
                    uint32_t d, rem, cn;
                    radix_find(hist, remaining, d, rem, cn);
                    if (l == 0) {
                        s_ctl[0] = d;
                        s_ctl[1] = rem;
                    }
                }
                lds_barrier();
                prefix |= uint64_t(s_ctl[0]) << pos;
                remaining = s_ctl[1];
                lds_barrier();  // hist and s_ctl are rewritten by the next pass
                if (pos == 0) break;
            }
        }
        thr = prefix;
    }
    const double lam = a.lambda;
    const double *h = a.history ? a.history + uint64_t(lane) * a.history_pages : nullptr;
    double *cd = a.candidate + uint64_t(lane) * n;
    double hv[CH];
#pragma unroll
    for (uint32_t c = 0; c < CH; ++c) hv[c] = (c < cnt && j0 + c < a.history_pages) ? h[j0 + c] : 0.;
#pragma unroll
    for (uint32_t c = 0; c < CH; ++c) {
        if (c >= cnt) continue;
        const double x = v[c];
        const double kept = (!a.gate || order_key(x) >= thr) ? x : (0. < x ? 0. : x);
        cd[j0 + c] = lam * hv[c] + kept;
    }
}

// Aggregation (optional) by the whole workgroup (up to 1024 threads), then
// selection by its first wave (up to 1024 pages) or by 256 threads.  Keys go
// to LDS when the lane's pages fit.  LT: the terms are in LDS (`lterms`,
// unit i's row at i*cols), not over the logits in memory.  SCORES: this
// launch's workgroups wrote the scores (aggregated already); they are read
// at device scope.
template <bool LT = false, bool SCORES = false>
__device__ __forceinline__ void lane_tail(const SelectArgs &a, uint32_t lane, const double *lterms = nullptr) {
    __shared__ uint32_t hist[256];
    __shared__ uint32_t fixed_small[kTailLdsPages / 32];  // the fixed-page bitmap of short rows
    __shared__ uint32_t s_fixed[16];
    const uint32_t tid = threadIdx.x, B = blockDim.x;
    const uint32_t cols = a.pages;         // softmax columns (half pages when folding)
    const uint32_t n = select_pages(a);    // pages scored and selected
    const bool lds = n <= kTailLdsPages;
    double *sc = a.scores + uint64_t(lane) * n;
    // Fixed pages (the inline list and the device list) go to a bitmap: LDS
    // beside the keys for short rows, the dynamic LDS (not holding keys) for
    // longer ones.  Cleared here, set once the sums below are done.
    const bool has_fixed = a.do_select && (a.n_mandatory || a.n_fixed);
    uint32_t *fbits = lds ? fixed_small : reinterpret_cast<uint32_t *>(tail_keys);
    const uint32_t words = (n + 31) / 32;
    if (has_fixed)
        for (uint32_t w = tid; w < words; w += B) fbits[w] = 0;
    // the status of this call, read early so its latency overlaps the sums
    bool failed = a.do_select && tid < kWave && epoch_failed(a.status, a.epoch);

    int bad = 0;
    auto note = [&](uint32_t j, double v) {
        bad |= !__builtin_isfinite(v) || (!a.signed_scores && v < 0.0);
        if (lds) tail_keys[key_slot(j)] = order_key(v);
    };
    if (!SCORES && a.do_aggregate) {
        // Contributing rows in the reference's order: (row, head) for Mean,
        // (row, kv-head group) for the group rules.  Two columns per pass and
        // up to 32 rows of loads in flight; the additions stay in order.
        const uint32_t group = a.qheads / a.kvheads;
        const bool mean = a.aggregation == kAggMean;
        const uint32_t nrows = mean ? a.rows * a.qheads : a.rows * a.kvheads;
        const double *terms = a.logits + uint64_t(lane) * a.rows * a.qheads * cols;
        auto row_of = [&](uint32_t i) -> uint64_t {
            return mean ? i : uint64_t(i / a.kvheads) * a.qheads + (i % a.kvheads) * group;
        };
        // contributing row i's offset, and a term at an offset
        auto row_off = [&](uint32_t i) -> uint64_t { return (LT ? uint64_t(i) : row_of(i)) * cols; };
        auto term = [&](uint64_t o) -> double {
            if constexpr (LT) return lterms[o];
            else return load_device(terms + o);
        };
        // acc0 += column c0's terms, acc1 += column c1's (c1 is loaded even
        // when the caller drops acc1: the loads stay unconditional)
        auto sum_rows = [&](uint32_t c0, uint32_t c1, double &acc0, double &acc1) {
            uint32_t i = 0;
            for (; i + 32 <= nrows; i += 32) {
                double v0[32], v1[32];
#pragma unroll
                for (int u = 0; u < 32; ++u) {
                    const uint64_t o = row_off(i + u);
                    v0[u] = term(o + c0);
                    v1[u] = term(o + c1);
                }
#pragma unroll
                for (int u = 0; u < 32; ++u) {
                    acc0 += v0[u];
                    acc1 += v1[u];
                }
            }
            for (; i + 16 <= nrows; i += 16) {
                double v0[16], v1[16];
#pragma unroll
                for (int u = 0; u < 16; ++u) {
                    const uint64_t o = row_off(i + u);
                    v0[u] = term(o + c0);
                    v1[u] = term(o + c1);
                }
#pragma unroll
                for (int u = 0; u < 16; ++u) {
                    acc0 += v0[u];
                    acc1 += v1[u];
                }
            }
            for (; i + 8 <= nrows; i += 8) {
                double v0[8], v1[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const uint64_t o = row_off(i + u);
                    v0[u] = term(o + c0);
                    v1[u] = term(o + c1);
                }
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    acc0 += v0[u];
                    acc1 += v1[u];
                }
            }
            for (; i < nrows; ++i) {
                const uint64_t o = row_off(i);
                acc0 += term(o + c0);
                acc1 += term(o + c1);
            }
        };
        if (a.fold) {
            // a page's two half masses from zero, then folded
            // (layerwise_selection.cpp:64-72: left + right; :24-30: the max)
            for (uint32_t j = tid; j < n; j += B) {
                double left = 0.0, right = 0.0;
                sum_rows(2 * j, 2 * j + 1, left, right);
                double v = a.fold == kFoldSum ? left + right : (left < right ? right : left);
                if (a.accumulate) v = sc[j] + v;
                sc[j] = v;
                note(j, v);
            }
        } else if (nrows <= 16) {
            // four columns per pass, their rows' loads in flight together
            // (a long row takes a quarter of the round trips); each column's
            // rows are still added in order
            for (uint32_t j0 = tid; j0 < n; j0 += 4 * B) {
                uint32_t jj[4];
                double acc[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    jj[q] = min(j0 + q * B, n - 1);
                    acc[q] = a.accumulate && j0 + q * B < n ? sc[jj[q]] : 0.0;
                }
                double v[4][16];
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (uint32_t u = 0; u < 16; ++u)
                        v[q][u] = term(row_off(min(u, nrows - 1)) + jj[q]);
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (uint32_t u = 0; u < 16; ++u)
                        if (u < nrows) acc[q] += v[q][u];
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    if (j0 + q * B < n) {
                        sc[jj[q]] = acc[q];
                        note(jj[q], acc[q]);
                    }
            }
        } else {
            for (uint32_t j0 = tid; j0 < n; j0 += 2 * B) {
                const uint32_t j1 = j0 + B;
                const bool has1 = j1 < n;
                double acc0 = a.accumulate ? sc[j0] : 0.0;
                double acc1 = has1 && a.accumulate ? sc[j1] : 0.0;
                sum_rows(j0, has1 ? j1 : j0, acc0, acc1);  // acc1 is dropped when !has1
                sc[j0] = acc0;
                note(j0, acc0);
                if (has1) {
                    sc[j1] = acc1;
                    note(j1, acc1);
                }
            }
        }
    } else {
        // 16 loads in flight per pass
        for (uint32_t j0 = tid; j0 < n; j0 += 16 * B) {
            double v[16];
#pragma unroll
            for (uint32_t u = 0; u < 16; ++u) {
                const uint32_t j = min(j0 + u * B, n - 1);
                v[u] = SCORES ? load_device(sc + j) : sc[j];
            }
#pragma unroll
            for (uint32_t u = 0; u < 16; ++u)
                if (j0 + u * B < n) note(j0 + u * B, v[u]);
        }
    }
    if (!a.do_select) return;
    if (has_fixed) {
        __syncthreads();  // the bitmap is clear
        for (uint32_t i = tid; i < a.n_mandatory; i += B) {
            const uint32_t id = a.mandatory[i];
            if (id < n) atomicOr(&fbits[id >> 5], 1u << (id & 31));
        }
        for (uint32_t i = tid; i < a.n_fixed; i += B) {
            const uint32_t id = a.fixed[i];  // pages past the row are ignored
            if (id < n) atomicOr(&fbits[id >> 5], 1u << (id & 31));
        }
    }
    // Reject invalid scores (pick_scored_blocks, kvmem_store.cpp:425-426).
    bad = __syncthreads_or(bad);  // also publishes the LDS keys and the bitmap
    uint32_t n_fixed = 0;         // distinct fixed pages
    if (has_fixed) {
        uint32_t c = 0;
        for (uint32_t w = tid; w < words; w += B) c += __popc(fbits[w]);
        c = wave_sum(c);
        if ((tid & (kWave - 1)) == 0) s_fixed[tid / kWave] = c;
        __syncthreads();
        for (uint32_t w = 0; w < B / kWave; ++w) n_fixed += s_fixed[w];
    }
    const bool wide = n > 16 * kWave;
    if (wide) failed = __syncthreads_or(failed);
    else if (tid >= kWave) return;
    if (bad && tid == 0) raise_status(a.status, kStatusScores, a.epoch);
    // more fixed pages than the budget (pick_scored_blocks' required keep)
    const bool over = n_fixed > a.k;
    if (over && !bad && !failed && tid == 0) raise_status(a.status, kStatusBudget, a.epoch);
    if (bad || failed || over) {
        if (tid == 0) a.count[lane] = 0;
        return;
    }
    const FixedPages fx{has_fixed ? fbits : nullptr};
    if (wide)
        wg_select(a, lane, n, lds, sc, hist, fx, n_fixed);
    else
        wave_select(a, lane, n, lds, sc, hist, fx, n_fixed);
}

// Softmax units -> terms; the lane's last workgroup aggregates (+ selects).
// grid (ceil(units/4), lanes), 256 threads (a unit per wave); dynamic LDS:
// the tail's keys.
// LOGITS: a.summaries may ask for the logits to be computed here (layer
// stacks); k_probs always gets them given.
template <int NPL, bool LOGITS>
__device__ __forceinline__ void probs_block(const SelectArgs &a, uint32_t unit_block, uint32_t lane,
                                            uint32_t blocks_per_lane) {
    __shared__ uint32_t s_last;
    const uint32_t unit = NPL > 0 ? unit_block * kUnitsPerBlock + (threadIdx.x >> 6) : unit_block;
    double *lane_base = a.logits + uint64_t(lane) * a.rows * a.qheads * a.pages;
    const uint32_t group = a.qheads / a.kvheads;
    const bool lds_logits = LOGITS && a.summaries && NPL > 0 && probs_lds_fits(a.aggregation, group, a.pages);
    if (LOGITS && a.summaries) {
        // the logits of this workgroup's units first, by all its waves
        const uint32_t u0 = NPL > 0 ? unit_block * kUnitsPerBlock : unit_block;
        const uint32_t u1 = min(a.units, u0 + (NPL > 0 ? kUnitsPerBlock : 1));
        if (lds_logits) {
            units_logits<true>(a, lane, u0, u1, probs_lds);
        } else {
            units_logits<false>(a, lane, u0, u1, nullptr);
            wait_vmem();  // stored at device scope: complete, so visible to the reads below
        }
        __syncthreads();
    }
    if (unit < a.units) {
        const double *lrows = lds_logits ? probs_lds + uint64_t(threadIdx.x >> 6) * (a.aggregation == kAggMean ? 1 : group) *
                                                           a.pages
                                         : nullptr;
        if (NPL > 0)
            unit_terms_regs<NPL ? NPL : 1>(a, lane_base, unit, lrows);
        else
            unit_terms_loop(a, lane_base, unit);
    }
    // Publish this workgroup's terms (stored at device scope: complete once
    // every thread's stores are), then count it.  Only the lane's last
    // workgroup continues; its counter is back at zero for the next launch.
    wait_vmem();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t done = atomicAdd(a.counters + lane, 1u);
        s_last = done == blocks_per_lane - 1;
        if (s_last) atomicExch(a.counters + lane, 0u);
    }
    __syncthreads();
    if (!s_last) return;
    // the tail reads the terms and status words at device scope
    lane_tail(a, lane);
}

template <int NPL>
__global__ __launch_bounds__(256) void k_probs(SelectArgs a) {
    probs_block<NPL, false>(a, blockIdx.x, blockIdx.y, gridDim.x);
}

// Rows of up to kOnePages softmax columns with at most kOneUnits units: one
// workgroup per lane, a wave per unit, and the terms kept in LDS after the
// tail's keys, so no device-scope hand-off between workgroups (and no
// second round trip through memory) sits between the softmax and the tail.
constexpr uint32_t kOnePages = 512, kOneUnits = 8;
template <int NPL>
__global__ __launch_bounds__(kOneUnits * kWave) void k_probs_one(SelectArgs a) {
    const uint32_t lane = blockIdx.x, unit = threadIdx.x >> 6;
    double *lterms = reinterpret_cast<double *>(tail_keys + key_slot(select_pages(a)) + 1);
    if (unit < a.units)
        unit_terms_regs<NPL>(a, a.logits + uint64_t(lane) * a.rows * a.qheads * a.pages, unit, nullptr,
                             lterms + uint64_t(unit) * a.pages);
    lds_barrier();
    lane_tail<true>(a, lane, lterms);
}

// Long Mean rows (more than 1024 pages, no half-page fold) in two launches
// instead of k_probs' units-then-tail: the units' statistics, then page
// slices that sum their terms over the rows and a tail that selects.  The
// terms are never stored: each is recomputed from its row's statistics by
// the expression k_probs stores, and a page's terms are added in row order
// from the stored score or zero, as k_probs' tail adds them, so the scores
// are bit-identical to k_probs' (and to the layer stack's).
// k_unit_stats: grid (units, lanes), 256 threads.
__global__ __launch_bounds__(256) void k_unit_stats(SelectArgs a) {
    const uint32_t lane = blockIdx.y, unit = blockIdx.x;
    const double *row = a.logits + (uint64_t(lane) * a.rows * a.qheads + unit) * a.pages;
    double m, s;
    long_row_stats<true>(a, row, false, m, s);
    if (threadIdx.x == 0) {
        a.stats[(uint64_t(lane) * a.units + unit) * 2] = m;
        a.stats[(uint64_t(lane) * a.units + unit) * 2 + 1] = s;
    }
}

// k_mean_scores: grid (ceil(pages / kScorePages), lanes), 256 threads, a
// quad of lanes per page: lane q of a quad computes the terms of rows q,
// q + 4, ... (the exponentials and divisions, the bulk of the work) and the
// quad adds them in row order from quad broadcasts, so every lane holds the
// page's score.  The lane's last workgroup selects (dynamic LDS: the tail's
// keys).
constexpr uint32_t kScorePages = 64, kScoreRows = 4;  // pages per workgroup, rows per lane per pass
__device__ __forceinline__ double quad_lane(double v, uint32_t q) {
    switch (q) {
        case 0: return dpp::move<0x00>(v);
        case 1: return dpp::move<0x55>(v);
        case 2: return dpp::move<0xAA>(v);
        default: return dpp::move<0xFF>(v);
    }
}
__global__ __launch_bounds__(256) void k_mean_scores(SelectArgs a) {
    __shared__ uint32_t s_last;
    const uint32_t lane = blockIdx.y, n = a.pages, q = threadIdx.x & 3u;
    const double *logits = a.logits + uint64_t(lane) * a.rows * a.qheads * n;
    const double *st = a.stats + uint64_t(lane) * a.units * 2;
    double *sc = a.scores + uint64_t(lane) * n;
    const uint32_t j = blockIdx.x * kScorePages + (threadIdx.x >> 2), jc = min(j, n - 1);
    const bool on = !a.mask || a.mask[jc >> a.mask_shift];
    double acc = a.accumulate ? sc[jc] : 0.0;
    for (uint32_t u0 = 0; u0 < a.units; u0 += 4 * kScoreRows) {
        double x[kScoreRows], m[kScoreRows], s[kScoreRows], t[kScoreRows];
#pragma unroll
        for (uint32_t k = 0; k < kScoreRows; ++k) {
            const uint32_t u = min(u0 + 4 * k + q, a.units - 1);
            x[k] = logits[uint64_t(u) * n + jc];
            m[k] = st[2 * u];
            s[k] = st[2 * u + 1];
        }
#pragma unroll
        for (uint32_t k = 0; k < kScoreRows; ++k) t[k] = (on ? row_prob(x[k], m[k], s[k]) : 0.0) / a.weight;
#pragma unroll
        for (uint32_t k = 0; k < kScoreRows; ++k)
#pragma unroll
            for (uint32_t r = 0; r < 4; ++r) {
                const double v = quad_lane(t[k], r);
                if (u0 + 4 * k + r < a.units) acc += v;
            }
    }
    if (q == 0 && j < n) store_device(sc + j, acc);
    // Publish (stores complete at device scope), count; the last selects.
    wait_vmem();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t done = atomicAdd(a.counters + lane, 1u);
        s_last = done == gridDim.x - 1;
        if (s_last) atomicExch(a.counters + lane, 0u);
    }
    __syncthreads();
    if (!s_last) return;
    lane_tail<false, true>(a, lane);
}

// The summary workgroups of a key-history stack group: every layer of the
// group has the geometry of the first, so a thread owns the same 8 channels
// of the same page in each, and one ring of loads runs through the layers'
// rows back to back -- the next layer's first rows are in flight while this
// layer's last ones are summed, so a layer boundary costs no load latency.
// Sums restart at each layer's first row (binary32, token order, as in
// summary_block).

// Channels per summary lane of a key-history stack: fp16 keys whose pages
// a wave's 64 lanes of 4 channels cover whole (widths a multiple of 256,
// pages under 4 GiB) take 4, so twice the waves stream the same rows;
// otherwise 8.
__host__ __device__ inline uint32_t stack_cpl(int src, uint32_t width, uint32_t page_tokens) {
    return src == kSrcKeysF16 && width % 256 == 0 && (uint64_t(page_tokens) + 64) * width * 2 < (uint64_t(1) << 32)
               ? 4u
               : 8u;
}

// PAGED: every wave's 64 channel groups lie in one page (width a multiple of
// 512 channels) and a page spans less than 4 GiB.  Then the page and its
// rows are wave-uniform: each layer's page is read through a buffer
// resource that ends at the page's last row, a row's address is one add of
// a scalar row offset to the lane's column (no 64-bit address or clamp per
// lane), and the pad rows of a page's last chunk read zeros from the
// hardware, which add nothing (acc is never -0), so no row is masked and
// the chunk loop has no branch.
// Otherwise each lane keeps its own row pointer, clamped to the page's last
// row.
// CPL: channels per lane (stack_cpl: 4 for paged fp16 keys, else 8).
template <int SRC, bool PAGED, int CPL = 8>
__device__ __forceinline__ void stack_summaries(const StackGroupArgs &g, uint32_t block, uint32_t l0, uint32_t m) {
    static_assert(CPL == 8 || (SRC == kSrcKeysF16 && PAGED && CPL == 4), "4-channel lanes read paged fp16 keys");
    __builtin_amdgcn_s_setprio(2);
    const SummaryArgs &a = g.s[0];
    const uint32_t gpp = a.width / CPL;
    uint32_t cg, page, lane;
    if constexpr (PAGED) {
        const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x) >> 6;
        const uint64_t gid0 = uint64_t(block) * 256 + wave * 64;  // the wave's first channel group
        if (gid0 >= uint64_t(a.lanes) * a.pages * gpp) return;  // whole waves; no barriers follow
        const uint64_t rest = gid0 / gpp;
        cg = uint32_t(gid0 % gpp) + (threadIdx.x & 63u);
        page = uint32_t(rest % a.pages);
        lane = uint32_t(rest / a.pages);
    } else {
        const uint64_t gid = uint64_t(block) * 256 + threadIdx.x;
        if (gid >= uint64_t(a.lanes) * a.pages * gpp) return;  // no barriers follow
        const uint64_t rest = gid / gpp;
        cg = uint32_t(gid % gpp);
        page = uint32_t(rest % a.pages);
        lane = uint32_t(rest / a.pages);
    }
    const uint32_t c0 = cg * CPL;
    const uint64_t t0 = uint64_t(page) * a.page_tokens;
    const uint64_t tail = a.tokens - t0;
    const uint32_t n = tail < a.page_tokens ? uint32_t(tail) : a.page_tokens;
    // this thread's column in a row, and the row stride
    const uint32_t row_bytes = SRC == kSrcKeysF16 ? a.width * 2 : (a.width >> 5) * kQ8Bytes;
    const uint32_t b = cg >> 2, s = cg & 3;  // q8_0: block and quarter (see summary_block)
    const uint32_t col = SRC == kSrcKeysF16 ? c0 * 2 : ((b * kQ8Bytes) & ~3u) + 8 * s;
    const bool odd = (b & 1) != 0;
    // q8_0: the 8 codes sit at byte 2 (even block) or 4 (odd block) of the
    // lane's 12 bytes; one byte permutation per dword extracts them.
    const uint32_t code_sel = odd ? 0x07060504u : 0x05040302u;
    // per-layer fields, read with constant indices (entries past m are
    // never used); `first` is the page's first row in the lane's history
    const uint8_t *first[kStackGroup];
    float *means[kStackGroup];
    uint16_t *sums[kStackGroup];
    uint32_t epoch[kStackGroup];
#pragma unroll
    for (uint32_t i = 0; i < kStackGroup; ++i) {
        first[i] = g.s[i].src + lane * g.s[i].src_lane_stride + t0 * row_bytes + (PAGED ? 0 : col);
        means[i] = g.s[i].means;
        sums[i] = g.s[i].summaries;
        epoch[i] = g.s[i].epoch;
    }
    // layer i of this workgroup's part is layer l0 + i of the group
    auto pick = [l0](uint32_t i, auto v0, auto v1, auto v2, auto v3) {
        i += l0;
        return i == 1 ? v1 : i == 2 ? v2 : i == 3 ? v3 : v0;
    };
    auto layer_first = [&](uint32_t i) { return pick(i, first[0], first[1], first[2], first[3]); };
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
    auto finish = [&](uint32_t i) {
        float *mo = pick(i, means[0], means[1], means[2], means[3]);
        uint16_t *so = pick(i, sums[0], sums[1], sums[2], sums[3]);
        const float inv = 1.0f / float(n);
        float mean[8];
        uint16_t hb[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        uint32_t bad = kOperandOk;
#pragma unroll
        for (int k = 0; k < CPL; ++k) {
            mean[k] = acc[k] * inv;
            const uint32_t e = recall16(mean[k], hb[k]);
            bad = bad ? bad : e;
            acc[k] = 0.0f;
        }
        const uint64_t out = (uint64_t(lane) * a.pages + page) * a.width + c0;
        if (mo) {
            float4 *m4 = reinterpret_cast<float4 *>(mo + out);
            m4[0] = make_float4(mean[0], mean[1], mean[2], mean[3]);
            if constexpr (CPL == 8) m4[1] = make_float4(mean[4], mean[5], mean[6], mean[7]);
        }
        if (bad) raise_operand(a.status, bad, pick(i, epoch[0], epoch[1], epoch[2], epoch[3]));
        if (so) {
            typedef typename F16Lane<CPL>::type V;
            V v;
#pragma unroll
            for (int k = 0; k < CPL / 2; ++k) v[k] = uint32_t(hb[2 * k]) | (uint32_t(hb[2 * k + 1]) << 16);
            *reinterpret_cast<V *>(so + out) = v;
        }
    };
    // Row u of a chunk is summed only when it is a real row (pad rows add
    // zeros: acc is never -0, so acc + (+-0) is acc bit for bit).
    auto consume = [&](const auto v, bool real) {
        if constexpr (SRC == kSrcKeysF16) {
#pragma unroll
            for (int k = 0; k < CPL / 2; ++k) {
                const uint32_t w = real ? uint32_t(v[k]) : 0u;
                acc[2 * k] += h2f(uint16_t(w & 0xffffu));
                acc[2 * k + 1] += h2f(uint16_t(w >> 16));
            }
        } else {
            const uint32_t lo = __builtin_amdgcn_perm(v[1], v[0], code_sel);
            const uint32_t hi = __builtin_amdgcn_perm(v[2], v[1], code_sel);
            const uint32_t dw = dpp::move<dpp::kQuadBcast0>(v[0]);
            const uint32_t d = odd ? dw >> 16 : dw & 0xffffu;
            add_q8x8(acc, real ? lo : 0u, real ? hi : 0u, h2f(uint16_t(real ? d : 0u)));
        }
    };
    // Each layer is read in chunks of D rows, the last one padded: then a
    // layer ends on a chunk boundary, its epilogue runs once outside the
    // unrolled steps, and the next chunk's loads (the next layer's first
    // rows at a boundary) are already in flight when it runs.  A chunk is
    // (layer li, first row r0); `left` = n - 1 - r0 rows follow its first.
    // PAGED: the page's n rows in the layer are one buffer resource, and
    // row u of a chunk sits at col + coff + u*row_bytes with coff =
    // r0*row_bytes; otherwise the chunk's first row is at cp.
    constexpr int D = SRC == kSrcKeysF16 ? kF16RingRows<CPL> : kQ8Rows;
    const uint32_t per_layer = (n + D - 1) / D;
    const uint32_t chunks = m * per_layer;
    const uint8_t *cp = layer_first(0);
    uint32_t left = n - 1, coff = 0;
    auto page_rsrc = [&]() {
        if constexpr (PAGED) return buffer_rsrc(cp, n * row_bytes); else return 0;
    };
    auto rs = page_rsrc();
    auto load_row = [&](int u) {
        if constexpr (PAGED) {
            // the row offset is a scalar computed per row (no per-lane table)
            const uint32_t off = col + __builtin_amdgcn_readfirstlane(coff + uint32_t(u) * row_bytes);
            if constexpr (SRC == kSrcKeysF16 && CPL == 4)
                return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, kBufferNontemporal));
            else if constexpr (SRC == kSrcKeysF16)
                return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, kBufferNontemporal));
            else
                return __builtin_bit_cast(u32x3, __builtin_amdgcn_raw_buffer_load_b96(rs, off, 0, kBufferNontemporal));
        } else {
            const uint8_t *p = cp + uint64_t(min(uint32_t(u), left)) * row_bytes;
            if constexpr (SRC == kSrcKeysF16)
                return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
            else
                return u32x3(__builtin_nontemporal_load(reinterpret_cast<const u32x3a *>(p)));
        }
    };
    decltype(load_row(0)) ring[D];
#pragma unroll
    for (int u = 0; u < D; ++u) {
        ring[u] = load_row(u);
        __builtin_amdgcn_sched_barrier(0);
    }
    // one chunk's rows consumed while the next chunk's rows are loaded
    auto step = [&](auto masked, uint32_t real_left) {
#pragma unroll
        for (int u = 0; u < D; ++u) {
            consume(ring[u], decltype(masked)::value ? uint32_t(u) <= real_left : true);
            ring[u] = load_row(u);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    uint32_t li = 0, lc = 0;  // layer and chunk within it of the ring's rows
    for (uint32_t c = 0; c + 1 < chunks; ++c) {
        const uint32_t real_left = left;
        const bool wrap = lc + 1 == per_layer;
        if constexpr (PAGED) {
            if (wrap) {
                cp = layer_first(li + 1);
                rs = page_rsrc();
            }
            coff = wrap ? 0u : coff + D * row_bytes;
        } else {
            cp = wrap ? layer_first(li + 1) : cp + uint64_t(D) * row_bytes;
        }
        left = wrap ? n - 1 : left - D;
        step(std::integral_constant<bool, !PAGED>{}, real_left);
        if (wrap) {
            finish(li);
            ++li;
            lc = 0;
        } else {
            ++lc;
        }
    }
#pragma unroll
    for (int u = 0; u < D; ++u) consume(ring[u], PAGED || uint32_t(u) <= left);
    finish(li);
}

// One launch of a layer stack: the summary workgroups of a group of up to
// kStackGroup consecutive layers (blocks [0, summary_blocks); each walks the
// group's layers in order with the layout of k_summary), then the previous
// group's softmax workgroups (layer-major, then lane-major).  Key-history
// layers get their logits from those softmax workgroups, which compute them
// from the stored summaries before their units; resident-summary layers get
// them from the summary workgroups (query staging alternates between two
// LDS buffers, so a layer's staging never overwrites rows the previous
// layer's epilogue may still read).
template <int SRC, int NPL>
__global__ __launch_bounds__(256) void k_stack_group(StackGroupArgs g) {
    const uint32_t sb = g.m ? g.summary_blocks : 0;
    if (blockIdx.x >= sb) {
        // default wave priority: below the summary's streaming waves on a
        // shared CU; these have the whole launch to finish in
        const uint32_t per_layer = g.probs_per_lane * g.p[0].lanes;
        const uint32_t b = blockIdx.x - sb, i = b / per_layer, r = b % per_layer;
        probs_block<NPL, true>(g.p[i], r % g.probs_per_lane, r / g.probs_per_lane, g.probs_per_lane);
        return;
    }
    // The group's layers are split into parts of layers_per_part
    // consecutive layers (one part when a layer's workgroups fill the GPU);
    // workgroup b covers summary slot b % layer_blocks of its part's layers.
    const uint32_t part = blockIdx.x / g.layer_blocks, blk = blockIdx.x - part * g.layer_blocks;
    const uint32_t l0 = part * g.layers_per_part, m = min(g.m - l0, g.layers_per_part);
    // Key histories leave the logits to the softmax workgroups of the next
    // launch; resident summaries have no stream, so they compute theirs here.
    if constexpr (SRC == kSrcSummary) {
        for (uint32_t i = 0; i < m; ++i) summary_block<SRC, true>(g.s[l0 + i], blk, q_lds_buf + (i & 1) * g.q_slot);
    } else {
        const SummaryArgs &a = g.s[0];
        const uint64_t row_bytes = SRC == kSrcKeysF16 ? a.width * 2 : (a.width >> 5) * kQ8Bytes;
        if (SRC == kSrcKeysF16 && stack_cpl(SRC, a.width, a.page_tokens) == 4)
            stack_summaries<SRC, true, SRC == kSrcKeysF16 ? 4 : 8>(g, blk, l0, m);
        else if ((a.width & 511) == 0 && (uint64_t(a.page_tokens) + 64) * row_bytes < (uint64_t(1) << 32))
            stack_summaries<SRC, true>(g, blk, l0, m);
        else
            stack_summaries<SRC, false>(g, blk, l0, m);
    }
}

// Selection over given scores (no softmax), one workgroup per lane.
__global__ __launch_bounds__(256) void k_select(SelectArgs a) { lane_tail(a, blockIdx.x); }

// Half-page masses folded into page scores, one lane per workgroup row of
// the grid (y); invalid halves make the lane's scores unwritten.
__global__ __launch_bounds__(256) void k_fold_halves(FoldArgs a) {
    const uint32_t lane = blockIdx.x;
    const double *h = a.halves + uint64_t(lane) * 2 * a.pages;
    double *out = a.scores + uint64_t(lane) * a.pages;
    int bad = 0;
    for (uint32_t j = threadIdx.x; j < a.pages; j += 256) {
        const double left = h[2 * j], right = h[2 * j + 1], sum = left + right;
        bad |= left < 0.0 || right < 0.0 || !__builtin_isfinite(sum) || (a.mask && !a.mask[j] && sum != 0.0);
    }
    bad = __syncthreads_or(bad);
    if (bad) {
        if (threadIdx.x == 0) raise_status(a.status, kStatusScores, a.epoch);
        return;
    }
    for (uint32_t j = threadIdx.x; j < a.pages; j += 256) {
        const double left = h[2 * j], right = h[2 * j + 1];
        out[j] = a.rule == kFoldSum ? left + right : (left < right ? right : left);
    }
}

// ---------------------------------------------------------------------------
// Selection with media groups: KvMemStore::pick_scored_blocks with media
// ranges (kvmem/src/host/kvmem_store.cpp:418-451) and the fill of
// constrain_media (:453-502).  A page in a group is kept only together with
// its whole group; fixed pages bring their groups and must fit; then the
// pages are visited in rank order -- preferred pages first, then score
// desc, then id by the tie rule -- and each visited group (or lone page)
// is kept when it still fits the budget, else skipped.  A group is met at
// its best-ranked page, so the lane's units are its lone pages and each
// group's best page.  One workgroup per lane: keys and each page's group
// bounds in LDS, the units put in rank order by a bitonic sort, then one
// thread walks them -- whether a group fits depends on everything taken
// before it.  Rows of up to kGroupSelectPages pages.
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool bit_at(const uint32_t *bits, uint32_t j) { return bits[j >> 5] >> (j & 31) & 1u; }
__device__ __forceinline__ void bit_set(uint32_t *bits, uint32_t j) { atomicOr(&bits[j >> 5], 1u << (j & 31)); }

__host__ __device__ constexpr uint32_t pow2_ceil(uint32_t n) {
    uint32_t p = 1;
    while (p < n) p <<= 1;
    return p;
}
// LDS of k_select_groups: keys (8 B), group begin and end (2 B each) per
// page, the sort order (2 B per slot of a power of two), three bitmaps.
__host__ __device__ constexpr size_t group_select_lds(uint32_t n) {
    return size_t(n) * 12 + ((size_t(pow2_ceil(n)) * 2 + 15) & ~size_t(15)) + size_t((n + 31) / 32) * 12;
}

__global__ __launch_bounds__(256) void k_select_groups(SelectArgs a) {
    __shared__ uint32_t s_red[4];
    __shared__ uint32_t s_count;
    constexpr uint32_t B = 256;
    const uint32_t lane = blockIdx.x, tid = threadIdx.x, n = a.pages;
    const uint32_t N = pow2_ceil(n), words = (n + 31) / 32;
    uint64_t *key = tail_keys;                                     // [n]
    uint16_t *glo = reinterpret_cast<uint16_t *>(key + n);         // [n] first page of the page's group
    uint16_t *ghi = glo + n;                                       // [n] one past its last page
    uint16_t *order = ghi + n;                                     // [N] page ids by rank
    uint32_t *kept = reinterpret_cast<uint32_t *>(reinterpret_cast<uint8_t *>(key) + size_t(n) * 12 +
                                                  ((size_t(N) * 2 + 15) & ~size_t(15)));  // [words]
    uint32_t *pref = kept + words;  // preferred pages
    uint32_t *unit = pref + words;  // pages the walk visits
    const double *sc = a.scores + uint64_t(lane) * n;

    bool failed = a.status && tid == 0 && epoch_failed(a.status, a.epoch);
    int bad = 0;
    for (uint32_t j = tid; j < n; j += B) {
        const double v = sc[j];
        bad |= !__builtin_isfinite(v) || (!a.signed_scores && v < 0.0);
        key[j] = order_key(v);
        glo[j] = uint16_t(j);
        ghi[j] = uint16_t(j + 1);
    }
    for (uint32_t w = tid; w < words; w += B) kept[w] = pref[w] = unit[w] = 0;
    __syncthreads();
    for (uint32_t g = tid; g < a.n_groups; g += B) {
        const uint32_t b = min(a.groups[2 * g], n), e = min(a.groups[2 * g + 1], n);
        for (uint32_t j = b; j < e; ++j) {
            glo[j] = uint16_t(b);
            ghi[j] = uint16_t(e);
        }
    }
    for (uint32_t i = tid; i < a.n_mandatory; i += B)
        if (a.mandatory[i] < n) bit_set(kept, a.mandatory[i]);
    for (uint32_t i = tid; i < a.n_fixed; i += B) {
        const uint32_t id = a.fixed[i];
        if (id < n) bit_set(kept, id);
    }
    if (a.preferred) {
        const uint32_t *ids = a.preferred + uint64_t(lane) * a.preferred_stride;
        const uint32_t cnt = min(a.preferred_count[lane], a.preferred_stride);
        for (uint32_t i = tid; i < cnt; i += B) {
            const uint32_t id = ids[i];
            if (id < n) bit_set(pref, id);
        }
    }
    bad = __syncthreads_or(bad);
    failed = __syncthreads_or(failed);
    if (bad || failed) {
        if (bad && tid == 0) raise_status(a.status, kStatusScores, a.epoch);
        if (tid == 0) a.count[lane] = 0;
        return;
    }
    // u ranks before v
    auto better = [&](uint32_t u, uint32_t v) -> bool {
        const bool cu = u < n && bit_at(unit, u), cv = v < n && bit_at(unit, v);
        if (cu != cv) return cu;
        if (!cu) return false;
        const bool pu = bit_at(pref, u), pv = bit_at(pref, v);
        if (pu != pv) return pu;
        if (key[u] != key[v]) return key[u] > key[v];
        return a.tie_higher_first ? u > v : u < v;
    };
    auto ranks_before = [&](uint32_t u, uint32_t v) -> bool {  // among pages of one group
        const bool pu = bit_at(pref, u), pv = bit_at(pref, v);
        if (pu != pv) return pu;
        if (key[u] != key[v]) return key[u] > key[v];
        return a.tie_higher_first ? u > v : u < v;
    };
    // A group holding a fixed page is kept whole; else its best page is its
    // unit.  One thread per group (the one whose page starts it).
    for (uint32_t j = tid; j < n; j += B) {
        const uint32_t e = ghi[j];
        if (glo[j] != j) continue;
        if (e == j + 1) {
            if (!bit_at(kept, j)) bit_set(unit, j);
            continue;
        }
        bool any = false;
        for (uint32_t i = j; i < e && !any; ++i) any = bit_at(kept, i);
        if (any) {
            for (uint32_t i = j; i < e; ++i) bit_set(kept, i);
        } else {
            uint32_t best = j;
            for (uint32_t i = j + 1; i < e; ++i)
                if (ranks_before(i, best)) best = i;
            bit_set(unit, best);
        }
    }
    __syncthreads();
    uint32_t c = 0;
    for (uint32_t w = tid; w < words; w += B) c += __popc(kept[w]);
    c = wave_sum(c);
    if ((tid & (kWave - 1)) == 0) s_red[tid / kWave] = c;
    for (uint32_t i = tid; i < N; i += B) order[i] = uint16_t(i);  // slots past the row: ids >= n, no unit
    __syncthreads();
    const uint32_t n_fixed = s_red[0] + s_red[1] + s_red[2] + s_red[3];
    if (n_fixed > a.k) {
        if (tid == 0) {
            raise_status(a.status, kStatusBudget, a.epoch);
            a.count[lane] = 0;
        }
        return;
    }
    // bitonic sort of the slots, best first; slots that hold no unit sort
    // last (they never swap among themselves)
    for (uint32_t size = 2; size <= N; size <<= 1) {
        for (uint32_t stride = size >> 1; stride; stride >>= 1) {
            for (uint32_t i = tid; i < N / 2; i += B) {
                const uint32_t x = ((i & ~(stride - 1)) << 1) | (i & (stride - 1)), y = x + stride;
                const uint32_t u = order[x], v = order[y];
                const bool desc = (x & size) == 0;
                if (desc ? better(v, u) : better(u, v)) {
                    order[x] = uint16_t(v);
                    order[y] = uint16_t(u);
                }
            }
            lds_barrier();
        }
    }
    if (tid == 0) {
        uint32_t cnt = n_fixed;
        for (uint32_t i = 0; i < N && cnt < a.k; ++i) {
            const uint32_t u = order[i];
            if (u >= n || !bit_at(unit, u)) break;
            const uint32_t b = glo[u], e = ghi[u];
            if (cnt + (e - b) > a.k) continue;
            for (uint32_t p = b; p < e; ++p) kept[p >> 5] |= 1u << (p & 31);
            cnt += e - b;
        }
        s_count = cnt;
    }
    __syncthreads();
    // kept pages in ascending order: each thread a run of whole words
    const uint32_t wpt = (words + B - 1) / B, w0 = min(words, tid * wpt), w1 = min(words, w0 + wpt);
    uint32_t mine = 0;
    for (uint32_t w = w0; w < w1; ++w) mine += __popc(kept[w]);
    const uint32_t incl = wave_inclusive_scan(mine);
    if ((tid & (kWave - 1)) == kWave - 1) s_red[tid / kWave] = incl;
    __syncthreads();
    uint32_t o = incl - mine;
    for (uint32_t w = 0; w < tid / kWave; ++w) o += s_red[w];
    uint32_t *out = a.selected + uint64_t(lane) * a.k;
    for (uint32_t w = w0; w < w1; ++w)
        for (uint32_t bits = kept[w]; bits; bits &= bits - 1)
            if (o < a.k) out[o++] = w * 32 + uint32_t(__ffs(bits) - 1);
    if (tid == 0) a.count[lane] = min(s_count, a.k);
}

// ---------------------------------------------------------------------------
// Stage-in gather.  One workgroup copies `chunk_rows` token rows of one
// selected page of one plane.  Sources are pinned host pages read directly
// over the host link (or staged device copies); destinations are slot rows
// [slot*page_tokens + r] (write_block_to_gpu, llama-memory-kvmem.cpp:4464-4520).
//   copy         bytes unchanged                       (stagein.cu:236-261)
//   dequant_f16  q8_0: y = q*d (stagein.cu:133-143); q4_1: y = nib*d + m;
//                then RNE binary16
//   requant_q8_0 d = amax/127, q = roundf(x/d)          (stagein.cu:181-199)
// ---------------------------------------------------------------------------
__device__ __forceinline__ void copy_span(const uint8_t *src, uint8_t *dst, uint32_t bytes) {
    const uint32_t nt = blockDim.x;
    if (((uintptr_t(src) | uintptr_t(dst) | bytes) & 15u) == 0) {
        const u32x4 *s = reinterpret_cast<const u32x4 *>(src);
        u32x4 *d = reinterpret_cast<u32x4 *>(dst);
        const uint32_t n = bytes >> 4;
        uint32_t i = threadIdx.x;
        for (; i + 3 * nt < n; i += 4 * nt) {
            const u32x4 v0 = __builtin_nontemporal_load(s + i), v1 = __builtin_nontemporal_load(s + i + nt),
                        v2 = __builtin_nontemporal_load(s + i + 2 * nt), v3 = __builtin_nontemporal_load(s + i + 3 * nt);
            d[i] = v0; d[i + nt] = v1; d[i + 2 * nt] = v2; d[i + 3 * nt] = v3;
        }
        for (; i < n; i += nt) d[i] = __builtin_nontemporal_load(s + i);
    } else if (((uintptr_t(src) | uintptr_t(dst) | bytes) & 3u) == 0) {
        const uint32_t *s = reinterpret_cast<const uint32_t *>(src);
        uint32_t *d = reinterpret_cast<uint32_t *>(dst);
        for (uint32_t i = threadIdx.x; i < bytes >> 2; i += nt) d[i] = s[i];
    } else {
        for (uint32_t i = threadIdx.x; i < bytes; i += nt) dst[i] = src[i];
    }
}

__device__ __forceinline__ void decode_block(const uint8_t *blk, uint32_t fmt, float *y) {
    const float d = h2f(ld_u16(blk));
    if (fmt == kFmtQ8) {
#pragma unroll
        for (int j = 0; j < kQK; ++j) y[j] = float(int8_t(blk[2 + j])) * d;
    } else if (fmt == kFmtQ40) {
        // (nib - 8) * d, low nibbles first (stagein.cu:145-158)
#pragma unroll
        for (int j = 0; j < kQK / 2; ++j) {
            const uint8_t b = blk[2 + j];
            y[j] = float(int(b & 15) - 8) * d;
            y[j + kQK / 2] = float(int(b >> 4) - 8) * d;
        }
    } else {
        const float m = h2f(ld_u16(blk + 2));
#pragma unroll
        for (int j = 0; j < kQK / 2; ++j) {
            const uint8_t b = blk[4 + j];
            // nib*d is exact, so fma(nib, d, m) rounds like "nib*d + m".
            y[j] = float(b & 15) * d + m;
            y[j + kQK / 2] = float(b >> 4) * d + m;
        }
    }
}

__device__ __forceinline__ void quant_block_q8(const float *x, uint8_t *blk) {
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < kQK; ++j) amax = fmaxf(amax, fabsf(x[j]));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const uint16_t dh = f2h(d);
    blk[0] = uint8_t(dh);
    blk[1] = uint8_t(dh >> 8);
#pragma unroll
    for (int j = 0; j < kQK; ++j) blk[2 + j] = uint8_t(int8_t(roundf(x[j] * id)));
}

// q4_0 (stagein.cu:201-234): the value of largest magnitude (first of
// equals) sets d = v / -8; codes (int)(x*id + 8.5) capped at 15, the
// multiply-add fused (explicitly, so it does not depend on contraction).
__device__ __forceinline__ void quant_block_q40(const float *x, uint8_t *blk) {
    float amax = 0.0f, vmax = 0.0f;
#pragma unroll
    for (int j = 0; j < kQK; ++j) {
        const float v = x[j];
        const bool more = amax < fabsf(v);
        amax = more ? fabsf(v) : amax;
        vmax = more ? v : vmax;
    }
    const float d = vmax / -8.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const uint16_t dh = f2h(d);
    blk[0] = uint8_t(dh);
    blk[1] = uint8_t(dh >> 8);
#pragma unroll
    for (int j = 0; j < kQK / 2; ++j) {
        const int x0 = min(int(__builtin_fmaf(x[j], id, 8.5f)), 15);
        const int x1 = min(int(__builtin_fmaf(x[j + kQK / 2], id, 8.5f)), 15);
        blk[2 + j] = uint8_t((x0 & 15) | ((x1 & 15) << 4));
    }
}

// sin and cos of a binary32 angle, each rounded once to binary32 from a
// binary64 evaluation: reduction by the nearest multiple k of pi/2
// (Cody-Waite, pi/2 in two binary64 parts, fused), Taylor polynomials of
// degree 21 (sin) and 20 (cos) on |r| <= pi/4 (truncation below 1e-24),
// then the quadrant k mod 4.  Written from those series; the oracle runs
// the same operations, so the results agree bit for bit.
__device__ __forceinline__ void rope_sincos(float angle, float &s, float &c) {
    const double x = angle;
    const double k = __builtin_rint(x * 0.6366197723675814);
    double r = __builtin_fma(-k, 1.5707963267948966, x);
    r = __builtin_fma(-k, 6.123233995736766e-17, r);
    const double r2 = r * r;
    double ps = 1.9572941063391263e-20;
    ps = __builtin_fma(ps, r2, -8.22063524662433e-18);
    ps = __builtin_fma(ps, r2, 2.8114572543455206e-15);
    ps = __builtin_fma(ps, r2, -7.647163731819816e-13);
    ps = __builtin_fma(ps, r2, 1.6059043836821613e-10);
    ps = __builtin_fma(ps, r2, -2.505210838544172e-08);
    ps = __builtin_fma(ps, r2, 2.7557319223985893e-06);
    ps = __builtin_fma(ps, r2, -0.0001984126984126984);
    ps = __builtin_fma(ps, r2, 0.008333333333333333);
    ps = __builtin_fma(ps, r2, -0.16666666666666666);
    const double sr = __builtin_fma(r * r2, ps, r);
    double pc = 4.110317623312165e-19;
    pc = __builtin_fma(pc, r2, -1.5619206968586225e-16);
    pc = __builtin_fma(pc, r2, 4.779477332387385e-14);
    pc = __builtin_fma(pc, r2, -1.1470745597729725e-11);
    pc = __builtin_fma(pc, r2, 2.08767569878681e-09);
    pc = __builtin_fma(pc, r2, -2.755731922398589e-07);
    pc = __builtin_fma(pc, r2, 2.48015873015873e-05);
    pc = __builtin_fma(pc, r2, -0.001388888888888889);
    pc = __builtin_fma(pc, r2, 0.041666666666666664);
    pc = __builtin_fma(pc, r2, -0.5);
    const double cr = __builtin_fma(r2, pc, 1.0);
    const uint32_t q = uint32_t(int64_t(k)) & 3u;
    const double sv = q == 0 ? sr : q == 1 ? cr : q == 2 ? -sr : -cr;
    const double cv = q == 0 ? cr : q == 1 ? -sr : q == 2 ? -cr : sr;
    s = float(sv);
    c = float(cv);
}

// The raw-K transform of one row staged in the wave's LDS (rope_neox_kernel,
// fwht_kernel, stagein.cu:105-130, 160-178, run in flush's order,
// stagein.cu:746-783): decode into a binary32 row, rotate each head's pairs
// at the row's position, scale and butterfly each run of `fwht` values
// (h = 1, 2, 4, ...: (a, b) -> (a+b, a-b), as the reference's loop nest),
// then requantize the row in place.  One wave; LDS order within a wave is
// program order, with a wave fence between phases.
// The transform's parameters of one work item, read once: uniform values
// and the lane's own rotation angle (theta of pair index = lane).
struct RopeRow {
    uint32_t width, head_dim, half, fwht, fwht_log2;
    float fwht_scale;
    bool q8;
    float theta_l[4];  // pair indices lane + 64k (half <= 256)
};
__device__ __forceinline__ void rope_fwht_row(const RopeRow &P, uint8_t *raw, float *fr, int64_t pos) {
    const uint32_t l = threadIdx.x & 63;
    const bool q8 = P.q8;
    const uint32_t bbytes = q8 ? kQ8Bytes : kQ40Bytes;
    // one element per lane, consecutive across the wave (a lane per block
    // would put the 32 lanes' row accesses in one LDS bank)
#pragma unroll 4
    for (uint32_t e = l; e < P.width; e += kWave) {
        const uint8_t *blk = raw + (e / kQK) * bbytes;
        const uint32_t j = e % kQK;
        const float d = h2f(ld_u16(blk));
        const uint8_t byte = blk[2 + (q8 ? j : j % 16)];
        const int code = q8 ? int(int8_t(byte)) : int(j < 16 ? byte & 15 : byte >> 4) - 8;
        fr[e] = float(code) * d;
    }
    wave_lds_sync();
    // the angle depends on the pair index and the position, not the head:
    // one sin/cos per pair index, applied to every head
    const uint32_t half = P.half, heads = P.width / P.head_dim;
    const float fpos = float(pos);
#pragma unroll
    for (uint32_t k = 0; k < 4; ++k) {
        const uint32_t i = l + k * kWave;
        if (i >= half) break;
        float sn, cs;
        rope_sincos(fpos * P.theta_l[k], sn, cs);
#pragma unroll 4
        for (uint32_t h = 0; h < heads; ++h) {
            float *row = fr + h * P.head_dim;
            const float x0 = row[i], x1 = row[i + half];
            row[i] = __builtin_fmaf(x0, cs, -(x1 * sn));
            row[i + half] = __builtin_fmaf(x0, sn, x1 * cs);
        }
    }
    wave_lds_sync();
    if (P.fwht) {
#pragma unroll 4
        for (uint32_t j = l; j < P.width; j += kWave) fr[j] *= P.fwht_scale;
        wave_lds_sync();
        // sizes are powers of two: butterfly q of a stage is run q >> (log2 - 1),
        // index w within it; pairs (a, a + hs)
        const uint32_t lh = P.fwht_log2 - 1;
        for (uint32_t ls = 0; ls <= lh; ++ls) {
            const uint32_t hs = 1u << ls;
#pragma unroll 4
            for (uint32_t q = l; q < P.width / 2; q += kWave) {
                const uint32_t g = q >> lh, w = q & ((1u << lh) - 1u);
                const uint32_t a = (g << P.fwht_log2) + ((w >> ls) << (ls + 1)) + (w & (hs - 1u));
                const float x = fr[a], y = fr[a + hs];
                fr[a] = x + y;
                fr[a + hs] = x - y;
            }
            wave_lds_sync();
        }
    }
    // requantize: each half wave one block, lane j its element
    for (uint32_t e0 = 0; e0 < P.width; e0 += kWave) {
        const uint32_t e = e0 + l, j = l % kQK;
        const bool on = e < P.width;  // uniform per half wave (width % 32 == 0)
        const float x = on ? fr[e] : 0.0f;
        uint8_t *blk = raw + (min(e, P.width - 1) / kQK) * bbytes;
        if (q8) {
            // quant_q8_0 (stagein.cu:181-199): d = amax/127, q = roundf(x*id)
            float amax = dpp::group_reduce(fabsf(x), 16, dpp::Max());
            amax = fmaxf(amax, __shfl_xor(amax, 16, kWave));
            const float d = amax / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            if (on) {
                blk[2 + j] = uint8_t(int8_t(roundf(x * id)));
                if (j == 0) {
                    const uint16_t dh = f2h(d);
                    blk[0] = uint8_t(dh);
                    blk[1] = uint8_t(dh >> 8);
                }
            }
        } else {
            // quant_q4_0 (stagein.cu:201-234): the first element of largest
            // magnitude sets d = v / -8 (argmax key: |x| bits, then lower index)
            uint64_t key = (uint64_t(__float_as_uint(fabsf(x))) << 32) | (31u - j);
            key = dpp::group_reduce(key, 16, dpp::Max());
            const uint64_t other = (uint64_t(uint32_t(__shfl_xor(int(key >> 32), 16, kWave))) << 32) |
                                   uint32_t(__shfl_xor(int(uint32_t(key)), 16, kWave));
            key = other > key ? other : key;
            const uint32_t src = (l & 32u) | (31u - uint32_t(key & 31u));
            const float vmax = __shfl(x, int(src), kWave);
            const float d = vmax / -8.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            const int c = min(int(__builtin_fmaf(x, id, 8.5f)), 15);
            const int hi = __shfl_down(c, 16, kWave);  // element j + 16 of the block
            if (on && j < 16) {
                blk[2 + j] = uint8_t((c & 15) | ((hi & 15) << 4));
                if (j == 0) {
                    const uint16_t dh = f2h(d);
                    blk[0] = uint8_t(dh);
                    blk[1] = uint8_t(dh >> 8);
                }
            }
        }
    }
    wave_lds_sync();
}

// Persistent: a bounded grid loops over (lane, slot, plane, chunk) items, so
// waves parked on host-link latency occupy a few CUs instead of all of them
// while the select stream's HBM-bound kernels run beside the gather.
// Dynamic LDS of the gather: one staging slice per wave.
extern __shared__ __align__(16) uint8_t gather_lds[];

// One wave copies `bytes` from src to dst: 16-byte lanes with up to 16
// loads (16 KiB per wave) in flight before the stores when both ends and
// the size are 16-byte aligned.
__device__ __forceinline__ void wave_copy(const uint8_t *src, uint8_t *dst, uint32_t bytes) {
    const uint32_t l = threadIdx.x & 63;
    if (((uintptr_t(src) | uintptr_t(dst) | bytes) & 15u) == 0) {
        const u32x4 *s = reinterpret_cast<const u32x4 *>(src);
        u32x4 *d = reinterpret_cast<u32x4 *>(dst);
        const uint32_t n = bytes >> 4;
        constexpr uint32_t B = 16;
        // Every load of a batch is issued before its stores; lanes past the
        // end of the last, partial batch re-read the final vector (clamped,
        // so no load is predicated and none waits for another).
        for (uint32_t base = 0; base < n; base += B * kWave) {
            u32x4 v[B];
#pragma unroll
            for (uint32_t u = 0; u < B; ++u) v[u] = __builtin_nontemporal_load(s + min(base + u * kWave + l, n - 1));
#pragma unroll
            for (uint32_t u = 0; u < B; ++u) {
                const uint32_t i = base + u * kWave + l;
                if (i < n) d[i] = v[u];
            }
        }
    } else if (((uintptr_t(src) | uintptr_t(dst) | bytes) & 3u) == 0) {
        const uint32_t *s = reinterpret_cast<const uint32_t *>(src);
        uint32_t *d = reinterpret_cast<uint32_t *>(dst);
        for (uint32_t i = l; i < bytes >> 2; i += kWave) d[i] = s[i];
    } else {
        for (uint32_t i = l; i < bytes; i += kWave) dst[i] = src[i];
    }
}

// Persistent gather, one work item per wave at a time: (lane, slot, plane,
// chunk of chunk_rows rows).  Copies go straight from the source rows to the
// slot rows; decoding modes stage the packed rows in the wave's LDS slice
// (no workgroup barrier), decode whole blocks from there and write fp16
// rows, or requantize in place and copy the slice out.
__global__ __launch_bounds__(256) void k_gather(GatherArgs a) {
    // the wave index as a scalar: every work item's fields are uniform
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = threadIdx.x & 63,
                   wpb = blockDim.x >> 6;
    uint8_t *wl = gather_lds + wave * a.lds_per_wave;
    const uint32_t per_lane = a.k * a.n_planes * a.chunks;
    const uint64_t total = uint64_t(a.lanes) * per_lane;
    const uint64_t step = uint64_t(gridDim.x) * wpb;
    for (uint64_t it = uint64_t(blockIdx.x) * wpb + wave; it < total; it += step) {
        const uint32_t lane = uint32_t(it / per_lane);
        uint32_t id = uint32_t(it % per_lane);
        const uint32_t chunk = id % a.chunks;
        id /= a.chunks;
        const uint32_t pi = id % a.n_planes;
        const uint32_t slot = id / a.n_planes;
        const uint32_t cnt = a.count ? a.count[lane] : a.k;
        if (slot >= cnt) continue;
        const GatherPlane &P = a.plane[pi];
        const uint32_t page = a.selected ? a.selected[uint64_t(lane) * a.k + slot] : slot;
        const uint64_t first = uint64_t(page) * a.page_tokens;
        if (first >= P.tokens) continue;
        const uint64_t left = P.tokens - first;
        const uint32_t valid = left < a.page_tokens ? uint32_t(left) : a.page_tokens;
        const uint32_t r0 = chunk * a.chunk_rows;
        if (r0 >= valid) continue;
        const uint32_t nr = min(a.chunk_rows, valid - r0);
        // Staged sources (src_page_stride != 0) hold slot s's page at s*stride;
        // record sources (P.page_stride != 0) page p at p*stride.
        const uint64_t at = a.src_page_stride ? uint64_t(slot) * a.src_page_stride + uint64_t(r0) * P.src_row
                            : P.page_stride   ? uint64_t(page) * P.page_stride + uint64_t(r0) * P.src_row
                                              : (first + r0) * P.src_row;
        const uint8_t *src = P.src + lane * P.src_lane_stride + at;
        uint8_t *dst = P.dst + lane * P.dst_lane_stride + (uint64_t(slot) * a.page_tokens + r0) * P.dst_row;
        const uint32_t sbytes = nr * P.src_row;
        if (P.mode == kModeCopy || P.format == kFmtF16) {
            wave_copy(src, dst, sbytes);
            continue;
        }
        wave_copy(src, wl, sbytes);
        wave_lds_sync();
        if (P.mode == kModeRopeFwht) {
            // binary32 row after the staged rows (16-byte aligned)
            float *fr = reinterpret_cast<float *>(wl + ((sbytes + 15u) & ~15u));
            RopeRow R;
            R.width = P.width;
            R.head_dim = P.head_dim;
            R.half = P.n_rot / 2;
            R.fwht = P.fwht;
            R.fwht_log2 = P.fwht ? 31u - __builtin_clz(P.fwht) : 0u;
            R.fwht_scale = P.fwht_scale;
            R.q8 = P.format == kFmtQ8;
#pragma unroll
            for (uint32_t k = 0; k < 4; ++k) R.theta_l[k] = l + k * kWave < R.half ? P.theta[l + k * kWave] : 0.0f;
            for (uint32_t r = 0; r < nr; ++r)
                rope_fwht_row(R, wl + r * P.src_row, fr, P.pos_base + int64_t(first + r0 + r));
            wave_copy(wl, dst, sbytes);
            wave_lds_sync();  // the slice is refilled by the next item
            continue;
        }
        const uint32_t bpr = P.width / kQK;
        const uint32_t bbytes = P.format == kFmtQ8 ? kQ8Bytes : kQ41Bytes;
        const uint32_t nblocks = nr * bpr;
        if (P.mode == kModeDequantF16) {
            for (uint32_t b = l; b < nblocks; b += kWave) {
                float y[kQK];
                decode_block(wl + b * bbytes, P.format, y);
                u32x4 *o = reinterpret_cast<u32x4 *>(dst + uint64_t(b / bpr) * P.dst_row + (b % bpr) * 64);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    u32x4 v;
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        v[i] = uint32_t(f2h(y[8 * q + 2 * i])) | (uint32_t(f2h(y[8 * q + 2 * i + 1])) << 16);
                    o[q] = v;
                }
            }
        } else {
            // each lane requantizes its own blocks in place, then the slice goes out
            for (uint32_t b = l; b < nblocks; b += kWave) {
                float y[kQK];
                decode_block(wl + b * kQ8Bytes, kFmtQ8, y);
                quant_block_q8(y, wl + b * kQ8Bytes);
            }
            wave_lds_sync();
            wave_copy(wl, dst, sbytes);
        }
        wave_lds_sync();  // the slice is refilled by the next item
    }
}

// ---------------------------------------------------------------------------
// Capture-side running mean-K sums (kvmem_meank_add, stagein.cu:270-320, and
// add_mean_f32's page restart rule, raw_kv_store.cpp:178-197).  One thread per
// (page segment, channel), sequential over the segment's tokens.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_accumulate(AccumulateArgs a) {
    const uint64_t gid = uint64_t(blockIdx.x) * 256 + threadIdx.x;
    if (gid >= uint64_t(a.segments) * a.width) return;
    const uint32_t c = uint32_t(gid % a.width);
    const uint32_t page = a.first_page + uint32_t(gid / a.width);
    const uint64_t pstart = uint64_t(page) * a.page_tokens;
    const uint64_t s = max(a.pos0, pstart), e = min(a.pos0 + a.n, pstart + a.page_tokens);
    const uint32_t off = uint32_t(s - pstart), take = uint32_t(e - s);
    float *sum = a.sums + uint64_t(page) * a.width + c;
    float acc = off == 0 ? 0.0f : *sum;
    const uint32_t h = c / a.dim, d = c % a.dim;
    const uint8_t *p = a.k + (s - a.pos0) * a.token_stride + h * a.head_stride + d * a.dim_stride;
    for (uint32_t t = 0; t < take; ++t) acc += load_scalar(p + uint64_t(t) * a.token_stride, a.scalar);
    *sum = acc;
    if (c == 0) a.counts[page] = off == 0 ? take : max(a.counts[page], off + take);
}

__global__ __launch_bounds__(256) void k_finalize(FinalizeArgs a) {
    const uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= uint64_t(a.pages) * a.width) return;
    const uint32_t n = a.counts[i / a.width];
    float mean = 0.0f;
    if (n) mean = a.sums[i] * (1.0f / float(n));
    if (a.means) a.means[i] = mean;
    if (a.summaries) {
        uint16_t hb = 0;
        const uint32_t e = recall16(mean, hb);
        if (e) raise_operand(a.status, e, a.epoch);
        a.summaries[i] = hb;
    }
}

// Batched byte copies (copy_bytes, stagein.cu:236-261): one workgroup per op.
// Host-link read probe: device-mapped pinned memory read by the CUs in
// 16-byte loads (four in flight per thread, grid-strided) and written to
// device memory.
__global__ __launch_bounds__(256) void k_link_read(const uint4 *src, uint4 *dst, uint64_t n16) {
    const uint64_t stride = uint64_t(gridDim.x) * 256;
    uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const uint4 a = src[i], b = src[i + stride], c = src[i + 2 * stride], d = src[i + 3 * stride];
        dst[i] = a;
        dst[i + stride] = b;
        dst[i + 2 * stride] = c;
        dst[i + 3 * stride] = d;
    }
    for (; i < n16; i += stride) dst[i] = src[i];
}

__global__ __launch_bounds__(256) void k_copy_ops(const CopyOp *ops, uint32_t n) {
    if (blockIdx.x >= n) return;
    const CopyOp op = ops[blockIdx.x];
    if (!op.src || !op.dst || !op.bytes) return;
    for (uint64_t off = 0; off < op.bytes; off += 0x40000000ull) {
        const uint64_t part = min(op.bytes - off, 0x40000000ull);
        copy_span(op.src + off, op.dst + off, uint32_t(part));
    }
}

// ---------------------------------------------------------------------------
// Seeded synthetic inputs (same arithmetic as the oracle's generator).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_synth(SynthArgs a) {
    const uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= a.count) return;
    switch (a.kind) {
    case kSynthNormalF16:
        static_cast<uint16_t *>(a.out)[i] = f2h(synth_normal(a.base, i));
        break;
    case kSynthScaledNormalF16:
        static_cast<uint16_t *>(a.out)[i] = f2h(__fmul_rn(synth_normal(a.base, i), a.scale[i % a.width]));
        break;
    case kSynthNormalF32:
        static_cast<float *>(a.out)[i] = synth_normal(a.base, i);
        break;
    case kSynthQ8: {
        uint8_t *blk = static_cast<uint8_t *>(a.out) + i * kQ8Bytes;
        for (int w = 0; w < 8; ++w) {
            const uint64_t r = synth_bits(a.base, i * 9 + w);
            for (int c = 0; c < 4; ++c)
                blk[2 + w * 4 + c] = uint8_t(int8_t(int((r >> (16 * c)) & 0xffffu) % 255 - 127));
        }
        const uint16_t d = f2h(synth_lerp(a.lo, a.hi, synth_unit24(synth_bits(a.base, i * 9 + 8))));
        blk[0] = uint8_t(d);
        blk[1] = uint8_t(d >> 8);
        break;
    }
    case kSynthQ41: {
        uint8_t *blk = static_cast<uint8_t *>(a.out) + i * kQ41Bytes;
        for (int w = 0; w < 2; ++w) {
            const uint64_t r = synth_bits(a.base, i * 4 + w);
            for (int c = 0; c < 8; ++c) blk[4 + w * 8 + c] = uint8_t(r >> (8 * c));
        }
        const uint16_t d = f2h(synth_lerp(a.lo, a.hi, synth_unit24(synth_bits(a.base, i * 4 + 2))));
        const uint16_t m = f2h(synth_lerp(a.lo2, a.hi2, synth_unit24(synth_bits(a.base, i * 4 + 3))));
        blk[0] = uint8_t(d); blk[1] = uint8_t(d >> 8);
        blk[2] = uint8_t(m); blk[3] = uint8_t(m >> 8);
        break;
    }
    case kSynthNormalQ8: {
        float x[kQK];
        for (int j = 0; j < kQK; ++j) x[j] = synth_normal(a.base, i * kQK + j);
        quant_block_q8(x, static_cast<uint8_t *>(a.out) + i * kQ8Bytes);
        break;
    }
    }
}

inline unsigned blocks_for(uint64_t threads, unsigned per = 256) {
    return unsigned((threads + per - 1) / per);
}

}  // namespace

// ---- launchers ------------------------------------------------------------
// One summary launch; start/stop (either may be null) are stamped with the
// kernel's own start and end.
template <class Kernel>
void launch_k_summary(Kernel kernel, dim3 grid, dim3 block, size_t lds, hipStream_t s, hipEvent_t start,
                      hipEvent_t stop, const SummaryArgs &a) {
    if (start || stop) hipExtLaunchKernelGGL(kernel, grid, block, uint32_t(lds), s, start, stop, 0u, a);
    else hipLaunchKernelGGL(kernel, grid, block, lds, s, a);
}

template <int BS>
void launch_summary_bs(int source, bool fuse, const SummaryArgs &a, uint64_t threads, size_t lds, hipStream_t s,
                       hipEvent_t start, hipEvent_t stop) {
    const dim3 grid(blocks_for(threads, BS)), block(BS);
    auto go = [&](auto kernel, size_t l) { launch_k_summary(kernel, grid, block, l, s, start, stop, a); };
    if (source == kSrcKeysF16 && fuse) go(k_summary<kSrcKeysF16, true, BS>, lds);
    else if (source == kSrcKeysF16) go(k_summary<kSrcKeysF16, false, BS>, 0);
    else if (source == kSrcKeysQ8 && fuse) go(k_summary<kSrcKeysQ8, true, BS>, lds);
    else if (source == kSrcKeysQ8) go(k_summary<kSrcKeysQ8, false, BS>, 0);
    else go(k_summary<kSrcSummary, true, BS>, lds);
}

template <int CPL>
void launch_summary_narrow(bool fuse, const SummaryArgs &a, size_t lds, hipStream_t s, hipEvent_t start,
                           hipEvent_t stop) {
    const dim3 grid(blocks_for(uint64_t(a.lanes) * a.pages * (a.width / CPL), 64)), block(64);
    if (fuse) launch_k_summary(k_summary<kSrcKeysF16, true, 64, CPL>, grid, block, lds, s, start, stop, a);
    else launch_k_summary(k_summary<kSrcKeysF16, false, 64, CPL>, grid, block, 0, s, start, stop, a);
}

constexpr uint64_t kSummarySpreadBlocks = 256;  // MI355X's CUs
hipError_t launch_summary(int source, bool fuse, const SummaryArgs &a, hipStream_t s, hipEvent_t start,
                          hipEvent_t stop) {
    (void)hipGetLastError();  // report only this launch\'s error
    const uint64_t threads = uint64_t(a.lanes) * a.pages * (a.width >> 3);
    const size_t lds = fuse && a.q_stage ? size_t(a.q.rows) * a.q.qheads * a.q.dim * 2 : 0;  // q_lds_buf
    // A launch of fewer 256-thread blocks than CUs leaves CUs idle: 64-thread
    // blocks spread the same key stream over four times as many CUs, and
    // fp16 rows are split over lanes of 4 or 2 channels until about four
    // waves per CU read them (a fused kv-head slice stays within a wave).
    if (blocks_for(threads) < kSummarySpreadBlocks) {
        const uint64_t waves = (threads + 63) / 64;
        const bool fits2 = a.width % 2 == 0 && (!fuse || a.q.dim / 2 <= 64);
        const bool fits4 = a.width % 4 == 0 && (!fuse || a.q.dim / 4 <= 64);
        if (source == kSrcKeysF16 && fits2 && 4 * waves <= 4 * kSummarySpreadBlocks)
            launch_summary_narrow<2>(fuse, a, lds, s, start, stop);
        else if (source == kSrcKeysF16 && fits4 && 2 * waves <= 4 * kSummarySpreadBlocks)
            launch_summary_narrow<4>(fuse, a, lds, s, start, stop);
        else
            launch_summary_bs<64>(source, fuse, a, threads, lds, s, start, stop);
    } else {
        launch_summary_bs<256>(source, fuse, a, threads, lds, s, start, stop);
    }
    return hipGetLastError();
}

hipError_t launch_pack_query(const PackQueryArgs &a, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch\'s error
    const uint64_t n = uint64_t(a.lanes) * a.q.rows * a.q.qheads * a.q.dim;
    hipLaunchKernelGGL(k_pack_query, dim3(blocks_for(n)), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_logits_mfma(const MfmaLogitsArgs &a, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch\'s error
    const dim3 grid((a.pages + 63) / 64, a.kvheads, a.lanes);
    hipLaunchKernelGGL(k_logits_mfma, grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

// Dynamic LDS of a selection tail: the keys of rows up to kTailLdsPages
// pages; for longer rows with fixed pages, their bitmap.
inline size_t tail_lds_bytes(const SelectArgs &a) {
    const uint32_t n = select_pages(a);
    if (n <= kTailLdsPages) return size_t(key_slot(n) + 1) * 8;
    return a.do_select && (a.n_mandatory || a.n_fixed) ? size_t((n + 31) / 32) * 4 : 0;
}

hipError_t launch_probs(const SelectArgs &a, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch\'s error
    if (a.pages > 1024 && a.aggregation == kAggMean && !a.fold && a.stats) {
        // long Mean rows: the units' statistics, then page slices + tail
        hipLaunchKernelGGL(k_unit_stats, dim3(a.units, a.lanes), dim3(256), 0, s, a);
        hipLaunchKernelGGL(k_mean_scores, dim3((a.pages + kScorePages - 1) / kScorePages, a.lanes), dim3(256),
                           tail_lds_bytes(a), s, a);
        return hipGetLastError();
    }
    if (a.pages <= kOnePages && a.units >= 1 && a.units <= kOneUnits && uint64_t(a.units) * a.pages <= 4096) {
        // few short softmax units: one workgroup per lane, terms in LDS
        const dim3 grid(a.lanes), block(kWave * a.units);
        const size_t lds = tail_lds_bytes(a) + size_t(a.units) * a.pages * 8;
        if (a.pages <= 64) hipLaunchKernelGGL(k_probs_one<1>, grid, block, lds, s, a);
        else if (a.pages <= 128) hipLaunchKernelGGL(k_probs_one<2>, grid, block, lds, s, a);
        else if (a.pages <= 256) hipLaunchKernelGGL(k_probs_one<4>, grid, block, lds, s, a);
        else hipLaunchKernelGGL(k_probs_one<8>, grid, block, lds, s, a);
        return hipGetLastError();
    }
    const uint32_t upb = units_per_block(a.pages);
    const dim3 grid((a.units + upb - 1) / upb, a.lanes), block(256);
    const size_t lds = tail_lds_bytes(a);
    if (a.pages <= 64) hipLaunchKernelGGL(k_probs<1>, grid, block, lds, s, a);
    else if (a.pages <= 128) hipLaunchKernelGGL(k_probs<2>, grid, block, lds, s, a);
    else if (a.pages <= 256) hipLaunchKernelGGL(k_probs<4>, grid, block, lds, s, a);
    else if (a.pages <= 512) hipLaunchKernelGGL(k_probs<8>, grid, block, lds, s, a);
    else if (a.pages <= 1024) hipLaunchKernelGGL(k_probs<16>, grid, block, lds, s, a);
    else hipLaunchKernelGGL(k_probs<0>, grid, block, lds, s, a);
    return hipGetLastError();
}

constexpr uint32_t kStackSpreadBlocks = 256;  // summary workgroups that fill MI355X's 256 CUs
hipError_t launch_stack_group(int source, StackGroupArgs g, hipStream_t s, hipEvent_t start, hipEvent_t stop) {
    (void)hipGetLastError();  // report only this launch\'s error
    const SummaryArgs &sa = g.s[0];
    const SelectArgs &pa = g.p[0];
    // A layer whose summaries take fewer workgroups than the GPU has CUs
    // leaves CUs idle if one workgroup walks all the group's layers: split
    // the layers into parts until the launch has a workgroup per CU.
    g.layer_blocks = g.m ? blocks_for(uint64_t(sa.lanes) * sa.pages * (sa.width / stack_cpl(source, sa.width, sa.page_tokens))) : 1;
    uint32_t parts = 1;
    if (g.m && g.layer_blocks < kStackSpreadBlocks)
        parts = min(g.m, (kStackSpreadBlocks + g.layer_blocks - 1) / g.layer_blocks);
    g.layers_per_part = g.m ? (g.m + parts - 1) / parts : 1;
    parts = g.m ? (g.m + g.layers_per_part - 1) / g.layers_per_part : 0;
    g.summary_blocks = g.layer_blocks * parts;
    const uint32_t sb = g.summary_blocks;
    const uint32_t probs_blocks = g.mp ? g.mp * g.probs_per_lane * pa.lanes : 0;
    const dim3 grid(unsigned(sb + probs_blocks)), block(256);
    const size_t q_lds_bytes = g.m && source == kSrcSummary && sa.q_stage ? size_t(2) * g.q_slot * 2 : 0;
    size_t keys = 0;  // the tails' keys or fixed-page bitmaps
    for (uint32_t i = 0; i < g.mp; ++i) keys = tail_lds_bytes(g.p[i]) > keys ? tail_lds_bytes(g.p[i]) : keys;
    size_t lds = q_lds_bytes > keys ? q_lds_bytes : keys;
    for (uint32_t i = 0; i < g.mp; ++i) {  // softmax workgroups' logits rows
        const SelectArgs &p = g.p[i];
        const uint32_t group = p.qheads / p.kvheads;
        if (p.summaries && probs_lds_fits(p.aggregation, group, p.pages)) {
            const size_t rows = size_t(probs_lds_rows(p.aggregation, group)) * p.pages * 8;
            lds = rows > lds ? rows : lds;
        }
    }
    const uint32_t pages = g.mp ? pa.pages : sa.pages;
    // start/stop: events stamped with the kernel's own start and end (no
    // markers on the stream between launches)
    auto go = [&](auto kernel) {
        if (start || stop) hipExtLaunchKernelGGL(kernel, grid, block, lds, s, start, stop, 0u, g);
        else hipLaunchKernelGGL(kernel, grid, block, lds, s, g);
    };
    const bool f16 = source == kSrcKeysF16, q8 = source == kSrcKeysQ8;
    if (pages <= 256) {
        if (f16) go(k_stack_group<kSrcKeysF16, 4>); else if (q8) go(k_stack_group<kSrcKeysQ8, 4>);
        else go(k_stack_group<kSrcSummary, 4>);
    } else if (pages <= 512) {
        if (f16) go(k_stack_group<kSrcKeysF16, 8>); else if (q8) go(k_stack_group<kSrcKeysQ8, 8>);
        else go(k_stack_group<kSrcSummary, 8>);
    } else if (pages <= 1024) {
        if (f16) go(k_stack_group<kSrcKeysF16, 16>); else if (q8) go(k_stack_group<kSrcKeysQ8, 16>);
        else go(k_stack_group<kSrcSummary, 16>);
    } else {
        if (f16) go(k_stack_group<kSrcKeysF16, 0>); else if (q8) go(k_stack_group<kSrcKeysQ8, 0>);
        else go(k_stack_group<kSrcSummary, 0>);
    }
    return hipGetLastError();
}

hipError_t launch_select(const SelectArgs &a, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch\'s error
    hipLaunchKernelGGL(k_select, dim3(a.lanes), dim3(256), tail_lds_bytes(a), s, a);
    return hipGetLastError();
}

hipError_t launch_fold_halves(const FoldArgs &a, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch\'s error
    hipLaunchKernelGGL(k_fold_halves, dim3(a.lanes), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_select_groups(const SelectArgs &a, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch\'s error
    hipLaunchKernelGGL(k_select_groups, dim3(a.lanes), dim3(256), group_select_lds(a.pages), s, a);
    return hipGetLastError();
}

hipError_t launch_graph_lrfu(GraphLrfuArgs a, const GraphLane *graphs, uint32_t lanes, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error
    const size_t lds = size_t(a.pages) * 8;
    for (uint32_t l0 = 0; l0 < lanes; l0 += kGraphLanes) {
        const uint32_t nl = lanes - l0 < kGraphLanes ? lanes - l0 : kGraphLanes;
        a.lane0 = l0;
        for (uint32_t i = 0; i < nl; ++i) a.graph[i] = graphs[l0 + i];
        hipLaunchKernelGGL(k_graph_lrfu, dim3(nl), dim3(kGraphThreads), lds, s, a);
        if (hipError_t e = hipGetLastError()) return e;
    }
    return hipSuccess;
}

hipError_t launch_gather(const GatherArgs &a, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch\'s error
    GatherArgs g = a;
    g.lds_per_wave = 0;
    for (uint32_t i = 0; i < a.n_planes; ++i) {
        const GatherPlane &p = a.plane[i];
        if (p.mode == kModeCopy || p.format == kFmtF16) continue;
        uint32_t need = (a.chunk_rows * p.src_row + 15u) & ~15u;
        if (p.mode == kModeRopeFwht) need += p.width * 4;  // the binary32 row
        g.lds_per_wave = need > g.lds_per_wave ? need : g.lds_per_wave;
    }
    const uint32_t wpb = a.threads / kWave;
    const uint64_t items = uint64_t(a.lanes) * a.k * a.n_planes * a.chunks;
    const uint64_t blocks = (items + wpb - 1) / wpb;
    const uint32_t wgs = unsigned(blocks < a.workgroups ? blocks : a.workgroups);
    hipLaunchKernelGGL(k_gather, dim3(wgs ? wgs : 1), dim3(a.threads), size_t(g.lds_per_wave) * wpb, s, g);
    return hipGetLastError();
}

hipError_t launch_accumulate(const AccumulateArgs &a, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch\'s error
    hipLaunchKernelGGL(k_accumulate, dim3(blocks_for(uint64_t(a.segments) * a.width)), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_finalize(const FinalizeArgs &a, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch\'s error
    hipLaunchKernelGGL(k_finalize, dim3(blocks_for(uint64_t(a.pages) * a.width)), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_link_read(const void *src, void *dst, uint64_t bytes, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error
    hipLaunchKernelGGL(k_link_read, dim3(1024), dim3(256), 0, s, static_cast<const uint4 *>(src),
                       static_cast<uint4 *>(dst), bytes / 16);
    return hipGetLastError();
}

hipError_t launch_copy_ops(const CopyOp *ops, uint32_t n, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch\'s error
    hipLaunchKernelGGL(k_copy_ops, dim3(n), dim3(256), 0, s, ops, n);
    return hipGetLastError();
}

hipError_t launch_synth(const SynthArgs &a, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch\'s error
    hipLaunchKernelGGL(k_synth, dim3(blocks_for(a.count)), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace kvr
