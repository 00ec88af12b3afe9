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
// Here the first step reads every key once: a workgroup owns one page of one
// kv-head and every (sampled row, query head of the group) pair of a tile,
// each lane one token of the page.  The lane decodes its token's key row
// 32 values (one block) at a time into binary32 and folds them into all the
// tile's dot products with the query tile in LDS (the reference re-reads the
// page once per query head and row).  The page log-sum-exp of each pair is
// a workgroup max and sum.  The second kernel does the normalization and
// the head average for one row per workgroup.  All arithmetic is binary32,
// as in the reference.
#include "kvr_device.hpp"
#include "kvr_internal.hpp"

namespace kvr {
namespace {

constexpr int kAttnThreads = 256;
constexpr int kAttnWaves = kAttnThreads / kWave;
constexpr uint32_t kAttnMaxDim = 256;

typedef uint32_t u32x4a __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float scalar_at(const uint8_t *p, uint32_t scalar, uint32_t i) {
    if (scalar == kScalarF32) return reinterpret_cast<const float *>(p)[i];
    const uint16_t h = reinterpret_cast<const uint16_t *>(p)[i];
    return scalar == kScalarF16 ? h2f(h) : bf2f(h);
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
        const uintptr_t a = reinterpret_cast<uintptr_t>(p);
        const uint32_t *base = reinterpret_cast<const uint32_t *>(a & ~uintptr_t(3));
        r.odd = uint32_t(a & 2);
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

// One page of one kv-head for a tile of NP (row, query head) pairs: pair
// p0 + i is sampled row (p0+i)/group and query head kv*group + (p0+i)%group.
template <int KF, int NP>
__global__ __launch_bounds__(kAttnThreads) void k_attn_lse(AttnArgs a) {
    __shared__ float qs[NP * kAttnMaxDim];
    __shared__ float red[2][kAttnWaves][NP];
    const uint32_t page = blockIdx.x % a.pages, kv = blockIdx.x / a.pages;
    const uint32_t p0 = blockIdx.y * NP, npairs = a.n_rows * a.group;
    const uint32_t dim = a.dim, tid = threadIdx.x;
    for (uint32_t i = tid; i < NP * dim; i += kAttnThreads) {
        const uint32_t p = p0 + i / dim;
        float v = 0.0f;
        if (p < npairs) {
            const uint32_t r = a.rows[p / a.group], h = kv * a.group + p % a.group;
            v = scalar_at(a.q + r * a.q_row_stride + h * a.q_head_stride, a.q_scalar, i % dim);
        }
        qs[i] = v;
    }
    const uint8_t *mask_row[NP];
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        const uint32_t p = min(p0 + i, npairs - 1);
        mask_row[i] = a.mask + a.rows[p / a.group] * a.mask_row_stride;
    }
    lds_barrier();

    float m[NP], s[NP];
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        m[i] = -__builtin_inff();
        s[i] = 0.0f;
    }
    const uint32_t t0 = page * a.page_tokens;
    const uint32_t t1 = min(t0 + a.page_tokens, a.tokens);
    const uint32_t nb = dim / 32;
    for (uint32_t t = t0 + tid; t < t1; t += kAttnThreads) {
        float bias[NP];
#pragma unroll
        for (int i = 0; i < NP; ++i) bias[i] = scalar_at(mask_row[i], a.mask_scalar, t);
        const uint8_t *row = a.k + t * a.k_row_stride + kv * a.k_head_stride;
        float acc[NP];
#pragma unroll
        for (int i = 0; i < NP; ++i) acc[i] = 0.0f;
        RawBlock<KF> cur = load_block<KF>(row, 0);
        for (uint32_t b = 0; b < nb; ++b) {
            // next block's loads go out before this block is used
            const RawBlock<KF> next = load_block<KF>(row, min(b + 1, nb - 1));
            float kv32[32];
            decode_block<KF>(cur, kv32);
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                const float4 *qv = reinterpret_cast<const float4 *>(qs + i * dim + 32 * b);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float4 q4 = qv[j];
                    acc[i] = __builtin_fmaf(q4.x, kv32[4 * j], acc[i]);
                    acc[i] = __builtin_fmaf(q4.y, kv32[4 * j + 1], acc[i]);
                    acc[i] = __builtin_fmaf(q4.z, kv32[4 * j + 2], acc[i]);
                    acc[i] = __builtin_fmaf(q4.w, kv32[4 * j + 3], acc[i]);
                }
            }
            cur = next;
        }
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            if (!__builtin_isfinite(bias[i])) continue;
            float l = acc[i] * a.scale;
            if (a.softcap > 0.0f) l = a.softcap * tanhf(l / a.softcap);
            l += bias[i];
            const float nm = fmaxf(m[i], l);
            s[i] = s[i] * expf(m[i] - nm) + expf(l - nm);
            m[i] = nm;
        }
    }

    // Page log-sum-exp of each pair: max over the workgroup, then the sum of
    // the lanes' partial sums rescaled to it (lanes that saw no token add 0).
    const uint32_t w = tid / kWave, lane = tid % kWave;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        const float wm = wave_max(m[i]);
        if (lane == 0) red[0][w][i] = wm;
    }
    lds_barrier();
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        float mx = red[0][0][i];
#pragma unroll
        for (int j = 1; j < kAttnWaves; ++j) mx = fmaxf(mx, red[0][j][i]);
        const float e = wave_sum(s[i] > 0.0f ? s[i] * expf(m[i] - mx) : 0.0f);
        if (lane == 0) red[1][w][i] = e;
    }
    lds_barrier();
    if (tid < NP && p0 + tid < npairs) {
        const uint32_t p = p0 + tid;
        float mx = red[0][0][tid], total = 0.0f;
#pragma unroll
        for (int j = 1; j < kAttnWaves; ++j) mx = fmaxf(mx, red[0][j][tid]);
#pragma unroll
        for (int j = 0; j < kAttnWaves; ++j) total += red[1][j][tid];
        const uint32_t r = p / a.group, h = kv * a.group + p % a.group;
        a.lse[(uint64_t(r) * a.heads + h) * a.pages + page] = total > 0.0f ? mx + logf(total) : -__builtin_inff();
    }
}

// Masses of one sampled row: per head, the max and 1/sum of exp over pages
// (one wave per head), then for each page the head average of
// exp(lse - max) * (1/sum).
__global__ __launch_bounds__(kAttnThreads) void k_attn_mass(AttnArgs a) {
    extern __shared__ float norm[];  // [heads][2]
    const uint32_t r = blockIdx.x, tid = threadIdx.x, w = tid / kWave, lane = tid % kWave;
    const float *lse = a.lse + uint64_t(r) * a.heads * a.pages;
    for (uint32_t h = w; h < a.heads; h += kAttnWaves) {
        const float *row = lse + uint64_t(h) * a.pages;
        float mx = -__builtin_inff();
        for (uint32_t p = lane; p < a.pages; p += kWave) mx = fmaxf(mx, row[p]);
        mx = wave_max(mx);
        float sum = 0.0f;
        for (uint32_t p = lane; p < a.pages; p += kWave) sum += expf(row[p] - mx);
        sum = wave_sum(sum);
        if (lane == 0) {
            norm[2 * h] = mx;
            norm[2 * h + 1] = 1.0f / sum;
        }
    }
    lds_barrier();
    for (uint32_t p = tid; p < a.pages; p += kAttnThreads) {
        float acc = 0.0f;
        for (uint32_t h = 0; h < a.heads; ++h) acc += expf(lse[uint64_t(h) * a.pages + p] - norm[2 * h]) * norm[2 * h + 1];
        a.mass[uint64_t(r) * a.pages + p] = acc / float(a.heads);
    }
}

template <int KF>
hipError_t launch_lse(const AttnArgs &a, uint32_t np, hipStream_t s) {
    const uint32_t npairs = a.n_rows * a.group;
    const dim3 grid(a.kvheads * a.pages, (npairs + np - 1) / np);
    if (np == 4) hipLaunchKernelGGL((k_attn_lse<KF, 4>), grid, dim3(kAttnThreads), 0, s, a);
    else if (np == 8) hipLaunchKernelGGL((k_attn_lse<KF, 8>), grid, dim3(kAttnThreads), 0, s, a);
    else hipLaunchKernelGGL((k_attn_lse<KF, 16>), grid, dim3(kAttnThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_attention(const AttnArgs &a, hipStream_t s) {
    const uint32_t npairs = a.n_rows * a.group;
    const uint32_t np = npairs <= 4 ? 4 : npairs <= 8 ? 8 : 16;
    hipError_t e = hipErrorInvalidValue;
    switch (a.k_format) {
    case kKeyF16: e = launch_lse<kKeyF16>(a, np, s); break;
    case kKeyBF16: e = launch_lse<kKeyBF16>(a, np, s); break;
    case kKeyF32: e = launch_lse<kKeyF32>(a, np, s); break;
    case kKeyQ8: e = launch_lse<kKeyQ8>(a, np, s); break;
    case kKeyQ4: e = launch_lse<kKeyQ4>(a, np, s); break;
    case kKeyQ5: e = launch_lse<kKeyQ5>(a, np, s); break;
    default: break;
    }
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_attn_mass, dim3(a.n_rows), dim3(kAttnThreads), size_t(a.heads) * 2 * sizeof(float), s, a);
    return hipGetLastError();
}

}  // namespace kvr
