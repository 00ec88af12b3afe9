// kvr_device.hpp -- device helpers shared by the recall kernels (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kvr {

constexpr int kWave = 64;

// ---- scalar conversions ---------------------------------------------------
// v_cvt_f16_f32 rounds to nearest even (default MODE), keeps binary16
// subnormals and overflows to infinity: the IEEE conversion the reference's
// f32_to_f16 (kvmem/src/host/raw_kv_store.cpp:43-78) spells out in integers.
__device__ __forceinline__ float h2f(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}
// The empty asm pins `f` as a rounded binary32 value: without it the
// compiler may fold a producing multiply or fma into v_fma_mixlo_f16, which
// rounds once to binary16 where the reference rounds to binary32 first.
__device__ __forceinline__ uint16_t f2h(float f) {
    asm volatile("" : "+v"(f));
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}
__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }

// The recall operand boundary (graph_recall.cpp:295-320): finite values are
// rounded to binary16; NaN/inf and values rounding to infinity are errors.
enum : uint32_t { kOperandOk = 0, kOperandNonfinite = 1, kOperandRange = 2 };
__device__ __forceinline__ uint32_t recall16(float v, uint16_t &h) {
    if (!__builtin_isfinite(v)) return kOperandNonfinite;
    h = f2h(v);
    return (h & 0x7fffu) == 0x7c00u ? kOperandRange : kOperandOk;
}

// Device status words, one per error class; each holds the epoch (call
// number) of the latest call that raised it.
enum : uint32_t {
    kStatusNonfinite = 0, kStatusRange = 1, kStatusScores = 2, kStatusGraph = 3, kStatusBudget = 4, kStatusWords = 5
};
__device__ __forceinline__ void raise_status(uint32_t *status, uint32_t word, uint32_t epoch) {
    atomicMax(status + word, epoch);
}
__device__ __forceinline__ void raise_operand(uint32_t *status, uint32_t code, uint32_t epoch) {
    if (code == kOperandNonfinite) raise_status(status, kStatusNonfinite, epoch);
    if (code == kOperandRange) raise_status(status, kStatusRange, epoch);
}
// Device-scope (all XCDs) relaxed stores and loads: they write through and
// read past the XCD's own L2, so data published this way between
// workgroups of one launch needs neither an L2 writeback on the writer's
// side nor an L2 invalidate on the reader's, only the stores' completion.
template <class T> __device__ __forceinline__ void store_device(T *p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T> __device__ __forceinline__ T load_device(const T *p) {
    return __hip_atomic_load(const_cast<T *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Raw buffer resource over `bytes` bytes from `p` (dword 3 selects the
// 32-bit data format, which enables untyped loads).  Loads at offsets past
// `bytes` return zeros instead of touching memory; offsets are 32-bit, so
// no 64-bit address arithmetic sits between a wave's loads.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), short(0), int(bytes), 0x00020000);
}
constexpr int kBufferNontemporal = 2;  // cache-policy bits of a streaming load
// Waits until this thread's vector memory operations have completed
// (s_waitcnt vmcnt(0)).  The memory clobber keeps the compiler from moving
// any load or store across the wait, so stores issued before it are
// complete -- for device-scope stores, written through to the device's
// coherence point -- before anything after it issues.
__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ __forceinline__ bool epoch_failed(const uint32_t *status, uint32_t epoch) {
    // all three loads in flight together
    const uint32_t s0 = load_device(status + kStatusNonfinite), s1 = load_device(status + kStatusRange),
                   s2 = load_device(status + kStatusScores);
    return (s0 == epoch) | (s1 == epoch) | (s2 == epoch);
}

// Workgroup barrier that orders LDS only.  __syncthreads() also waits for
// the thread's outstanding global stores, a full memory round trip when
// HBM is busy; use this one where the barrier publishes LDS and nothing else.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ---- wave reductions (64 lanes) --------------------------------------------
// Cross-lane moves are DPP (VALU) within 16-lane rows and readlane across
// rows; no LDS permutes.  Every lane gets the same result, combined in one
// fixed order.
namespace dpp {
constexpr int kQuadBcast0 = 0x00;    // quad_perm [0,0,0,0]
constexpr int kQuadXor1 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int kHalfMirror = 0x141;   // lane i <-> 7-i within each 8 lanes
constexpr int kMirror = 0x140;       // lane i <-> 15-i within each row
constexpr int kRowShr = 0x110;       // + n: lane i reads lane i-n of its row

// Row shifts leave the first lanes of a row without a source: those keep
// zero.  The other controls give every lane a source, so no old value is
// named (bound_ctrl set, which then changes nothing) and the move can fold
// into the instruction that consumes it (v_add_f32_dpp and the like).
template <int CTRL>
__device__ __forceinline__ int move32(int v) {
    if constexpr ((CTRL & 0x1f0) == kRowShr) return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
    else return __builtin_amdgcn_mov_dpp(v, CTRL, 0xf, 0xf, true);
}
template <int CTRL, class T>
__device__ __forceinline__ T move(T v) {
    static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32- or 64-bit lanes");
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(T, move32<CTRL>(__builtin_bit_cast(int, v)));
    } else {
        const uint64_t u = __builtin_bit_cast(uint64_t, v);
        const uint32_t lo = uint32_t(move32<CTRL>(int(uint32_t(u))));
        const uint32_t hi = uint32_t(move32<CTRL>(int(uint32_t(u >> 32))));
        return __builtin_bit_cast(T, (uint64_t(hi) << 32) | lo);
    }
}

template <class T>
__device__ __forceinline__ T readlane(T v, int lane) {
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
    } else {
        const uint64_t u = __builtin_bit_cast(uint64_t, v);
        const uint32_t lo = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(u)), lane));
        const uint32_t hi = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(u >> 32)), lane));
        return __builtin_bit_cast(T, (uint64_t(hi) << 32) | lo);
    }
}

// op over aligned groups of `width` lanes (1, 2, 4, 8 or 16), every lane
// of a group gets its group's result.
template <class T, class Op>
__device__ __forceinline__ T group_reduce(T v, int width, Op op) {
    if (width >= 2) v = op(v, move<kQuadXor1>(v));
    if (width >= 4) v = op(v, move<kQuadXor2>(v));
    if (width >= 8) v = op(v, move<kHalfMirror>(v));
    if (width >= 16) v = op(v, move<kMirror>(v));
    return v;
}

template <class T, class Op>
__device__ __forceinline__ T wave_reduce(T v, Op op) {
    v = group_reduce(v, 16, op);
    return op(op(readlane(v, 0), readlane(v, 16)), op(readlane(v, 32), readlane(v, 48)));
}

struct Add { template <class T> __device__ T operator()(T a, T b) const { return a + b; } };
struct Max { template <class T> __device__ T operator()(T a, T b) const { return b > a ? b : a; } };
// fmaxf: a NaN operand gives the other one
struct FMax { __device__ float operator()(float a, float b) const { return fmaxf(a, b); } };
struct And { template <class T> __device__ T operator()(T a, T b) const { return a & b; } };
struct Or { template <class T> __device__ T operator()(T a, T b) const { return a | b; } };
}  // namespace dpp

template <class T> __device__ __forceinline__ T wave_sum(T v) { return dpp::wave_reduce(v, dpp::Add()); }
template <class T> __device__ __forceinline__ T wave_max(T v) { return dpp::wave_reduce(v, dpp::Max()); }
__device__ __forceinline__ float wave_fmax(float v) { return dpp::wave_reduce(v, dpp::FMax()); }
__device__ __forceinline__ uint64_t wave_and(uint64_t v) { return dpp::wave_reduce(v, dpp::And()); }
__device__ __forceinline__ uint64_t wave_or(uint64_t v) { return dpp::wave_reduce(v, dpp::Or()); }

// Sum over aligned groups of `width` lanes (power of two <= 64).
template <class T> __device__ __forceinline__ T group_sum(T v, int width) {
    v = dpp::group_reduce(v, width < 16 ? width : 16, dpp::Add());
    for (int o = 16; o < width; o <<= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// group_sum(v, width) over `width` groups of G adjacent lanes, every lane
// of a group holding its group's value: the same pairwise tree, taken at
// lane strides G, 2G, ...  (DPP mirrors pair the groups as the xor strides
// do: the lane read belongs to the partner group, whose lanes all agree).
template <int G, class T> __device__ __forceinline__ T spread_group_sum(T v, int width) {
    static_assert(G == 1 || G == 2 || G == 4, "groups within a quad");
    const int end = G * width;
    int s = G;
    if (s == 1 && s < end) v += dpp::move<dpp::kQuadXor1>(v), s = 2;
    if (s == 2 && s < end) v += dpp::move<dpp::kQuadXor2>(v), s = 4;
    if (s == 4 && s < end) v += dpp::move<dpp::kHalfMirror>(v), s = 8;
    if (s == 8 && s < end) v += dpp::move<dpp::kMirror>(v), s = 16;
    for (; s < end; s <<= 1) v += __shfl_xor(v, s, kWave);
    return v;
}

// Inclusive prefix sum over the wave: rows by DPP shifts, then the totals
// of the rows below.
__device__ __forceinline__ uint32_t wave_inclusive_scan(uint32_t v) {
    v += dpp::move<dpp::kRowShr + 1>(v);
    v += dpp::move<dpp::kRowShr + 2>(v);
    v += dpp::move<dpp::kRowShr + 4>(v);
    v += dpp::move<dpp::kRowShr + 8>(v);
    const uint32_t t0 = dpp::readlane(v, 15), t1 = dpp::readlane(v, 31), t2 = dpp::readlane(v, 47);
    const uint32_t row = (threadIdx.x & (kWave - 1)) >> 4;
    return v + (row >= 1 ? t0 : 0u) + (row >= 2 ? t1 : 0u) + (row >= 3 ? t2 : 0u);
}

// The value of lane `src` (uniform `src`).
template <class T> __device__ __forceinline__ T wave_bcast(T v, int src) { return dpp::readlane(v, src); }

// ---- block formats ---------------------------------------------------------
constexpr int kQK = 32;
constexpr int kQ8Bytes = 34;  // {fp16 d; int8 qs[32]}
constexpr int kQ41Bytes = 20; // {fp16 d; fp16 m; uint8 qs[16]}

__device__ __forceinline__ uint16_t ld_u16(const uint8_t *p) {
    return uint16_t(p[0] | (uint16_t(p[1]) << 8));
}

// ---- seeded synthetic inputs --------------------------------------------
// bits(c) = fmix64(base + (c + 1) * G); base is computed on the host.
constexpr uint64_t kSynthG = 0x9E3779B97F4A7C15ull;
__host__ __device__ __forceinline__ uint64_t fmix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__host__ __device__ __forceinline__ uint64_t synth_base(uint64_t seed, uint64_t stream) {
    return fmix64(fmix64(seed + kSynthG) ^ ((stream + 1) * 0xD1B54A32D192ED03ull));
}
__device__ __forceinline__ uint64_t synth_bits(uint64_t base, uint64_t counter) {
    return fmix64(base + (counter + 1) * kSynthG);
}
// N(0,1) by Box-Muller: normals 2j and 2j+1 are R cos(2 pi u2) and
// R sin(2 pi u2), R = sqrt(-2 ln u1), where draws 2j and 2j+1 give u1 in
// (0, 1] and u2 in [0, 1) with 53 bits each.  Everything is binary64 from
// correctly rounded +, -, *, / only, so the oracle's statement of the same
// steps gives the same bits on the CPU:
//   ln x   = e ln 2 + 2 atanh(s), s = (m - 1)/(m + 1), x = m 2^e with m in
//            (sqrt(1/2), sqrt(2)], the atanh series to s^23;
//   sqrt y = six Newton steps y_{k+1} = (y_k + y/y_k)/2 from the power of
//            two that halves y's exponent;
//   2 pi t: the quarter turn q = floor(4t) and an eighth-turn reflection
//            are exact, then Taylor series of sin and cos on [0, pi/4] (to
//            x^15 and x^16).
// No contraction into fused multiply-adds.  One rounding to binary32 last.
__device__ __forceinline__ double synth_ln(double x) {
#pragma clang fp contract(off)
    uint64_t b = uint64_t(__double_as_longlong(x));
    int e = int((b >> 52) & 0x7ffu) - 1023;
    double m = __longlong_as_double((long long)((b & 0x000fffffffffffffull) | 0x3ff0000000000000ull));
    if (m > 1.4142135623730951) {
        m = m * 0.5;
        e += 1;
    }
    const double s = (m - 1.0) / (m + 1.0), s2 = s * s;
    double p = 1.0 / 23.0;
    p = 1.0 / 21.0 + s2 * p;
    p = 1.0 / 19.0 + s2 * p;
    p = 1.0 / 17.0 + s2 * p;
    p = 1.0 / 15.0 + s2 * p;
    p = 1.0 / 13.0 + s2 * p;
    p = 1.0 / 11.0 + s2 * p;
    p = 1.0 / 9.0 + s2 * p;
    p = 1.0 / 7.0 + s2 * p;
    p = 1.0 / 5.0 + s2 * p;
    p = 1.0 / 3.0 + s2 * p;
    const double t = s2 * p;
    return double(e) * 0.69314718055994530942 + 2.0 * (s + s * t);
}
__device__ __forceinline__ double synth_sqrt(double y) {
#pragma clang fp contract(off)
    if (y == 0.0) return 0.0;
    const int e = int((uint64_t(__double_as_longlong(y)) >> 52) & 0x7ffu) - 1023;
    double r = __longlong_as_double((long long)(uint64_t((e >> 1) + 1023) << 52));
#pragma unroll
    for (int k = 0; k < 6; ++k) r = (r + y / r) * 0.5;
    return r;
}
// cos (SIN false) or sin (SIN true) of 2 pi t, t in [0, 1)
template <bool SIN>
__device__ __forceinline__ double synth_turn(double t) {
#pragma clang fp contract(off)
    const int q = int(t * 4.0);  // exact
    double r = t - double(q) * 0.25;
    const bool swap = r > 0.125;
    if (swap) r = 0.25 - r;
    const double x = r * 6.28318530717958647692, x2 = x * x;
    double c = 1.0 / 20922789888000.0;
    c = 1.0 / 87178291200.0 - x2 * c;
    c = 1.0 / 479001600.0 - x2 * c;
    c = 1.0 / 3628800.0 - x2 * c;
    c = 1.0 / 40320.0 - x2 * c;
    c = 1.0 / 720.0 - x2 * c;
    c = 1.0 / 24.0 - x2 * c;
    c = 0.5 - x2 * c;
    c = 1.0 - x2 * c;
    double sn = 1.0 / 1307674368000.0;
    sn = 1.0 / 6227020800.0 - x2 * sn;
    sn = 1.0 / 39916800.0 - x2 * sn;
    sn = 1.0 / 362880.0 - x2 * sn;
    sn = 1.0 / 5040.0 - x2 * sn;
    sn = 1.0 / 120.0 - x2 * sn;
    sn = 1.0 / 6.0 - x2 * sn;
    sn = 1.0 - x2 * sn;
    sn = x * sn;
    const double cr = swap ? sn : c, sr = swap ? c : sn;  // cos and sin of 2 pi r
    if constexpr (SIN) return q == 0 ? sr : q == 1 ? cr : q == 2 ? -sr : -cr;
    else return q == 0 ? cr : q == 1 ? -sr : q == 2 ? -cr : sr;
}
__device__ __forceinline__ float synth_normal(uint64_t base, uint64_t index) {
#pragma clang fp contract(off)
    const uint64_t j = index >> 1;
    const uint64_t r1 = synth_bits(base, 2 * j), r2 = synth_bits(base, 2 * j + 1);
    const double u1 = double((r1 >> 11) + 1) * 1.1102230246251565404e-16;  // 2^-53
    const double u2 = double(r2 >> 11) * 1.1102230246251565404e-16;
    const double radius = synth_sqrt(-2.0 * synth_ln(u1));
    return float(radius * ((index & 1) ? synth_turn<true>(u2) : synth_turn<false>(u2)));
}
__device__ __forceinline__ float synth_unit24(uint64_t r) {
    return float(r >> 40) * 5.9604644775390625e-08f;
}
// lo + u * (hi - lo) with three separate roundings: contraction into a fused
// multiply-add is switched off here (HIP's __fadd_rn/__fmul_rn are plain
// operators that clang would otherwise fuse).
__device__ __forceinline__ float synth_lerp(float lo, float hi, float u) {
#pragma clang fp contract(off)
    const float span = hi - lo;
    const float prod = u * span;
    return lo + prod;
}

}  // namespace kvr
