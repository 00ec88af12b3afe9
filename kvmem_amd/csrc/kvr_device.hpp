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
enum : uint32_t { kStatusNonfinite = 0, kStatusRange = 1, kStatusScores = 2, kStatusWords = 4 };
__device__ __forceinline__ void raise_status(uint32_t *status, uint32_t word, uint32_t epoch) {
    atomicMax(status + word, epoch);
}
__device__ __forceinline__ void raise_operand(uint32_t *status, uint32_t code, uint32_t epoch) {
    if (code == kOperandNonfinite) raise_status(status, kStatusNonfinite, epoch);
    if (code == kOperandRange) raise_status(status, kStatusRange, epoch);
}
__device__ __forceinline__ bool epoch_failed(const uint32_t *status, uint32_t epoch) {
    return status[kStatusNonfinite] == epoch || status[kStatusRange] == epoch ||
           status[kStatusScores] == epoch;
}

// ---- wave reductions (64 lanes) --------------------------------------------
template <class T> __device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}
template <class T> __device__ __forceinline__ T wave_max(T v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const T w = __shfl_xor(v, o, kWave);
        v = w > v ? w : v;
    }
    return v;
}
// Sum over aligned groups of `width` lanes (power of two <= 64).
template <class T> __device__ __forceinline__ T group_sum(T v, int width) {
    for (int o = width >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}
// Inclusive prefix sum over the wave.
__device__ __forceinline__ uint32_t wave_inclusive_scan(uint32_t v) {
    const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const uint32_t w = __shfl_up(v, o, kWave);
        if (lane >= o) v += w;
    }
    return v;
}

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
// Irwin-Hall(12) - 6: exact in binary64, then one rounding to binary32.
__device__ __forceinline__ float synth_normal(uint64_t base, uint64_t index) {
    int64_t total = 0;
#pragma unroll
    for (uint64_t j = 0; j < 6; ++j) {
        const uint64_t r = synth_bits(base, index * 6 + j);
        total += int64_t(r >> 40) + int64_t((r >> 16) & 0xffffffu);
    }
    return float(double(total - 100663296) * 5.9604644775390625e-08);
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
