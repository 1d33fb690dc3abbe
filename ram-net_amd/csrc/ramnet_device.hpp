// Device-side helpers shared by the RAM-Net HIP kernels (gfx950, wave64).
//
// Storage types, the total order used for top-K selection, sorting networks
// over per-lane register arrays, and the gated-sparse-update (GSU) scalar math.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ramnet {

// Buffer resource word 3 for untyped 32-bit accesses on gfx9 parts.
constexpr int kBufWord3 = 0x00020000;

constexpr int kWave = 64;
// Index value marking an invalid (padding) top-K entry. Real content
// indices are < A < 2^30, so a padding entry never collides with one.
constexpr int kNoIdx = 0x7fffffff;

// bfloat16 kept as raw bits: conversion is done explicitly with
// round-to-nearest-even, matching torch's float -> bfloat16 cast.
struct bf16_t {
    uint16_t bits;
};

__device__ __forceinline__ float load_f32(const float *p) { return *p; }
__device__ __forceinline__ float load_f32(const _Float16 *p) { return static_cast<float>(*p); }
__device__ __forceinline__ float load_f32(const bf16_t *p) {
    return __uint_as_float(static_cast<uint32_t>(p->bits) << 16);
}

// The raw storage bits of one element (zero-extended) and their value as
// float. Converting at the use rather than at the load keeps a prefetched
// load from waiting for its data before the value is needed.
__device__ __forceinline__ uint32_t load_bits(const float *p) { return __float_as_uint(*p); }
__device__ __forceinline__ uint32_t load_bits(const _Float16 *p) { return *reinterpret_cast<const uint16_t *>(p); }
__device__ __forceinline__ uint32_t load_bits(const bf16_t *p) { return p->bits; }
template<typename T>
__device__ __forceinline__ float bits_f32(uint32_t b) {
    if constexpr (sizeof(T) == 4) {
        return __uint_as_float(b);
    } else if constexpr (__is_same(T, bf16_t)) {
        return __uint_as_float(b << 16);
    } else {
        return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(b)));
    }
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u)  // NaN: keep it a quiet NaN
        return static_cast<uint16_t>((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

// Natural logarithm as the hardware log2 (v_log_f32) times ln 2, for the
// log-sum-exp terms of the address search. Its error (a few ulp) shifts every
// candidate score of a digit, or every top-K value, by the same amount, so it
// never changes a ranking; inputs are sums of exponentials >= 1.
__device__ __forceinline__ float log_sum(float x) { return __builtin_amdgcn_logf(x) * 0.6931471805599453f; }

__device__ __forceinline__ void store_f32(float *p, float v) { *p = v; }
__device__ __forceinline__ void store_f32(_Float16 *p, float v) { *p = static_cast<_Float16>(v); }
__device__ __forceinline__ void store_f32(bf16_t *p, float v) { p->bits = f32_to_bf16_bits(v); }

// Total order of top-K candidates: higher score first, then lower content
// index. -inf scores tie with each other and fall back to the index order.
__device__ __forceinline__ bool before(float av, int ai, float bv, int bi) {
    return av > bv || (av == bv && ai < bi);
}

// Compare-exchange so that (v[i], id[i]) ends up ordered before (v[l], id[l]).
template<int N>
__device__ __forceinline__ void cmp_swap(float (&v)[N], int (&id)[N], int i, int l) {
    const bool sw = before(v[l], id[l], v[i], id[i]);
    const float tv = v[i];
    const int ti = id[i];
    v[i] = sw ? v[l] : v[i];
    id[i] = sw ? id[l] : id[i];
    v[l] = sw ? tv : v[l];
    id[l] = sw ? ti : id[l];
}

// Bitonic sort of the sub-range [OFF, OFF+N) of a register array into the
// total order above. N is a power of two; every index is a compile-time
// constant so the arrays stay in VGPRs.
template<int N, int OFF, int M>
__device__ __forceinline__ void bitonic_sort(float (&v)[M], int (&id)[M]) {
#pragma unroll
    for (int k = 2; k <= N; k <<= 1) {
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
#pragma unroll
            for (int i = 0; i < N; ++i) {
                const int l = i ^ j;
                if (l > i) {
                    if ((i & k) == 0)
                        cmp_swap(v, id, OFF + i, OFF + l);
                    else
                        cmp_swap(v, id, OFF + l, OFF + i);
                }
            }
        }
    }
}

// Given two sorted lists a and b of length K, leave in a the sorted top-K of
// their union. Pairing a[i] with b[K-1-i] keeps the better of each pair,
// which yields the top-K as a bitonic sequence; half-cleaners then sort it.
template<int K>
__device__ __forceinline__ void merge_topk(float (&av)[K], int (&ai)[K], const float (&bv)[K], const int (&bi)[K]) {
#pragma unroll
    for (int i = 0; i < K; ++i) {
        const bool take_b = before(bv[K - 1 - i], bi[K - 1 - i], av[i], ai[i]);
        av[i] = take_b ? bv[K - 1 - i] : av[i];
        ai[i] = take_b ? bi[K - 1 - i] : ai[i];
    }
#pragma unroll
    for (int j = K >> 1; j > 0; j >>= 1) {
#pragma unroll
        for (int i = 0; i < K; ++i) {
            const int l = i ^ j;
            if (l > i)
                cmp_swap(av, ai, i, l);
        }
    }
}

// Forget coefficient of the gated sparse update for write weight w and
// forget control g:
//   alpha = (1 - w) / (1 - w + e^g w).
// For g >= 0 numerator and denominator are rescaled by e^-g so that the
// exponential stays <= 1 (same value, no overflow for large g).
__device__ __forceinline__ float gsu_alpha(float w, float g) {
    const bool pos = g >= 0.f;
    const float eg = expf(pos ? -g : g);
    const float cw = 1.f - w;
    const float den = pos ? fmaf(eg, cw, w) : fmaf(eg, w, cw);
    const float num = pos ? cw * eg : cw;
    return num / den;
}

// Non-negative remainder of a position modulo the slot count.
__device__ __forceinline__ int pos_mod(int pos, int A) {
    if ((A & (A - 1)) == 0)  // a power of two: two's complement gives the non-negative residue
        return pos & (A - 1);
    int r = pos % A;
    return r < 0 ? r + A : r;
}

__device__ __forceinline__ int readlane_i(int v, int lane) { return __builtin_amdgcn_readlane(v, lane); }
__device__ __forceinline__ float readlane_f(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

}  // namespace ramnet
