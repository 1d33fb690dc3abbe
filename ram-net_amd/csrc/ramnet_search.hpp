// Top-K address search routines shared by the decoder and the decode step.
//
// All routines compute the per-digit log-softmax with the same operation
// order (max, exp(x - max), a pairwise tree sum over a power-of-two padded
// digit, log), sum digit scores as ((L_0 + L_1) + L_2) ..., and select under
// the (score desc, content index asc) order, so every path produces the
// same scores bit for bit.
#pragma once

#include "ramnet_device.hpp"

#include <math.h>

namespace ramnet {

constexpr float kNegInfF = -__builtin_huge_valf();

// Result of decoding one address: K content slots (before CAPE), the
// log-domain scores, and whether the address is inactive.
//
// Exact search by one workgroup: all A scores in LDS, bitonic sort.
// Scratch: lg[U*P], ex[U*NPD], sv[NA], si[NA]; NA = pow2 >= A,
// NPD = pow2 >= P. `ptr` points at digit 0 / radix 0 of the address and
// consecutive logits are `stride` elements apart. Writes the sorted top
// entries to sv/si[0..K) and returns the inactive flag (uniform).
template<typename T>
__device__ bool block_search_exact(const T *ptr, int64_t stride, int U, int P, int A, int NA, int NPD,
                                   float *lg, float *ex, float *sv, int *si, int *flag) {
    const int tid = threadIdx.x;
    const int nt = blockDim.x;
    if (tid == 0)
        *flag = 0;
    for (int i = tid; i < U * P; i += nt)
        lg[i] = load_f32(ptr + static_cast<int64_t>(i) * stride);
    __syncthreads();
    if (tid < U) {
        const int u = tid;
        float mx = kNegInfF;
        bool all_ninf = true;
        for (int p = 0; p < P; ++p) {
            const float x = lg[u * P + p];
            mx = fmaxf(mx, x);
            all_ninf = all_ninf && x == kNegInfF;
        }
        if (all_ninf)
            atomicOr(flag, 1);
        float *e = ex + u * NPD;
        for (int p = 0; p < NPD; ++p)
            e[p] = p < P ? expf(lg[u * P + p] - mx) : 0.f;
        for (int s = NPD / 2; s >= 1; s >>= 1)
            for (int p = 0; p < s; ++p)
                e[p] += e[p + s];
        const float ls = logf(e[0]);
        for (int p = 0; p < P; ++p)
            lg[u * P + p] = (lg[u * P + p] - mx) - ls;
    }
    __syncthreads();
    for (int c = tid; c < NA; c += nt) {
        if (c < A) {
            int rem = c;
            float s = lg[rem % P];
            rem /= P;
            for (int u = 1; u < U; ++u) {
                s = s + lg[u * P + rem % P];
                rem /= P;
            }
            sv[c] = s;
            si[c] = c;
        } else {
            sv[c] = kNegInfF;
            si[c] = kNoIdx;
        }
    }
    __syncthreads();
    for (int k = 2; k <= NA; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = tid; i < NA; i += nt) {
                const int l = i ^ j;
                if (l > i) {
                    const int lo = (i & k) == 0 ? i : l;
                    const int hi = (i & k) == 0 ? l : i;
                    if (before(sv[hi], si[hi], sv[lo], si[lo])) {
                        const float tv = sv[lo];
                        const int ti = si[lo];
                        sv[lo] = sv[hi];
                        si[lo] = si[hi];
                        sv[hi] = tv;
                        si[hi] = ti;
                    }
                }
            }
            __syncthreads();
        }
    }
    return *flag != 0;
}

// log-sum-exp of the K best (sorted) scores, summed from the smallest term to
// the largest; 0 when re-normalisation is off or nothing is finite.
__device__ __forceinline__ float topk_lse_serial(const float *sv, int K) {
    const float mx = sv[0];
    if (!(mx > kNegInfF))
        return 0.f;
    float sum = 0.f;
    for (int k = K - 1; k >= 0; --k)
        sum += expf(sv[k] - mx);
    return mx + logf(sum);
}

// ---------------------------------------------------------------------------
// Cooperative search by a group of GW lanes (GW = 32: two addresses per
// wave, one per half; GW = 64: one address per wave). One digit value per
// lane, bitonic sorts across lanes, and for each further digit the
// prefix x digit candidates (i, j) with (i+1)(j+1) <= K: any other candidate
// is preceded by at least K candidates that dominate it in both digits.
// Requires P <= GW and the candidate count of K to fit in GW lanes.

template<int GW>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
    for (int s = GW / 2; s >= 1; s >>= 1)
        v = fmaxf(v, __shfl_xor(v, s));
    return v;
}

// Sum with the same pairwise tree as e[p] += e[p + s], s = GW/2 .. 1.
template<int GW>
__device__ __forceinline__ float group_tree_sum(float v) {
#pragma unroll
    for (int s = GW / 2; s >= 1; s >>= 1)
        v += __shfl_xor(v, s);
    return v;
}

template<int GW>
__device__ __forceinline__ void group_sort(float &v, int &id, int li) {
#pragma unroll
    for (int k = 2; k <= GW; k <<= 1) {
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
            const float pv = __shfl_xor(v, j);
            const int pi = __shfl_xor(id, j);
            const bool up = (li & k) == 0;
            const bool lower = (li & j) == 0;
            const bool take = (lower == up) ? before(pv, pi, v, id) : before(v, id, pv, pi);
            v = take ? pv : v;
            id = take ? pi : id;
        }
    }
}

// Number of staircase candidates (i+1)(j+1) <= K.
__host__ __device__ inline int staircase_count(int K) {
    int n = 0;
    for (int i = 1; i <= K; ++i)
        n += K / i;
    return n;
}

// Logits of one address as seen by one lane of a GW-lane group: digit u,
// radix li. The first kPreDigits digits are loaded up front in one batch
// (unconditionally, from a clamped radix), later digits on demand.
constexpr int kPreDigits = 4;

template<typename T>
struct GroupLogits {
    float pre[kPreDigits];
    const T *ptr;
    int P;

    __device__ __forceinline__ void load(const T *p, int U, int P_, int li) {
        ptr = p;
        P = P_;
        const int r = li < P_ ? li : P_ - 1;
#pragma unroll
        for (int u = 0; u < kPreDigits; ++u)
            pre[u] = load_f32(p + (u < U ? u : U - 1) * P_ + r);
    }

    __device__ __forceinline__ float get(int u, int li) const {
        if (u < kPreDigits) {
            float v = pre[0];
#pragma unroll
            for (int k = 1; k < kPreDigits; ++k)
                v = u == k ? pre[k] : v;
            return li < P ? v : kNegInfF;
        }
        return li < P ? load_f32(ptr + u * P + li) : kNegInfF;
    }
};

// Decode one address with a group of GW lanes starting at lane g0. On return
// lanes g0 .. g0+K-1 hold the sorted top entries (score, content slot).
// Returns the inactive flag (uniform within the group).
template<typename T, int GW>
__device__ bool group_search(const GroupLogits<T> &lg, int U, int P, int K, int li, float &out_v, int &out_i) {
    float cv = kNegInfF;
    int ci = kNoIdx;
    bool inactive = false;
    int stride = 1;
    // staircase slot of this lane
    int si_ = -1, sj_ = -1;
    {
        int q = li;
        for (int i = 0; i < K; ++i) {
            const int cnt = K / (i + 1);
            if (q < cnt) {
                si_ = i;
                sj_ = q;
                break;
            }
            q -= cnt;
        }
    }
    const int g0 = (threadIdx.x & (kWave - 1)) & ~(GW - 1);
    for (int u = 0; u < U; ++u) {
        const float x = lg.get(u, li);
        const bool fin = li < P && x != kNegInfF;
        // any finite logit in this digit, within the group
        float any = fin ? 1.f : 0.f;
        any = group_max<GW>(any);
        inactive = inactive || any == 0.f;
        const float mx = group_max<GW>(x);
        const float e = li < P ? expf(x - mx) : 0.f;
        const float ssum = group_tree_sum<GW>(e);
        const float ls = logf(ssum);
        float dv = li < P ? (x - mx) - ls : kNegInfF;
        int di = li < P ? li : kNoIdx;
        group_sort<GW>(dv, di, li);
        if (u == 0) {
            const bool keep = li < K;
            cv = keep ? dv : kNegInfF;
            ci = keep ? di : kNoIdx;
        } else {
            const int ii = si_ < 0 ? 0 : si_;
            const int jj = sj_ < 0 ? 0 : sj_;
            const float pv = __shfl(cv, g0 + ii);
            const int pi = __shfl(ci, g0 + ii);
            const float qv = __shfl(dv, g0 + jj);
            const int qi = __shfl(di, g0 + jj);
            const bool ok = si_ >= 0 && pi != kNoIdx && qi != kNoIdx;
            float nv = ok ? pv + qv : kNegInfF;
            int ni = ok ? pi + stride * qi : kNoIdx;
            group_sort<GW>(nv, ni, li);
            const bool keep = li < K;
            cv = keep ? nv : kNegInfF;
            ci = keep ? ni : kNoIdx;
        }
        stride *= P;
    }
    out_v = cv;
    out_i = ci;
    return inactive;
}

}  // namespace ramnet
