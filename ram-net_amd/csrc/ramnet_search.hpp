// Top-K address search routines shared by the decoder and the decode step.
//
// All routines compute the per-digit log-softmax with the same operation
// order (max, exp(x - max), a pairwise tree sum over a power-of-two padded
// digit, log), sum digit scores as ((L_0 + L_1) + L_2) ..., and select under
// the (score desc, content index asc) order, so every path produces the
// same scores bit for bit.
#pragma once

#include "ramnet_device.hpp"
#include "lane_search.hpp"

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
// Loads an address's U x P logits into lg (stride `stride` elements apart)
// and replaces them by their per-digit log-softmax; ex[U*NPD] is scratch.
// Sets *flag when a digit is entirely -inf (inactive address).
template<typename T>
__device__ void block_log_softmax(const T *ptr, int64_t stride, int U, int P, int NPD, float *lg, float *ex,
                                  int *flag) {
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
        const float ls = log_sum(e[0]);
        for (int p = 0; p < P; ++p)
            lg[u * P + p] = (lg[u * P + p] - mx) - ls;
    }
    __syncthreads();
}

// Bitonic sort of independent runs of n (a power of two) entries, all runs
// at once: run r holds sv/si[r*n, (r+1)*n); order (score desc, index asc).
__device__ __forceinline__ void block_sort_runs(float *sv, int *si, int n, int runs) {
    const int tid = threadIdx.x;
    const int nt = blockDim.x;
    const int total = n * runs;
    for (int k = 2; k <= n; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = tid; i < total; i += nt) {
                const int l = i ^ j;
                if (l > i) {
                    const int lo = ((i % n) & k) == 0 ? i : l;
                    const int hi = ((i % n) & k) == 0 ? l : i;
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
}

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
    block_log_softmax(ptr, stride, U, P, NPD, lg, ex, flag);
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
    block_sort_runs(sv, si, NA, 1);
    return *flag != 0;
}

// Candidates of one staircase combination step: prefix entries i < n and
// digit entries j < P with (i + 1)(j + 1) <= K. Any other pair is preceded,
// in both digits, by at least K pairs of the staircase.
__host__ __device__ inline int stair_count(int n, int P, int K) {
    int c = 0;
    for (int i = 0; i < n; ++i) {
        const int m = K / (i + 1);
        c += m < P ? m : P;
    }
    return c;
}

// Staircase search by one workgroup, for slot spaces of any size: the
// per-digit log-softmax as above; every digit sorted; the sorted top list of
// digits 0..d-1 combined with digit d over the staircase candidates and
// sorted again, digit by digit. Scores are summed ((L_0 + L_1) + L_2) ...
// like every other path, so the selection agrees with theirs.
// Scratch: lg[U*P], ex[U*NPD] (then the sorted digit scores), di[U*NPD],
// sv[NC], si[NC], pv[K], pi[K], off[K + 1]; NC = pow2 >= the largest
// candidate count (at most stair_count(K, P, K)) and >= NPD.
// Writes the sorted top entries to sv/si[0..K) and returns the inactive flag.
template<typename T>
__device__ bool block_search_stair(const T *ptr, int64_t stride, int U, int P, int K, int NPD, int NC, float *lg,
                                   float *ex, int *di, float *sv, int *si, float *pv, int *pi, int *off, int *flag) {
    const int tid = threadIdx.x;
    const int nt = blockDim.x;
    block_log_softmax(ptr, stride, U, P, NPD, lg, ex, flag);
    // every digit sorted: (score, digit value) runs of NPD
    for (int i = tid; i < U * NPD; i += nt) {
        const int u = i / NPD, p = i % NPD;
        ex[i] = p < P ? lg[u * P + p] : kNegInfF;
        di[i] = p < P ? p : kNoIdx;
    }
    __syncthreads();
    block_sort_runs(ex, di, NPD, U);
    int n = K < P ? K : P;  // prefix list length
    for (int c = tid; c < NC; c += nt) {
        sv[c] = c < n ? ex[c] : kNegInfF;
        si[c] = c < n ? di[c] : kNoIdx;
    }
    __syncthreads();
    int pw = 1;
    for (int d = 1; d < U; ++d) {
        pw *= P;
        for (int i = tid; i < n; i += nt) {
            pv[i] = sv[i];
            pi[i] = si[i];
        }
        if (tid == 0) {
            off[0] = 0;
            for (int i = 0; i < n; ++i) {
                const int m = K / (i + 1);
                off[i + 1] = off[i] + (m < P ? m : P);
            }
        }
        __syncthreads();
        const int count = off[n];
        const float *dv = ex + d * NPD;
        const int *dd = di + d * NPD;
        for (int c = tid; c < NC; c += nt) {
            if (c < count) {
                int lo = 0, hi = n - 1;  // the prefix entry i with off[i] <= c < off[i + 1]
                while (lo < hi) {
                    const int mid = (lo + hi + 1) >> 1;
                    if (off[mid] <= c)
                        lo = mid;
                    else
                        hi = mid - 1;
                }
                const int j = c - off[lo];
                sv[c] = pv[lo] + dv[j];
                si[c] = pi[lo] + dd[j] * pw;
            } else {
                sv[c] = kNegInfF;
                si[c] = kNoIdx;
            }
        }
        __syncthreads();
        block_sort_runs(sv, si, NC, 1);
        n = count < K ? count : K;
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
    return mx + log_sum(sum);
}

// ---------------------------------------------------------------------------
// Cooperative search by a group of GW lanes (GW = 32: two addresses per
// wave, one per half; GW = 64: one address per wave). One digit value per
// lane; candidates are packed sort keys (see lane_search.hpp) sorted with a
// bitonic network whose lane exchanges are single VALU moves (DPP within a
// row, v_permlane16/32_swap across rows). For each further digit the
// prefix x digit candidates (i, j) with (i+1)(j+1) <= K are formed: any other
// candidate is preceded by at least K candidates that dominate it in both
// digits. Requires P <= GW and the candidate count of K to fit in GW lanes.

// DPP move with bound_ctrl (lanes without a source read 0): every pattern
// used here has a source in the same row for the lanes that keep the
// result, and the form lets the compiler fold the move into its consumer.
template<int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), CTRL, 0xf, 0xf, true));
}

// Value of lane (lane ^ J), J a power of two below 64.
template<int J>
__device__ __forceinline__ uint32_t lane_xor(uint32_t v) {
    const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    if constexpr (J == 1) {
        return dpp_u<0xB1>(v);  // quad_perm [1,0,3,2]
    } else if constexpr (J == 2) {
        return dpp_u<0x4E>(v);  // quad_perm [2,3,0,1]
    } else if constexpr (J == 4) {
        const uint32_t up = dpp_u<0x104>(v);  // row_shl:4 -> lane + 4
        const uint32_t dn = dpp_u<0x114>(v);  // row_shr:4 -> lane - 4
        return (lane & 4) ? dn : up;
    } else if constexpr (J == 8) {
        return dpp_u<0x128>(v);  // row_ror:8
    } else if constexpr (J == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);  // {rows 0,0,2,2}, {rows 1,1,3,3}
        return (lane & 16) ? r[0] : r[1];
    } else {
        static_assert(J == 32, "lane_xor distance");
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);  // {low, low}, {high, high}
        return (lane & 32) ? r[0] : r[1];
    }
}
template<int J>
__device__ __forceinline__ float lane_xor_f(float v) { return __uint_as_float(lane_xor<J>(__float_as_uint(v))); }
template<int J>
__device__ __forceinline__ uint64_t lane_xor(uint64_t v) {
    return (static_cast<uint64_t>(lane_xor<J>(static_cast<uint32_t>(v >> 32))) << 32) |
           lane_xor<J>(static_cast<uint32_t>(v));
}

// The sort networks below select with per-lane bit masks held in vector
// registers (v_bfi_b32) instead of 64-bit lane masks in scalar registers: a
// network has one mask per stage, and as scalar pairs they crowd out the
// kernels' other scalars. The masks depend only on the lane index, so a
// caller's loop computes them once. `opaque` hides from the optimiser that a
// mask is all ones or zero, which would otherwise turn the bitwise select
// back into a scalar-mask select.
__device__ __forceinline__ uint32_t opaque(uint32_t m) {
    asm("" : "+v"(m));
    return m;
}
// All ones where bit J (a power of two) of `idx` is set, else zero.
template<int J>
__device__ __forceinline__ uint32_t bit_mask(int idx) {
    return opaque(0u - ((static_cast<uint32_t>(idx) / J) & 1u));
}
// Bitwise select: bits of a where m is set, of b elsewhere (v_bfi_b32).
__device__ __forceinline__ uint32_t bitsel(uint32_t m, uint32_t a, uint32_t b) { return (a & m) | (b & ~m); }

// lane_xor with the vector-mask selects.
template<int J>
__device__ __forceinline__ uint32_t lane_xor_v(uint32_t v) {
    const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    if constexpr (J == 4) {
        const uint32_t up = dpp_u<0x104>(v);  // row_shl:4 -> lane + 4
        const uint32_t dn = dpp_u<0x114>(v);  // row_shr:4 -> lane - 4
        return bitsel(bit_mask<4>(lane), dn, up);
    } else if constexpr (J == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return bitsel(bit_mask<16>(lane), r[0], r[1]);
    } else if constexpr (J == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return bitsel(bit_mask<32>(lane), r[0], r[1]);
    } else {
        return lane_xor<J>(v);
    }
}
template<int J>
__device__ __forceinline__ float lane_xor_vf(float v) { return __uint_as_float(lane_xor_v<J>(__float_as_uint(v))); }
template<int J>
__device__ __forceinline__ uint64_t lane_xor_v(uint64_t v) {
    return (static_cast<uint64_t>(lane_xor_v<J>(static_cast<uint32_t>(v >> 32))) << 32) |
           lane_xor_v<J>(static_cast<uint32_t>(v));
}

// Value of the group's first lane (lane 0, or 32 for the upper half-wave).
template<int GW>
__device__ __forceinline__ float group_first(float v) {
    const int b = __float_as_int(v);
    if constexpr (GW == 64) {
        return __int_as_float(__builtin_amdgcn_readlane(b, 0));
    } else {
        static_assert(GW == 32, "group_first: GW is 32 or 64");
        const uint32_t lo = __builtin_amdgcn_readlane(b, 0), hi = __builtin_amdgcn_readlane(b, 32);
        return __uint_as_float(bitsel(bit_mask<32>(static_cast<int>(threadIdx.x)), hi, lo));
    }
}
// Butterfly sum over GW lanes, widest exchange first; every lane of the group
// ends with the bitwise same result. With zeros past the digit this is the
// pairwise tree e[p] += e[p + s], s = NP/2 .. 1, of the per-lane decoder, so
// both paths get the same log-sum-exp bit for bit.
template<int GW>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (GW >= 64) v += lane_xor_vf<32>(v);
    if constexpr (GW >= 32) v += lane_xor_vf<16>(v);
    if constexpr (GW >= 16) v += lane_xor_vf<8>(v);
    if constexpr (GW >= 8) v += lane_xor_vf<4>(v);
    if constexpr (GW >= 4) v += lane_xor_vf<2>(v);
    if constexpr (GW >= 2) v += lane_xor_vf<1>(v);
    return v;
}

// Descending bitonic sort of one key per lane over GW lanes. A 32-bit
// compare-exchange is max, min and a bitwise select by the lane's keep-max
// mask; a 64-bit one is one 64-bit compare whose result is flipped on the
// lanes that keep the smaller key, then a bitwise select of both halves.
// The keep-max mask (bits J and K2 of the group lane index agree) is a
// function of the lane index only.
template<int J, int K2>
__device__ __forceinline__ uint32_t keep_max_mask(int li) {
    return opaque(((li & J) == 0) == ((li & K2) == 0) ? 0xffffffffu : 0u);
}
template<int J, int K2>
__device__ __forceinline__ uint32_t keep_min_mask(int li) {
    return opaque(((li & J) == 0) == ((li & K2) == 0) ? 0u : 0xffffffffu);
}
template<int J, int K2>
__device__ __forceinline__ void ce_lane(uint32_t &key, int li) {
    const uint32_t p = lane_xor_v<J>(key);
    const uint32_t hi = key > p ? key : p;
    const uint32_t lo = key > p ? p : key;
    key = bitsel(keep_max_mask<J, K2>(li), hi, lo);
}
template<int J, int K2>
__device__ __forceinline__ void ce_lane(uint64_t &key, int li) {
    const uint64_t p = lane_xor_v<J>(key);
    const uint32_t gt = p > key ? 0xffffffffu : 0u;
    const uint32_t take = gt ^ keep_min_mask<J, K2>(li);  // (p > key) == keep_max
    key = (static_cast<uint64_t>(bitsel(take, static_cast<uint32_t>(p >> 32), static_cast<uint32_t>(key >> 32)))
           << 32) |
          bitsel(take, static_cast<uint32_t>(p), static_cast<uint32_t>(key));
}
template<int GW, int K2, int J, typename Key>
__device__ __forceinline__ void sort_step(Key &key, int li) {
    ce_lane<J, K2>(key, li);
    if constexpr (J > 1)
        sort_step<GW, K2, J / 2>(key, li);
}
template<int GW, int K2 = 2, typename Key>
__device__ __forceinline__ void group_sort_desc(Key &key, int li) {
    sort_step<GW, K2, K2 / 2>(key, li);
    if constexpr (K2 < GW)
        group_sort_desc<GW, K2 * 2>(key, li);
}
// Two independent sorts interleaved stage by stage (each fills the other's
// DPP wait states).
template<int GW, int K2, int J, typename Key>
__device__ __forceinline__ void sort_step2(Key &a, Key &b, int li) {
    ce_lane<J, K2>(a, li);
    ce_lane<J, K2>(b, li);
    if constexpr (J > 1)
        sort_step2<GW, K2, J / 2>(a, b, li);
}
template<int GW, int K2 = 2, typename Key>
__device__ __forceinline__ void group_sort_desc2(Key &a, Key &b, int li) {
    sort_step2<GW, K2, K2 / 2>(a, b, li);
    if constexpr (K2 < GW)
        group_sort_desc2<GW, K2 * 2>(a, b, li);
}

// Number of staircase candidates (i+1)(j+1) <= K.
__host__ __device__ inline int staircase_count(int K) {
    int n = 0;
    for (int i = 1; i <= K; ++i)
        n += K / i;
    return n;
}

// Staircase pairs of the prefix x digit combine for top-K (K = 1..16), in
// (i, j) order: entry li of row K - 1 is (i << 4) | j of the li-th pair with
// (i+1)(j+1) <= K, 0xFF past the last. A lookup replaces the per-lane search
// with its integer divisions.
constexpr int kStairMaxK = 16;
struct StairTable {
    uint8_t e[kStairMaxK][kWave];
};
constexpr StairTable make_stair_table() {
    StairTable t{};
    for (int K = 1; K <= kStairMaxK; ++K) {
        int n = 0;
        for (int i = 0; i < K; ++i)
            for (int j = 0; (i + 1) * (j + 1) <= K; ++j)
                t.e[K - 1][n++] = static_cast<uint8_t>((i << 4) | j);
        for (; n < kWave; ++n)
            t.e[K - 1][n] = 0xFF;
    }
    return t;
}
static_assert(make_stair_table().e[kStairMaxK - 1][49] != 0xFF && make_stair_table().e[kStairMaxK - 1][50] == 0xFF,
              "50 staircase pairs for K = 16");
__constant__ constexpr StairTable kStairTab = make_stair_table();

// Logits of one address as seen by one lane of a GW-lane group: digit u,
// radix li. The first kPreDigits digits are loaded up front in one batch
// (unconditionally, from a clamped radix), later digits on demand.
constexpr int kPreDigits = 4;

// The prefetched digits are kept as raw storage bits and converted when
// read, so a prefetch does not wait for its data before the search.
template<typename T>
struct GroupLogits {
    uint32_t pre[kPreDigits];
    const T *ptr;
    int P;

    __device__ __forceinline__ void load(const T *p, int U, int P_, int li) {
        ptr = p;
        P = P_;
        const int r = li < P_ ? li : P_ - 1;
#pragma unroll
        for (int u = 0; u < kPreDigits; ++u)
            pre[u] = load_bits(p + (u < U ? u : U - 1) * P_ + r);
    }

    __device__ __forceinline__ float get(int u, int li) const {
        if (u < kPreDigits) {
            uint32_t v = pre[0];
#pragma unroll
            for (int k = 1; k < kPreDigits; ++k)
                v = u == k ? pre[k] : v;
            return li < P ? bits_f32<T>(v) : kNegInfF;
        }
        return li < P ? load_f32(ptr + u * P + li) : kNegInfF;
    }
};

// Digit sort key of a logit held as float: for 16-bit inputs the low
// mantissa bits of the float are zero, so the radix index fits in the low 6
// bits of a 32-bit key; fp32 inputs use 64-bit keys.
template<typename T>
using GroupKey = std::conditional_t<sizeof(T) == 2, uint32_t, uint64_t>;

template<typename T>
__device__ __forceinline__ GroupKey<T> group_digit_key(float x, int li) {
    const uint32_t o = ord32(__float_as_uint(x));
    if constexpr (sizeof(T) == 2)
        return (o & ~63u) | static_cast<uint32_t>(63 - li);
    else
        return (static_cast<uint64_t>(o) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(li));
}
template<typename T>
__device__ __forceinline__ void group_digit_unkey(GroupKey<T> k, float &x, int &li) {
    if constexpr (sizeof(T) == 2) {
        const uint32_t hi = k & ~63u;
        x = __uint_as_float(unord32((hi & 0x80000000u) ? hi : (hi | 63u)));
        li = 63 - static_cast<int>(k & 63u);
    } else {
        x = __uint_as_float(unord32(static_cast<uint32_t>(k >> 32)));
        li = static_cast<int>(0xFFFFFFFFu - static_cast<uint32_t>(k));
    }
}

// Decode one address with a group of GW lanes starting at lane g0. On return
// lanes g0 .. g0+K-1 hold the sorted top entries (score, content slot).
// Returns the inactive flag (uniform within the group).
template<typename T, int GW>
__device__ bool group_search(const GroupLogits<T> &lg, int U, int P, int K, int li, float &out_v, int &out_i) {
    using Key = GroupKey<T>;
    constexpr float kLog2e = 1.4426950408889634f;
    // staircase slot (si_, sj_) of this lane (K <= 16 on this path)
    const uint32_t st = kStairTab.e[(K < 1 ? 1 : K > kStairMaxK ? kStairMaxK : K) - 1][li];
    const int si_ = st == 0xFFu ? -1 : static_cast<int>(st >> 4);
    const int sj_ = st == 0xFFu ? -1 : static_cast<int>(st & 15u);
    const int g0 = (static_cast<int>(threadIdx.x) & (kWave - 1)) & ~(GW - 1);
    const int ii = si_ < 0 ? 0 : si_;
    const int jj = sj_ < 0 ? 0 : sj_;
    float cv = kNegInfF;  // prefix score of this lane's rank
    int ci = -1;          // its content slot, -1 = none
    bool inactive = false;
    int stride = 1;
    // prefix x digit over the staircase -> new sorted prefix
    auto combine = [&](float dv, int di) {
        const float pv = __shfl(cv, g0 + ii);
        const int pi = __shfl(ci, g0 + ii);
        const float qv = __shfl(dv, g0 + jj);
        const int qi = __shfl(di, g0 + jj);
        // (bitwise tests and a select: a short-circuit test of the shuffled
        // values would put the key's computation in an exec-mask region,
        // which the scheduler does not cross)
        const bool ok = (si_ >= 0) & (pi >= 0) & (qi >= 0);
        const uint64_t key = (static_cast<uint64_t>(ord32(__float_as_uint(pv + qv))) << 32) |
                             (0xFFFFFFFFu - static_cast<uint32_t>(pi + stride * qi));
        uint64_t ck = ok ? key : uint64_t(0);
        group_sort_desc<GW>(ck, li);
        cv = __uint_as_float(unord32(static_cast<uint32_t>(ck >> 32)));
        ci = ck != 0 ? static_cast<int>(0xFFFFFFFFu - static_cast<uint32_t>(ck)) : -1;
    };
    // digits two at a time: their statistics and sorts are independent
    for (int u = 0; u < U; u += 2) {
        const bool two = u + 1 < U;
        const float xa = lg.get(u, li);  // -inf for li >= P
        const float xb = two ? lg.get(u + 1, li) : kNegInfF;
        // keys of lanes past the digit are 0 (masked, without a branch)
        const uint32_t pm = opaque(li < P ? 0xffffffffu : 0u);
        Key pmk = static_cast<Key>(pm);
        if constexpr (sizeof(Key) == 8)
            pmk |= static_cast<Key>(pm) << 32;
        Key ka = group_digit_key<T>(xa, li) & pmk;
        Key kb = two ? group_digit_key<T>(xb, li) & pmk : Key(0);
        group_sort_desc2<GW>(ka, kb, li);
        // the maxima are the group's first sorted entries
        float xsa, xsb;
        int da, db;
        group_digit_unkey<T>(ka, xsa, da);
        group_digit_unkey<T>(kb, xsb, db);
        const float mxa = group_first<GW>(xsa);
        const float mxb = two ? group_first<GW>(xsb) : kNegInfF;
        inactive = inactive | !(mxa > kNegInfF) | (two & !(mxb > kNegInfF));
        const float ea = li < P ? __builtin_amdgcn_exp2f((xa - mxa) * kLog2e) : 0.f;
        const float eb = li < P ? __builtin_amdgcn_exp2f((xb - mxb) * kLog2e) : 0.f;
        const float lsa = log_sum(group_sum<GW>(ea));
        const float lsb = log_sum(group_sum<GW>(eb));
        const float dva = (xsa - mxa) - lsa;  // this lane's rank of digit u
        const int dia = ka != Key(0) ? da : -1;
        const float dvb = (xsb - mxb) - lsb;  // ... of digit u + 1
        const int dib = kb != Key(0) ? db : -1;
        if (u == 0) {
            cv = dva;
            ci = dia;
        } else {
            combine(dva, dia);
        }
        stride *= P;
        if (two) {
            combine(dvb, dib);
            stride *= P;
        }
    }
    const bool keep = li < K;
    out_v = keep ? cv : kNegInfF;
    out_i = (keep & (ci >= 0)) ? ci : kNoIdx;
    return inactive;
}

}  // namespace ramnet
