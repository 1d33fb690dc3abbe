// Per-lane Product-Softmax top-K search on packed sort keys.
//
// One lane decodes one address. Candidates are ordered by (score desc,
// content index asc); both parts are packed into one unsigned key so that a
// compare-exchange is a max/min pair:
//   digit keys      16-bit inputs: ord16(logit) << 16 | (0xFFFF - digit)
//                   fp32 inputs:   ord32(logit) << 31 | (0x7FFFFFFF - digit)
//   prefix keys     ord32(score) << 31 | (0x7FFFFFFF - content index)
// where ord maps a float's bits to an unsigned integer with the same order
// (-0 is folded onto +0 first so that equal values compare equal). Within a
// digit, log_softmax is a monotone shift of the logits, so ordering by logit
// orders by log-probability. Key 0 marks "no candidate".
//
// The 64-bit keys stay below 2^63, so read as IEEE doubles they are
// non-negative and ordered as the integers are; a 64-bit compare-exchange
// is then one v_max_f64 and one v_min_f64 instead of a 64-bit compare and
// four selects. The exponent field of a key is bits 30..20 of its ord32
// value: it is all ones or all zeros only for NaN inputs (positive NaNs
// from 0x7FE00000 up, negative ones from 0xFFE00000 up), whose keys would
// read as NaN or subnormal doubles; -inf, finite values and +inf give
// normal doubles, and key 0 reads as +0.
//
// Search (U digits, top-KM lists): the sorted top-KM of each digit is
// combined with the sorted top-KM prefix list over the staircase
// (i + 1)(j + 1) <= KM of prefix i x digit j -- every element outside it has
// at least KM elements before it in both orders -- and the top-KM of those
// candidates becomes the next prefix.
#pragma once

#include "ramnet_device.hpp"

#include <stdint.h>
#include <type_traits>
#include <utility>

namespace ramnet {

__device__ __forceinline__ uint32_t ord16(uint32_t h) {
    h = h == 0x8000u ? 0u : h;
    return (h & 0x8000u) ? (~h & 0xFFFFu) : (h | 0x8000u);
}
__device__ __forceinline__ uint32_t unord16(uint32_t o) { return (o & 0x8000u) ? (o & 0x7FFFu) : (~o & 0xFFFFu); }
__device__ __forceinline__ uint32_t ord32(uint32_t u) {
    u = u == 0x80000000u ? 0u : u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ uint32_t unord32(uint32_t o) { return (o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o; }

// Descending compare-exchange: a gets the larger key.
__device__ __forceinline__ void ce_desc(uint32_t &a, uint32_t &b) {
    const uint32_t hi = a > b ? a : b;
    const uint32_t lo = a > b ? b : a;
    a = hi;
    b = lo;
}
__device__ __forceinline__ uint32_t key_max(uint32_t a, uint32_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint64_t key_max(uint64_t a, uint64_t b) {
    uint64_t r;
    asm("v_max_f64 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ __forceinline__ void ce_desc(uint64_t &a, uint64_t &b) {
    uint64_t hi, lo;
    asm("v_max_f64 %0, %1, %2" : "=v"(hi) : "v"(a), "v"(b));
    asm("v_min_f64 %0, %1, %2" : "=v"(lo) : "v"(a), "v"(b));
    a = hi;
    b = lo;
}

// Batcher's odd-even merge sort network on N = 2^n keys, generated at
// compile time: comparator c orders positions (a[c], b[c]), a < b. It takes
// 19 compare-exchanges for 8 keys and 63 for 16, where the bitonic network
// takes 24 and 80.
template<int N>
struct SortNet {
    int a[N * N > 0 ? N * N : 1] = {};
    int b[N * N > 0 ? N * N : 1] = {};
    int n = 0;
    constexpr SortNet() { sort_range(0, N - 1); }
    constexpr void merge(int lo, int hi, int r) {
        const int step = r * 2;
        if (step < hi - lo) {
            merge(lo, hi, step);
            merge(lo + r, hi, step);
            for (int i = lo + r; i < hi - r; i += step) {
                a[n] = i;
                b[n] = i + r;
                ++n;
            }
        } else {
            a[n] = lo;
            b[n] = lo + r;
            ++n;
        }
    }
    constexpr void sort_range(int lo, int hi) {
        if (hi - lo >= 1) {
            const int mid = lo + (hi - lo) / 2;
            sort_range(lo, mid);
            sort_range(mid + 1, hi);
            merge(lo, hi, 1);
        }
    }
};
template<int N, int OFF, typename K, int M, int... C>
__device__ __forceinline__ void sort_net_apply(K (&k)[M], std::integer_sequence<int, C...>) {
    constexpr SortNet<N> net{};
    (ce_desc(k[OFF + net.a[C]], k[OFF + net.b[C]]), ...);
}

// Descending sort of keys [OFF, OFF + N); N a power of two.
template<int N, int OFF, typename K, int M>
__device__ __forceinline__ void sort_desc(K (&k)[M]) {
    if constexpr (N > 1)
        sort_net_apply<N, OFF>(k, std::make_integer_sequence<int, SortNet<N>().n>{});
}

// a <- sorted top-KM of sorted a and the sorted group [OFF, OFF + KM) of b.
template<int KM, int OFF, typename K, int M>
__device__ __forceinline__ void merge_top(K (&a)[KM], const K (&b)[M]) {
#pragma unroll
    for (int i = 0; i < KM; ++i) {
        a[i] = key_max(a[i], b[OFF + KM - 1 - i]);
    }
#pragma unroll
    for (int j = KM >> 1; j > 0; j >>= 1) {
#pragma unroll
        for (int i = 0; i < KM; ++i) {
            const int l = i ^ j;
            if (l > i)
                ce_desc(a[i], a[l]);
        }
    }
}

template<int KM, int G, int NG, typename K, int N>
__device__ __forceinline__ void sort_groups_desc(K (&k)[N]) {
    if constexpr (G < NG) {
        sort_desc<KM, G * KM>(k);
        sort_groups_desc<KM, G + 1, NG>(k);
    }
}
template<int KM, int G, int NG, typename K, int N>
__device__ __forceinline__ void merge_groups(K (&top)[KM], const K (&k)[N]) {
    if constexpr (G < NG) {
        merge_top<KM, G * KM>(top, k);
        merge_groups<KM, G + 1, NG>(top, k);
    }
}

// Sorted top-KM of N keys (N a multiple of KM, or N <= KM).
template<int KM, typename K, int N>
__device__ __forceinline__ void top_keys(K (&k)[N], K (&top)[KM]) {
    if constexpr (N <= KM) {
        sort_desc<N, 0>(k);
#pragma unroll
        for (int i = 0; i < KM; ++i)
            top[i] = i < N ? k[i < N ? i : 0] : K(0);
    } else {
        static_assert(N % KM == 0, "key count must be a multiple of KM");
        sort_groups_desc<KM, 0, N / KM>(k);
#pragma unroll
        for (int i = 0; i < KM; ++i)
            top[i] = k[i];
        merge_groups<KM, 1, N / KM>(top, k);
    }
}

// Staircase (i + 1)(j + 1) <= KM: candidate count and the (i, j) of entry n.
template<int KM>
constexpr int stair_count() {
    int n = 0;
    for (int i = 0; i < KM; ++i)
        n += KM / (i + 1);
    return n;
}
template<int KM>
constexpr int stair_i(int n) {
    for (int i = 0; i < KM; ++i) {
        if (n < KM / (i + 1))
            return i;
        n -= KM / (i + 1);
    }
    return 0;
}
template<int KM>
constexpr int stair_j(int n) {
    for (int i = 0; i < KM; ++i) {
        if (n < KM / (i + 1))
            return n;
        n -= KM / (i + 1);
    }
    return 0;
}

template<typename Scalar>
using DigitKey = std::conditional_t<sizeof(Scalar) == 2, uint32_t, uint64_t>;

template<typename Scalar>
__device__ __forceinline__ uint32_t raw_bits(const Scalar *p) {
    if constexpr (sizeof(Scalar) == 2)
        return *reinterpret_cast<const uint16_t *>(p);
    else
        return *reinterpret_cast<const uint32_t *>(p);
}
template<typename Scalar>
__device__ __forceinline__ float bits_value(uint32_t b) {
    if constexpr (sizeof(Scalar) == 4)
        return __uint_as_float(b);
    else if constexpr (__is_same(Scalar, bf16_t))
        return __uint_as_float(b << 16);
    else
        return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(b)));
}
template<typename Scalar>
__device__ __forceinline__ DigitKey<Scalar> digit_key(uint32_t bits, int p) {
    if constexpr (sizeof(Scalar) == 2)
        return (ord16(bits) << 16) | (0xFFFFu - static_cast<uint32_t>(p));
    else
        return (static_cast<uint64_t>(ord32(bits)) << 31) | (0x7FFFFFFFu - static_cast<uint32_t>(p));
}
template<typename Scalar>
__device__ __forceinline__ void digit_unkey(DigitKey<Scalar> k, float &x, int &p) {
    if constexpr (sizeof(Scalar) == 2) {
        x = bits_value<Scalar>(unord16(k >> 16));
        p = static_cast<int>(0xFFFFu - (k & 0xFFFFu));
    } else {
        x = __uint_as_float(unord32(static_cast<uint32_t>(k >> 31)));
        p = static_cast<int>(0x7FFFFFFFu - (static_cast<uint32_t>(k) & 0x7FFFFFFFu));
    }
}

__device__ __forceinline__ uint64_t prefix_key(float s, int c) {
    return (static_cast<uint64_t>(ord32(__float_as_uint(s))) << 31) | (0x7FFFFFFFu - static_cast<uint32_t>(c));
}

// One digit: sorted top-KM log-probabilities (lv) and digit values (dv),
// valid flags; returns false when every logit of the digit is -inf.
// Logit loaders: load(u, p) gives the raw bits of logit p of digit u.
// GlobalLogits walks a per-lane pointer (any tensor size); BufferLogits
// reads through one buffer resource based at the wave's first lane with
// 32-bit per-lane offsets, which keeps the per-load addresses out of scalar
// registers (the host picks it when every offset fits in 31 bits).
template<typename Scalar>
struct GlobalLogits {
    const Scalar *base;  // logit 0 of digit 0 for this lane
    int stride;          // elements between consecutive logits (T); U * P * T fits an int
    int P;
    __device__ __forceinline__ uint32_t operator()(int u, int p) const {
        return raw_bits<Scalar>(base + (u * P + p) * stride);
    }
};
template<typename Scalar>
struct BufferLogits {
    __amdgpu_buffer_rsrc_t rsrc;
    int lane_off;  // bytes from the resource base to this lane's logit 0 of digit 0
    int step;      // bytes between consecutive logits (T * sizeof(Scalar))
    int P;
    __device__ __forceinline__ uint32_t operator()(int u, int p) const {
        const int off = lane_off + (u * P + p) * step;
        if constexpr (sizeof(Scalar) == 2)
            return __builtin_amdgcn_raw_buffer_load_b16(rsrc, off, 0, 0);
        else
            return __builtin_amdgcn_raw_buffer_load_b32(rsrc, off, 0, 0);
    }
};

// Validity flags are kept as 0 / all-ones 32-bit masks in vector registers
// (bool arrays would live as 64-bit lane masks in scalar registers and spill).
// FULL: P == NP, so no logit is padding (the padding selects compile away).
template<typename Scalar, int NP, int KM, bool FULL, typename Load>
__device__ __forceinline__ bool digit_top(const Load &load, int u, int P_, float (&lv)[KM], int (&dv)[KM],
                                          uint32_t (&ok)[KM]) {
    using K = DigitKey<Scalar>;
    const int P = FULL ? NP : P_;
    K keys[NP];
    float x[NP];
    // All loads first, unconditional: the padding repeats the digit's last
    // logit. A guarded load or a branch on P would wait for each load's data
    // before issuing the next.
    uint32_t bits[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p)
        bits[p] = load(u, p < P ? p : P - 1);
    // padding keys are masked to 0 arithmetically (no branch)
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        x[p] = bits_value<Scalar>(bits[p]);
        const K live = p < P ? ~K(0) : K(0);
        keys[p] = digit_key<Scalar>(bits[p], p) & live;
    }
    K top[KM];
    top_keys<KM>(keys, top);
    float mx;
    int p0;
    digit_unkey<Scalar>(top[0], mx, p0);
    const bool live = mx > -__builtin_huge_valf();
    // log-sum-exp around the maximum; exp2 of a prescaled argument, summed
    // with a fixed pairwise tree (padding contributes exact zeros)
    constexpr float kLog2e = 1.4426950408889634f;
    float e[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p)
            e[p] = __builtin_amdgcn_exp2f((x[p] - mx) * kLog2e) * (p < P ? 1.f : 0.f);
#pragma unroll
    for (int s = NP / 2; s >= 1; s >>= 1)
#pragma unroll
        for (int p = 0; p < s; ++p)
            e[p] += e[p + s];
    const float ls = log_sum(e[0]);
#pragma unroll
    for (int k = 0; k < KM; ++k) {
        float xv;
        int p;
        digit_unkey<Scalar>(top[k], xv, p);
        ok[k] = top[k] != K(0) ? ~0u : 0u;
        lv[k] = (xv - mx) - ls;
        dv[k] = p;
    }
    return live;
}

// The staircase row merge. Row i of the staircase (prefix i with digit
// entries j < KM / (i + 1)) is already sorted: the prefix score is fixed and
// the digit's log-probabilities descend with j (equal sums from distinct
// log-probabilities, where fp32 rounding absorbs their difference, can
// break the content-index order of a tie, which the parity bar allows). So
// the top KM of the staircase is a merge of sorted lists, not a sort: rows
// [LO, HI) are merged recursively, each list padded with empty keys to a
// power of two, keeping the top KM. KM = 16: about half the compare-
// exchanges of sorting the 50 candidates in groups.
template<int KM>
constexpr int stair_row_len(int i) { return KM / (i + 1); }
constexpr int pow2_up(int n) { return n <= 1 ? 1 : 2 * pow2_up((n + 1) / 2); }
template<int KM, int LO, int HI>
constexpr int stair_list_len() {
    if constexpr (HI - LO == 1) {
        return pow2_up(stair_row_len<KM>(LO));
    } else {
        constexpr int MID = (LO + HI) / 2;
        constexpr int A = stair_list_len<KM, LO, MID>(), B = stair_list_len<KM, MID, HI>();
        constexpr int L = 2 * (A > B ? A : B);
        return L < KM ? L : KM;
    }
}
template<int N>
struct KeyList {
    uint64_t k[N];
};
// Descending bitonic merge of a bitonic list of N (a power of two).
template<int N>
__device__ __forceinline__ void bitonic_merge_desc(uint64_t (&k)[N]) {
#pragma unroll
    for (int j = N >> 1; j > 0; j >>= 1) {
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const int l = i ^ j;
            if (l > i)
                ce_desc(k[i], k[l]);
        }
    }
}
// Top min(KM, 2 max(NA, NB)) of two sorted lists, sorted. Entries of the
// shorter list past its length are empty and take no compare.
template<int KM, int NA, int NB>
__device__ __forceinline__ auto merge_lists(const KeyList<NA> &a, const KeyList<NB> &b) {
    if constexpr (NA < NB) {
        return merge_lists<KM, NB, NA>(b, a);
    } else {
        constexpr int L = 2 * NA <= KM ? 2 * NA : KM;
        KeyList<L> out;
        if constexpr (L == 2 * NA) {
            // a then reversed b: bitonic; its first stage pairs a[i] with b[NA - 1 - i]
#pragma unroll
            for (int i = 0; i < NA; ++i) {
                const int jb = NA - 1 - i;
                if (jb < NB) {
                    uint64_t x = a.k[i], y = b.k[jb];
                    ce_desc(x, y);
                    out.k[i] = x;
                    out.k[NA + i] = y;
                } else {
                    out.k[i] = a.k[i];
                    out.k[NA + i] = 0;
                }
            }
            KeyList<NA> lo, hi;
#pragma unroll
            for (int i = 0; i < NA; ++i) {
                hi.k[i] = out.k[i];
                lo.k[i] = out.k[NA + i];
            }
            bitonic_merge_desc<NA>(hi.k);
            bitonic_merge_desc<NA>(lo.k);
#pragma unroll
            for (int i = 0; i < NA; ++i) {
                out.k[i] = hi.k[i];
                out.k[NA + i] = lo.k[i];
            }
        } else {
            // NA == KM: the larger of a[i] and b[KM - 1 - i] are the top KM, bitonic
#pragma unroll
            for (int i = 0; i < KM; ++i) {
                const int jb = KM - 1 - i;
                out.k[i] = jb < NB ? key_max(a.k[i], b.k[jb]) : a.k[i];
            }
            bitonic_merge_desc<KM>(out.k);
        }
        return out;
    }
}
// Candidate keys of staircase rows [LO, HI), merged.
template<int KM, int LO, int HI, typename RowKey>
__device__ __forceinline__ KeyList<stair_list_len<KM, LO, HI>()> stair_rows(const RowKey &key) {
    if constexpr (HI - LO == 1) {
        constexpr int N = stair_list_len<KM, LO, HI>();
        KeyList<N> r;
#pragma unroll
        for (int j = 0; j < N; ++j)
            r.k[j] = j < stair_row_len<KM>(LO) ? key(LO, j) : 0;
        return r;
    } else {
        constexpr int MID = (LO + HI) / 2;
        return merge_lists<KM>(stair_rows<KM, LO, MID>(key), stair_rows<KM, MID, HI>(key));
    }
}

// Prefix (score sv, content cv) x digit (lv, dv) over the staircase ->
// sorted top-KM new prefix. `stride` is P^u of the digit.
template<int KM>
__device__ __forceinline__ void combine_prefix(float (&sv)[KM], int (&cv)[KM], uint32_t (&ok)[KM],
                                               const float (&lv)[KM], const int (&dv)[KM], const uint32_t (&dok)[KM],
                                               int stride) {
    auto key = [&](int i, int j) -> uint64_t {
        const uint64_t m = ok[i] & dok[j];
        return prefix_key(sv[i] + lv[j], cv[i] + stride * dv[j]) & ((m << 32) | m);
    };
    const auto merged = stair_rows<KM, 0, KM>(key);
    static_assert(stair_list_len<KM, 0, KM>() == KM, "the staircase merge keeps KM keys");
    const uint64_t(&top)[KM] = merged.k;
#pragma unroll
    for (int k = 0; k < KM; ++k) {
        ok[k] = top[k] != 0 ? ~0u : 0u;
        sv[k] = __uint_as_float(unord32(static_cast<uint32_t>(top[k] >> 31)));
        cv[k] = static_cast<int>(0x7FFFFFFFu - (static_cast<uint32_t>(top[k]) & 0x7FFFFFFFu));
    }
}

// Full search of one address: sorted top-KM (score, content index, valid)
// over all U digits. Returns false if any digit is all -inf (inactive).
template<typename Scalar, int NP, int KM, bool FULL, typename Load>
__device__ __forceinline__ bool lane_search(const Load &load, int U, int P_, float (&sv)[KM], int (&cv)[KM],
                                            uint32_t (&ok)[KM]) {
    const int P = FULL ? NP : P_;
    bool live = digit_top<Scalar, NP, KM, FULL>(load, 0, P, sv, cv, ok);
    int stride = P;
    for (int u = 1; u < U; ++u) {
        float lv[KM];
        int dv[KM];
        uint32_t dok[KM];
        live = digit_top<Scalar, NP, KM, FULL>(load, u, P, lv, dv, dok) && live;
        combine_prefix<KM>(sv, cv, ok, lv, dv, dok, stride);
        stride *= P;
    }
    return live;
}

}  // namespace ramnet
