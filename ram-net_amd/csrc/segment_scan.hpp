// Time-ordered segment scan kernel (gated sparse update + top-K read).
//
// A workgroup of NW state waves owns one (b, h, channel slice) unit and walks
// the whole sequence with the unit's A x CS slot slice resident in LDS; each
// state wave owns CSW channels of the slice. The slot masses are kept by one
// extra mass wave, or, in the precomputed-gain form, replaced by the gains a
// mass pre-pass wrote into the records. The lane layout is fixed at compile
// time:
//   EPP events per pass, LPE = 64 / EPP lanes per event,
//   VEC channels per lane, CSW = LPE * VEC channels per wave,
//   NP passes cover up to NP * EPP write and NP * EPP read events per token.
// Per-event records ({slot, w, alpha} for writes, {slot, r} for reads; see
// ramnet_kernels.hpp) and x are staged per 16-token chunk through LDS.
// Events that must not act point at two dummy LDS rows in front of the
// state (slot -2 for writes, -1 for reads), so the token body is
// branch-free. LDS executes a wave's accesses in program order, which
// carries the read-modify-write dependency from one token to the next.
#pragma once

#include "ramnet_device.hpp"
#include "ramnet_kernels.hpp"
#include "ramnet_search.hpp"

#include <type_traits>

namespace ramnet {

constexpr int kChunk = kScanChunk;

struct ScanGeom {
    int n_units;  // B * H * n_slices
    int n_slices; // ceil(C / CS)
    int n_chunks; // ceil(T / kChunk)
    int t_pad;    // T rounded up to kScanPad (record row length)
    // Slot range of this launch (precomputed-gain form): slots [r0, r0 +
    // n_local) are resident and events on other slots act on the dummy rows.
    // The ranges run in order; each adds its read sums to the fp32 sums of
    // the ranges before it (job.yacc), and the last (last != 0) stores y. One
    // range (r0 = 0, n_local = A) unless A is too wide for LDS.
    int r0;
    int n_local;
    int last;
};

// 1/d refined by one Newton step; gain = w / (m + eps) to ~1 ulp.
__device__ __forceinline__ float scan_gain(float w, float d) {
    float r = __builtin_amdgcn_rcpf(d);
    r = fmaf(r, fmaf(-d, r, 1.f), r);
    return w * r;
}

template<int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum over the EPP consecutive lanes of an event group; every lane of the
// group receives the same value. DPP within a 16-lane row, shuffles across.
template<int EPP>
__device__ __forceinline__ float event_sum(float v) {
    if constexpr (EPP >= 2) v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    if constexpr (EPP >= 4) v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    if constexpr (EPP >= 8) v += dpp_f<0x141>(v);  // row_half_mirror
    if constexpr (EPP >= 16) v += dpp_f<0x140>(v); // row_mirror
    if constexpr (EPP >= 32) v += __shfl_xor(v, 16);
    if constexpr (EPP >= 64) v += __shfl_xor(v, 32);
    return v;
}

// a + (lane CTRL of a), for DPP patterns whose source lane always exists or
// whose missing-source lanes are not used (bound_ctrl: reads 0, no old value)
template<int CTRL>
__device__ __forceinline__ float add_dpp(float a) {
    return a + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(a), CTRL, 0xf, 0xf, true));
}

// bits of a where m is set, of b elsewhere, as one v_bfi_b32 (the bitwise
// form alone is split into two instructions once ~m is hoisted)
__device__ __forceinline__ uint32_t bfi(uint32_t m, uint32_t a, uint32_t b) {
    uint32_t r;
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(m), "v"(a), "v"(b));
    return r;
}

// One exchange of a reduce-scatter over lane bit LB, partner = lane ^ (1 <<
// LB): lanes with the bit clear receive a + a(partner), lanes with it set
// b + b(partner). Across rows v_permlane16/32_swap trades a's upper half for
// b's lower half in one instruction, so the two outputs add to the pair sum
// with no select; within a row, two DPP adds and a bit select (hi = all ones
// in the lanes with the bit set).
template<int LB>
__device__ __forceinline__ float scatter_pair(float a, float b, uint32_t hi) {
    if constexpr (LB == 5) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
        return __uint_as_float(r[0]) + __uint_as_float(r[1]);
    } else if constexpr (LB == 4) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
        return __uint_as_float(r[0]) + __uint_as_float(r[1]);
    } else {
        float pa, pb;
        if constexpr (LB == 3) {
            pa = add_dpp<0x128>(a);  // row_ror:8 (lane ^ 8 within a row)
            pb = add_dpp<0x128>(b);
        } else if constexpr (LB == 2) {
            pa = add_dpp<0x104>(a);  // row_shl:4 -> lane + 4 (used where bit 2 is clear)
            pb = add_dpp<0x114>(b);  // row_shr:4 -> lane - 4 (used where bit 2 is set)
        } else if constexpr (LB == 1) {
            pa = add_dpp<0x4E>(a);  // quad_perm [2,3,0,1]
            pb = add_dpp<0x4E>(b);
        } else {
            static_assert(LB == 0, "scatter_pair: lane bit 0..5");
            pa = add_dpp<0xB1>(a);  // quad_perm [1,0,3,2]
            pb = add_dpp<0xB1>(b);
        }
        return __uint_as_float(bfi(hi, __float_as_uint(pb), __float_as_uint(pa)));
    }
}

// Reduce-scatter of N = 2^(I+1) tokens' partial sums over event lane bits
// SH .. SH + I (highest first): afterwards part[0] of a lane holds, for the
// token whose index equals the lane's event bits, the total over the event
// lanes. N - 1 exchanges serve N tokens, where a per-token all-reduce costs
// log2(N) exchanges and a select per token.
template<int I, int SH, int N>
__device__ __forceinline__ void event_scatter(float (&part)[N], const uint32_t (&hi)[6]) {
    if constexpr (I >= 0) {
        constexpr int H = 1 << I;
#pragma unroll
        for (int m = 0; m < H; ++m)
            part[m] = scatter_pair<SH + I>(part[m], part[m + H], hi[SH + I]);
        event_scatter<I - 1, SH, N>(part, hi);
    }
}

// Overlap flag read when a head has no write events (a global, not a
// constant: a constant-space pointer would make the flag load a flat one).
static __device__ int kNoFlag = 0;

// 16-byte load and store through a vector type: int4 is a struct, and its
// copies between memory and a register array become memcpys that can keep
// the array in scratch memory.
typedef int i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int4 ld16(const void *p) {
    const i32x4 v = *reinterpret_cast<const i32x4 *>(p);
    return make_int4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st16(void *p, const int4 &v) {
    *reinterpret_cast<i32x4 *>(p) = i32x4{v.x, v.y, v.z, v.w};
}

// LDS byte address of a pointer into the workgroup's LDS, and back: a row
// offset computed once per chunk then addresses its LDS access directly.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char *)p));
}
__device__ __forceinline__ float *lds_at(uint32_t a) {
    return (float *)(__attribute__((address_space(3))) float *)(uintptr_t)a;
}
// a * b + c for a, b in the signed 24-bit range (slots include the dummy
// rows -2 and -1), as one v_mad_i32_i24 (left to itself the compiler keeps
// the product and adds c at every use)
__device__ __forceinline__ int mad24(int a, int b, int c) {
    int r;
    asm("v_mad_i32_i24 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

// Sum over the lanes whose indices differ from a lane's own only in bits
// J .. 32 (J a power of two): exact xor exchanges by DPP within a row
// (quad_perm, row_shl/shr:4, row_ror:8), then v_permlane16/32_swap, whose two
// outputs hold the two halves being combined.
template<int J>
__device__ __forceinline__ float strided_sum(float v) {
    if constexpr (J >= kWave) {
        return v;
    } else if constexpr (J < 8) {
        return strided_sum<J * 2>(v + lane_xor_f<J>(v));
    } else if constexpr (J == 8) {
        return strided_sum<16>(v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xf, 0xf, true)));
    } else if constexpr (J == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        return strided_sum<32>(__uint_as_float(r[0]) + __uint_as_float(r[1]));
    } else {
        static_assert(J == 32, "strided_sum: J in {8, 16, 32}");
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        return __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
}

// VEC consecutive floats with the widest LDS access their alignment allows.
template<int VEC>
struct FVec {
    float v[VEC];
};

template<int VEC>
__device__ __forceinline__ FVec<VEC> lds_load(const float *p) {
    FVec<VEC> r;
    if constexpr (VEC == 4) {
        const float4 t = *reinterpret_cast<const float4 *>(p);
        r.v[0] = t.x; r.v[1] = t.y; r.v[2] = t.z; r.v[3] = t.w;
    } else if constexpr (VEC == 2) {
        const float2 t = *reinterpret_cast<const float2 *>(p);
        r.v[0] = t.x; r.v[1] = t.y;
    } else {
        r.v[0] = *p;
    }
    return r;
}

template<int VEC>
__device__ __forceinline__ void lds_store(float *p, const FVec<VEC> &r) {
    if constexpr (VEC == 4)
        *reinterpret_cast<float4 *>(p) = make_float4(r.v[0], r.v[1], r.v[2], r.v[3]);
    else if constexpr (VEC == 2)
        *reinterpret_cast<float2 *>(p) = make_float2(r.v[0], r.v[1]);
    else
        *p = r.v[0];
}

// float -> activation element, scalar and VEC-wide (the wide forms need
// VEC-element alignment).
__device__ __forceinline__ void store_out(float *p, float v) { *p = v; }
__device__ __forceinline__ void store_out(_Float16 *p, float v) { *p = static_cast<_Float16>(v); }
__device__ __forceinline__ void store_out(bf16_t *p, float v) {
    p->bits = __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));  // hardware round-to-nearest-even
}

// VEC activation elements kept as their raw bits until use, so a prefetch of
// the next chunk needs no conversion (and no wait) when it is issued.
template<typename Scalar, int VEC>
struct XBits {
    static constexpr int kWords = (VEC * static_cast<int>(sizeof(Scalar)) + 3) / 4;
    uint32_t w[kWords];
};

template<typename Scalar>
__device__ __forceinline__ float half_bits_to_f(uint32_t h) {
    if constexpr (sizeof(Scalar) == 4)
        return __uint_as_float(h);
    else if constexpr (__is_same(Scalar, bf16_t))
        return __uint_as_float(h << 16);
    else
        return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

// Element-wise bit load; XV: the VEC elements are one aligned vector.
template<typename Scalar, int VEC, bool XV>
__device__ __forceinline__ XBits<Scalar, VEC> load_x_bits(const Scalar *row, int c, int C) {
    XBits<Scalar, VEC> r;
    if constexpr (sizeof(Scalar) == 4 && XV && VEC == 4) {
        const uint4 t = *reinterpret_cast<const uint4 *>(row + c);
        r.w[0] = t.x; r.w[1] = t.y; r.w[2] = t.z; r.w[3] = t.w;
    } else if constexpr (sizeof(Scalar) == 4 && XV && VEC == 2) {
        const uint2 t = *reinterpret_cast<const uint2 *>(row + c);
        r.w[0] = t.x; r.w[1] = t.y;
    } else if constexpr (sizeof(Scalar) == 2 && XV && VEC == 4) {
        const uint2 t = *reinterpret_cast<const uint2 *>(row + c);
        r.w[0] = t.x; r.w[1] = t.y;
    } else if constexpr (sizeof(Scalar) == 2 && XV && VEC == 2) {
        r.w[0] = *reinterpret_cast<const uint32_t *>(row + c);
    } else if constexpr (sizeof(Scalar) == 4) {
#pragma unroll
        for (int v = 0; v < VEC; ++v)
            r.w[v] = *reinterpret_cast<const uint32_t *>(row + (c + v < C ? c + v : 0));
    } else {
#pragma unroll
        for (int i = 0; i < r.kWords; ++i)
            r.w[i] = 0;
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
            const uint32_t h = *reinterpret_cast<const uint16_t *>(row + (c + v < C ? c + v : 0));
            r.w[v / 2] |= h << (16 * (v % 2));
        }
    }
    return r;
}

template<typename Scalar, int VEC>
__device__ __forceinline__ FVec<VEC> x_bits_to_f(const XBits<Scalar, VEC> &b) {
    FVec<VEC> r;
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
        if constexpr (sizeof(Scalar) == 4)
            r.v[v] = __uint_as_float(b.w[v]);
        else
            r.v[v] = half_bits_to_f<Scalar>((b.w[v / 2] >> (16 * (v % 2))) & 0xffffu);
    }
    return r;
}

template<typename Scalar>
__device__ __forceinline__ uint16_t to_bits16(float v) {
    if constexpr (sizeof(Scalar) == 2) {
        Scalar s;
        store_out(&s, v);
        return __builtin_bit_cast(uint16_t, s);
    } else {
        return 0;
    }
}

template<typename Scalar, int VEC>
__device__ __forceinline__ void store_act_vec(Scalar *p, const FVec<VEC> &r) {
    if constexpr (sizeof(Scalar) == 4 && VEC == 4) {
        *reinterpret_cast<float4 *>(p) = make_float4(r.v[0], r.v[1], r.v[2], r.v[3]);
    } else if constexpr (sizeof(Scalar) == 4 && VEC == 2) {
        *reinterpret_cast<float2 *>(p) = make_float2(r.v[0], r.v[1]);
    } else if constexpr (sizeof(Scalar) == 2 && VEC == 4) {
        const uint32_t lo = to_bits16<Scalar>(r.v[0]) | (static_cast<uint32_t>(to_bits16<Scalar>(r.v[1])) << 16);
        const uint32_t hi = to_bits16<Scalar>(r.v[2]) | (static_cast<uint32_t>(to_bits16<Scalar>(r.v[3])) << 16);
        *reinterpret_cast<uint2 *>(p) = make_uint2(lo, hi);
    } else if constexpr (sizeof(Scalar) == 2 && VEC == 2) {
        *reinterpret_cast<uint32_t *>(p) =
            to_bits16<Scalar>(r.v[0]) | (static_cast<uint32_t>(to_bits16<Scalar>(r.v[1])) << 16);
    } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i)
            store_out(p + i, r.v[i]);
    }
}

// Read in place of the mask when the caller passes none.
__device__ const uint8_t kScanAllValid = 1;

// Row stride (floats) of the LDS slot slice: one pad float per row spreads
// rows over banks; VEC-wide rows keep VEC-float alignment.
__host__ __device__ constexpr int scan_row_stride(int vec, int cs) { return cs + (vec == 1 ? 1 : vec); }

// Staged event: {write slot, gain, read slot, read weight}.
struct StageRec {
    int wslot;
    float g;
    int rslot;
    float r;
};

// LDS layout of a workgroup: slot slice (A + 2 rows: the dummy write row,
// the dummy read row, A slots), the masses (2 dummies + A), then two chunk
// buffers, 16-byte aligned, each holding the staged events (kChunk x E), x
// (CS rows), the overlap flags and the raw records (kChunk x E) for the mass
// wave. The precomputed-gain form has no masses and, per state wave, one
// private stage of its records and x.
__host__ __device__ constexpr size_t scan_stage_offset(int A, int rs, bool pre = false) {
    return ((static_cast<size_t>(A + 2) * rs + (pre ? 0 : static_cast<size_t>(A + 2))) * 4 + 15) / 16 * 16;
}
// Tokens per chunk: 16, or 8 when more than 64 events per token would make
// the double-buffered stage outgrow LDS. The precomputed-gain form with at
// most 8 events per token takes 32: its per-chunk work (fetch, deposit, row
// addresses, y stores) is spread over twice the tokens for a few KB more of
// private stage (config 2: segment stage 0.80 -> 0.78 ms). The records are
// padded to whole 32-token chunks either way.
__host__ __device__ constexpr int scan_chunk_len(int events, bool pre = false) {
    return events > 64 ? 8 : (pre && events <= 8) ? 2 * kChunk : kChunk;
}

// PRE: gains precomputed by the mass pre-pass (no mass column; the state
// waves stream their records from global memory and stage only x, one
// buffer). The mass-wave form double-buffers the raw records for the mass
// wave, the StageRec it produces, x and the overlap flags.
inline size_t scan_lds_bytes(int A, int vec, int epp, int np, int nw, int elem, bool pre = false) {
    const int cs = nw * (kWave / epp) * vec;
    const int ch = scan_chunk_len(epp * np, pre);
    const size_t state = scan_stage_offset(A, scan_row_stride(vec, cs), pre);
    const size_t x = static_cast<size_t>(cs) * (ch * elem + 16);
    if (pre)  // one private stage per wave: its records and its channels' x
        return state + static_cast<size_t>(nw) * ch * epp * np * 16 + x;
    const size_t rec = sizeof(StageRec) + sizeof(WriteRec) + sizeof(ReadRec);
    return state + 2 * (static_cast<size_t>(ch) * epp * np * rec + x + ch * sizeof(int));
}

// A workgroup owns one (b, h, CS-channel slice) unit: NW state waves, each
// owning CSW channels of the slice, and one mass wave. Per 16-token chunk:
//  * the mass wave replays the slot masses one chunk ahead of the state
//    waves (m <- alpha m + w per write event, in token order) and stages
//    each event's gain g = w / (m + eps) and effective read weight
//    (mass-aware: (sum r) (m r) / (sum m r + eps), else r);
//  * the state waves stage the chunk's x (one or two elements per thread),
//    read their events and x from the stage in bulk, and run the token loop:
//    s <- s + g (x - s) for the writes, then the weighted read sum -- the
//    per-token dependency chain is one LDS row read-modify-write;
//  * one barrier per chunk hands the double-buffered stage over.
// FAST: C is a multiple of CS, so every lane owns VEC real channels.
// PRE: the mass pre-pass (segment_mass_kernel) has already written the gain
// records (each write event's gain and, mass-aware, each read's effective
// weight); there is no mass wave and no mass column. Each state wave fetches
// its chunks (records, x of its channels, overlap flags) two chunks ahead
// into registers and stages them in a private LDS region: the waves run
// without a barrier from the first chunk to the write-back.
// RANGE (precomputed-gain form only): one slot range of a split slot space
// (segment_scan_range_kernel); the whole space otherwise.
template<typename Scalar, int VEC, int EPP, int NP, int NW, bool MA, bool FAST, bool PRE, bool RANGE, bool SAVE = false>
__device__ __forceinline__ void segment_scan_body(const SegmentJob &job, const ScanGeom &geo) {
    static_assert(PRE || !RANGE, "slot ranges need the precomputed-gain form");
    static_assert(!SAVE || (PRE && !RANGE && FAST && VEC == 1), "rows are saved by whole-slice one-channel lanes");
    constexpr int NWT = NW + (PRE ? 0 : 1);  // waves of the workgroup
    constexpr int LPE = kWave / EPP;
    constexpr int CSW = LPE * VEC;
    constexpr int CS = NW * CSW;
    constexpr int RS = scan_row_stride(VEC, CS);
    constexpr int NST = kWave * NW;           // state threads
    constexpr int E = EPP * NP;               // event lanes per token
    constexpr int CH = scan_chunk_len(E, PRE);  // tokens per chunk
    constexpr int MP = (E + 31) / 32;         // mass-wave passes (32 events each)
    constexpr int ES = static_cast<int>(sizeof(Scalar));
    constexpr int XRB = CH * ES + 16;  // staged x row: CH elements + 16 bytes against bank conflicts
    constexpr int XI = (CS * CH + NST - 1) / NST;  // staged x elements per state thread
    constexpr int NSL = EPP <= CH ? CH / EPP : 1;  // tokens whose y a lane stores
    constexpr int kStageRecBytes = PRE ? 0 : static_cast<int>(sizeof(StageRec));
    constexpr int kRawBytes = PRE ? 0 : static_cast<int>(sizeof(WriteRec) + sizeof(ReadRec));
    constexpr int kStageBytes = CH * E * (kStageRecBytes + kRawBytes) + CS * XRB + CH * 4;
    constexpr int RI = (E * CH + NST - 1) / NST;  // raw records per state thread
    using Bits = std::conditional_t<ES == 4, uint32_t, uint16_t>;

    extern __shared__ __align__(16) float lds[];
    // Workgroups are dealt round-robin to the 8 XCDs; give each XCD a
    // contiguous run of units so the slices of one (b, h) share an L2.
    const int per_xcd = (geo.n_units + 7) / 8;
    const int unit = static_cast<int>(blockIdx.x % 8) * per_xcd + static_cast<int>(blockIdx.x / 8);
    if (unit >= geo.n_units)
        return;
    const int tid = static_cast<int>(threadIdx.x);
    const int wave = tid / kWave;
    const int lane = tid % kWave;
    const bool mass_wave = !PRE && wave == NW;
    const int bh = unit / geo.n_slices;
    const int c0 = (unit - bh * geo.n_slices) * CS;
    const int T = job.T, A = job.A, C = job.C, Kw = job.Kw, Kr = job.Kr, Tp = geo.t_pad;
    const float eps = job.eps;
    // resident slot range: [r0, r0 + AL) (the whole space but in the
    // split launches of a wide one)
    const int r0 = RANGE ? geo.r0 : 0;
    const int AL = RANGE ? geo.n_local : A;
    const bool first_range = r0 == 0, last_range = geo.last != 0;

    float *st = lds + 2 * RS;              // slot 0 of the slice
    float *ms = lds + (AL + 2) * RS + 2;   // mass of slot 0
    char *stage0 = reinterpret_cast<char *>(lds) + scan_stage_offset(AL, RS, PRE);
    auto stage_e = [&](int buf) { return reinterpret_cast<StageRec *>(stage0 + buf * kStageBytes); };
    auto stage_x = [&](int buf) { return stage0 + buf * kStageBytes + CH * E * kStageRecBytes; };
    // per token: 1 if its writes may overlap the previous token's
    auto stage_f = [&](int buf) { return reinterpret_cast<int *>(stage_x(buf) + CS * XRB); };
    auto raw_w = [&](int buf) { return reinterpret_cast<WriteRec *>(stage_f(buf) + CH); };
    auto raw_r = [&](int buf) { return reinterpret_cast<ReadRec *>(raw_w(buf) + CH * E); };

    // ---- state slice and masses -> LDS
    {
        const float *src = job.init_slot + (static_cast<int64_t>(bh) * A + r0) * C;
        for (int i = tid; i < AL * CS; i += kWave * NWT) {
            const int a = i / CS, c = i - a * CS;
            const bool ok = c0 + c < C;
            const float v = src[static_cast<int64_t>(a) * C + (ok ? c0 + c : 0)];
            st[a * RS + c] = ok ? v : 0.f;
        }
        for (int i = tid; i < 2 * RS; i += kWave * NWT)
            lds[i] = 0.f;
        if constexpr (!PRE) {
            const float *msrc = job.init_mass + static_cast<int64_t>(bh) * A;
            for (int a = tid; a < A; a += kWave * NWT)
                ms[a] = msrc[a];
            if (tid < 2)
                ms[tid - 2] = 1.f;
        }
    }

    // ---- raw records: fetched by the state threads two chunks ahead (one
    // or two unique records per thread, clamped as for x) and deposited in
    // LDS for the mass wave, whose lanes 0..31 take write events
    // p * 32 + lane and lanes 32..63 read events p * 32 + lane - 32.
    const WriteRec *gw = job.wrec + static_cast<int64_t>(bh) * Kw * Tp;
    const ReadRec *gr = job.rrec + static_cast<int64_t>(bh) * Kr * Tp;
    // PRE: the gain records of the mass pre-pass, max(Kw, Kr) events per token
    const int EK = Kw > Kr ? Kw : Kr;
    const GainRec *gp = PRE ? job.gain + static_cast<int64_t>(bh) * EK * Tp : nullptr;
    const int hl = lane & 31;
    const bool wlane = lane < 32;
    struct RawRegs {
        int4 w[RI];  // write record (PRE: gain record)
        int2 r[RI];  // read record (unused in PRE)
    };
    auto raw_fetch = [&](int t0, RawRegs &rg) {
#pragma unroll
        for (int k = 0; k < RI; ++k) {
            const int it = min(tid + k * NST, E * CH - 1);
            const int e = it / CH, j = it % CH;
            const int ew = e < Kw ? e : Kw - 1, er = e < Kr ? e : Kr - 1;
            rg.w[k] = ld16(gw + static_cast<int64_t>(ew) * Tp + t0 + j);
            rg.r[k] = *reinterpret_cast<const int2 *>(gr + static_cast<int64_t>(er) * Tp + t0 + j);
        }
    };
    auto raw_deposit = [&](int buf, const RawRegs &rg) {
        WriteRec *rw = raw_w(buf);
        ReadRec *rr = raw_r(buf);
#pragma unroll
        for (int k = 0; k < RI; ++k) {
            const int it = min(tid + k * NST, E * CH - 1);
            const int e = it / CH, j = it % CH;
            st16(rw + j * E + e, rg.w[k]);
            *reinterpret_cast<int2 *>(rr + j * E + e) = rg.r[k];
        }
    };
    struct Raw {
        int4 w[MP][CH];
        int2 r[MP][CH];
    };
    auto mass_load = [&](int buf, Raw &raw) {
        const WriteRec *rw = raw_w(buf);
        const ReadRec *rr = raw_r(buf);
#pragma unroll
        for (int p = 0; p < MP; ++p) {
            const int e = min(p * 32 + hl, E - 1);
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                raw.w[p][j] = *reinterpret_cast<const int4 *>(rw + j * E + e);
                raw.r[p][j] = *reinterpret_cast<const int2 *>(rr + j * E + e);
            }
        }
    };
    // Replays the chunk's mass updates and stages {slot, gain, slot, weight}
    // and the overlap flags. Tokens go in pairs: the second token's masses
    // are read before the first token's writes and read again only when the
    // two tokens' write sets may overlap (flag of the second token).
    auto mass_chunk = [&](int buf) {
        Raw raw;
        mass_load(buf, raw);
        StageRec *se = stage_e(buf);
        int *sf = stage_f(buf);
        auto wev = [&](int p, int j, int &a, float &w, float &al) {
            const bool on = wlane && p * 32 + hl < Kw;
            a = on ? raw.w[p][j].x : -2;
            w = on ? __int_as_float(raw.w[p][j].y) : 0.f;
            al = on ? __int_as_float(raw.w[p][j].z) : 1.f;
        };
        // Stage entries are kept in registers and written after the chunk, so
        // the LDS ops of the mass chain are only the mass reads and writes.
        int2 out[MP][CH];
        // writes of token j from masses m, then its reads
        auto finish = [&](int j, const int (&a)[MP], const float (&w)[MP], const float (&al)[MP], float (&m)[MP]) {
            float gg[MP];
#pragma unroll
            for (int p = 0; p < MP; ++p) {
                const float m2 = fmaf(al[p], m[p], w[p]);
                ms[a[p]] = m2;
                gg[p] = scan_gain(w[p], m2 + eps);
            }
            int rb[MP];
            float rr[MP];
            float sr = 0.f, srm = 0.f;
#pragma unroll
            for (int p = 0; p < MP; ++p) {
                const bool on = !wlane && p * 32 + hl < Kr;
                rb[p] = on ? raw.r[p][j].x : -1;
                rr[p] = on ? __int_as_float(raw.r[p][j].y) : 0.f;
                if constexpr (MA) {
                    const float wm = rr[p] * ms[rb[p]];  // post-write mass
                    sr += rr[p];
                    srm += wm;
                    rr[p] = wm;
                }
            }
            if constexpr (MA) {
                sr = event_sum<32>(sr);
                srm = event_sum<32>(srm);
                const float scale = sr / (srm + eps);
#pragma unroll
                for (int p = 0; p < MP; ++p)
                    rr[p] *= scale;
            }
#pragma unroll
            for (int p = 0; p < MP; ++p)
                out[p][j] = wlane ? make_int2(a[p], __float_as_int(gg[p])) : make_int2(rb[p], __float_as_int(rr[p]));
        };
#pragma unroll
        for (int j0 = 0; j0 < CH; j0 += 2) {
            const int j1 = j0 + 1;
            const int ov = __builtin_amdgcn_readfirstlane(raw.w[0][j1].w) & 1;  // shares a slot with token j0
            int a0[MP], a1[MP];
            float w0[MP], w1[MP], al0[MP], al1[MP], m0[MP], m1[MP];
#pragma unroll
            for (int p = 0; p < MP; ++p) {
                wev(p, j0, a0[p], w0[p], al0[p]);
                wev(p, j1, a1[p], w1[p], al1[p]);
                m0[p] = ms[a0[p]];
                m1[p] = ms[a1[p]];
            }
            finish(j0, a0, w0, al0, m0);
            if (ov) {
#pragma unroll
                for (int p = 0; p < MP; ++p)
                    m1[p] = ms[a1[p]];
            }
            finish(j1, a1, w1, al1, m1);
        }
#pragma unroll
        for (int p = 0; p < MP; ++p) {
            const int e = p * 32 + hl;
            if (e < E) {
#pragma unroll
                for (int j = 0; j < CH; ++j)
                    *(reinterpret_cast<int2 *>(se + j * E + e) + (wlane ? 0 : 1)) = out[p][j];
            }
        }
        if (lane == 0) {  // write event 0 carries every token's flag
#pragma unroll
            for (int q = 0; q < CH / 4; ++q)
                reinterpret_cast<int4 *>(sf)[q] =
                    make_int4(raw.w[0][4 * q].w, raw.w[0][4 * q + 1].w, raw.w[0][4 * q + 2].w, raw.w[0][4 * q + 3].w);
        }
    };

    // ---- state waves
    // Lane order. With LPE >= 8 lanes per event, channel-fastest: an event's
    // lanes read consecutive channels of its row, so an LDS pass meets fewer
    // distinct (random) rows and fewer bank conflicts, and the event sum is
    // a strided butterfly of three exchanges. With fewer lanes per event the
    // strided butterfly costs more than the conflicts it saves, and events
    // run fastest (event sum by DPP within a row).
    constexpr bool CFL = LPE >= 8;
    const int ev = CFL ? lane / LPE : lane % EPP;  // event slot within a pass
    const int cg = CFL ? lane % LPE : lane / EPP;  // channel group within the wave
    const int cl = wave * CSW + cg * VEC;     // first channel of this lane within the slice
    // Read sums by reduce-scatter over each run of EPP tokens (EPP <= CH):
    // event bit i sits on lane bit i + SH. Masks of the lane bits, once.
    constexpr bool BFLY = EPP <= CH;
    constexpr int LOGE = __builtin_ctz(EPP);
    constexpr int SH = CFL ? 6 - LOGE : 0;
    uint32_t hi[6];
    hi[0] = bit_mask<1>(lane);
    hi[1] = bit_mask<2>(lane);
    hi[2] = bit_mask<4>(lane);
    hi[3] = bit_mask<8>(lane);
    hi[4] = bit_mask<16>(lane);
    hi[5] = bit_mask<32>(lane);
    // LDS address of this lane's first channel in slot 0
    const uint32_t lrow = lds_addr(st) + static_cast<uint32_t>(cl) * 4;
    // SAVE: each token's x - s of every write row and every read row go to
    // the backward's slices (SavedRows), through buffer resources over the
    // head's region: a byte offset per lane and pass (its channel and event
    // slot) plus a scalar offset per token. The host guarantees that every
    // lane's channel is below C and its event slot below kp. The region
    // holds Tp tokens, so the tail chunk stores without a guard: a store
    // under a branch would make the compiler assume fewer stores in flight
    // on every path and wait for the chunk's stores before each deposit.
    const SavedRows &sv = job.save;
    const int64_t sv_head = SAVE ? static_cast<int64_t>(bh) * sv.n_sub * Tp * sv.kp * sv.csw : 0;
    const int sv_bytes = SAVE ? sv.n_sub * Tp * sv.kp * sv.csw * 4 : 0;
    [[maybe_unused]] const auto svw = __builtin_amdgcn_make_buffer_rsrc(SAVE ? sv.w + sv_head : nullptr, 0, sv_bytes, kBufWord3);
    [[maybe_unused]] const auto svr = __builtin_amdgcn_make_buffer_rsrc(SAVE ? sv.r + sv_head : nullptr, 0, sv_bytes, kBufWord3);
    [[maybe_unused]] int svo[NP] = {};
    [[maybe_unused]] int sv_tok = 0;
    if constexpr (SAVE) {
        const int c = c0 + cl, lg = __builtin_ctz(static_cast<unsigned>(sv.csw));
#pragma unroll
        for (int p = 0; p < NP; ++p)
            svo[p] = (((c >> lg) * Tp * sv.kp + p * EPP + ev) * sv.csw + (c & (sv.csw - 1))) * 4;
        sv_tok = sv.kp * sv.csw * 4;
    }
    const Scalar *gx = static_cast<const Scalar *>(job.x) + static_cast<int64_t>(bh) * T * C;
    Scalar *gy = static_cast<Scalar *>(job.y) + static_cast<int64_t>(bh) * T * C;
    // Items past the end are clamped to the last item, so the threads that
    // hold them load and store identical data (no branch).
    auto x_fetch = [&](int t0, Bits (&xb)[XI]) {
#pragma unroll
        for (int k = 0; k < XI; ++k) {
            const int it = min(tid + k * NST, CS * CH - 1);
            const int j = it / CS, c = it % CS;
            const int t = t0 + j < T ? t0 + j : T - 1;
            const int ch = c0 + c < C ? c0 + c : C - 1;
            xb[k] = *reinterpret_cast<const Bits *>(gx + static_cast<int64_t>(t) * C + ch);
        }
    };
    auto x_deposit = [&](int buf, const Bits (&xb)[XI]) {
        char *sx = stage_x(buf);
#pragma unroll
        for (int k = 0; k < XI; ++k) {
            const int it = min(tid + k * NST, CS * CH - 1);
            const int j = it / CS, c = it % CS;
            *reinterpret_cast<Bits *>(sx + c * XRB + j * ES) = xb[k];
        }
    };
    // Records {write slot, gain, read slot, read weight} of one chunk, per
    // pass and token, as the state waves use them.
    struct Recs {
        int4 r[NP][CH];
    };
    // Row address arithmetic per pass: slot * amul + base. In the PRE form
    // lanes past the head's events (their staged records are copies of the
    // last event's) write the dummy row -2 and read the zero row -1.
    int amul[NP], awb[NP], arb[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        const bool dead = PRE && p * EPP + ev >= EK;
        amul[p] = dead ? 0 : RS * 4;
        awb[p] = dead ? static_cast<int>(lds_addr(lds) + cl * 4) : static_cast<int>(lrow);
        arb[p] = dead ? static_cast<int>(lds_addr(lds + RS) + cl * 4) : static_cast<int>(lrow);
    }
    // PRE: every wave stages its own chunk -- the gain records of all events
    // (token-major, as the pre-pass writes them) and the x of its CSW
    // channels -- in a private LDS region, from registers filled two chunks
    // ahead. A wave's LDS accesses stay in program order, so the waves need
    // no barrier until the write-back.
    constexpr int RW = (CH * E + kWave - 1) / kWave;   // records per lane
    constexpr int XIW = (CSW * CH + kWave - 1) / kWave;  // x elements per lane
    constexpr int kPrivRec = CH * E * 16;
    constexpr int kPrivBytes = kPrivRec + CSW * XRB;
    char *priv = stage0 + wave * kPrivBytes;
    const char *priv_x = priv + kPrivRec - wave * CSW * XRB;  // row of slice channel c at c * XRB
    struct Fetch {
        int4 rec[RW];
        Bits x[XIW];
        int flag;  // overlap flag of token (lane), lanes < CH
    };
    auto pre_fetch = [&](int t0, Fetch &f) {
        const char *g = reinterpret_cast<const char *>(gp + static_cast<int64_t>(t0) * EK);
#pragma unroll
        for (int k = 0; k < RW; ++k) {
            const int it = min(lane + k * kWave, CH * E - 1);
            const int j = it / E, e = it % E;
            f.rec[k] = ld16(g + static_cast<uint32_t>(j * EK + min(e, EK - 1)) * 16u);
        }
#pragma unroll
        for (int k = 0; k < XIW; ++k) {
            const int it = min(lane + k * kWave, CSW * CH - 1);
            const int j = it / CSW, c = wave * CSW + it % CSW;
            const int t = t0 + j < T ? t0 + j : T - 1;
            const int ch = c0 + c < C ? c0 + c : C - 1;
            f.x[k] = *reinterpret_cast<const Bits *>(gx + static_cast<int64_t>(t) * C + ch);
        }
        // write event 0's record carries the token's overlap flag (a load
        // without a branch: a conditional one would be waited for at once)
        const int *fp = Kw > 0 ? reinterpret_cast<const int *>(&gw[t0 + min(lane, CH - 1)].overlap) : &kNoFlag;
        f.flag = *fp;
    };
    auto pre_deposit = [&](const Fetch &f) {
#pragma unroll
        for (int k = 0; k < RW; ++k) {
            const int it = min(lane + k * kWave, CH * E - 1);
            st16(priv + it * 16, f.rec[k]);
        }
        char *px = const_cast<char *>(priv_x);
#pragma unroll
        for (int k = 0; k < XIW; ++k) {
            const int it = min(lane + k * kWave, CSW * CH - 1);
            const int j = it / CSW, c = wave * CSW + it % CSW;
            *reinterpret_cast<Bits *>(px + c * XRB + j * ES) = f.x[k];
        }
    };
    // Reload mask of a chunk from its tokens' overlap flags (one token per
    // lane): token j, at position i = j % 4 of its group, is reloaded when it
    // may share a written slot with one of the i tokens before it.
    auto flag_mask = [&](int fv) -> uint64_t {
        return __ballot(lane < CH && (fv & ((1 << (lane & 3)) - 1)) != 0);
    };
    // records of one chunk from a stage laid out [token][event]
    auto stage_recs = [&](const void *se, Recs &rc) {
#pragma unroll
        for (int j = 0; j < CH; ++j)
#pragma unroll
            for (int p = 0; p < NP; ++p)
                rc.r[p][j] = ld16(static_cast<const int4 *>(se) + j * E + p * EPP + ev);
    };
    // One chunk of the state waves. The token body is branch-free; each lane
    // keeps the read sum of the tokens whose y it stores. TAIL guards tokens
    // past T.
    // rc: the chunk's records, consumed (turned into row addresses).
    auto state_chunk = [&](const char *sx, int t0, auto tail_tag, Recs &rc, uint64_t fm) {
        constexpr bool TAIL = decltype(tail_tag)::value;
        auto &rec = rc.r;
        constexpr int XW = CH * ES / 16;  // 16-byte words per staged channel row
        uint4 xr[VEC][XW];
#pragma unroll
        for (int v = 0; v < VEC; ++v)
#pragma unroll
            for (int q = 0; q < XW; ++q)
                xr[v][q] = *reinterpret_cast<const uint4 *>(sx + (cl + v) * XRB + q * 16);
        auto x_at = [&](int v, int j) -> float {
            const uint4 q4 = xr[v][(j * ES) / 16];
            const int wi = ((j * ES) % 16) / 4;
            const uint32_t wd = wi == 0 ? q4.x : wi == 1 ? q4.y : wi == 2 ? q4.z : q4.w;
            if constexpr (ES == 4)
                return __uint_as_float(wd);
            else
                return half_bits_to_f<Scalar>((wd >> (16 * (j % 2))) & 0xffffu);
        };

        FVec<VEC> ykeep[NSL];
#pragma unroll
        for (int q = 0; q < NSL; ++q)
#pragma unroll
            for (int v = 0; v < VEC; ++v)
                ykeep[q].v[v] = 0.f;
        auto flag = [&](int j) { return ((fm >> j) & 1u) != 0; };
        // LDS addresses of the rows of token j's events (a 24-bit
        // multiply-add each). The first group's are
        // computed before the token loop, each later group's during the
        // group before it, where they fill the wait for that group's rows.
        // PRE records past T were never written: those tokens act on the
        // dummy rows.
        auto addresses = [&](int j) {
#pragma unroll
                for (int p = 0; p < NP; ++p) {
                    int wa = rec[p][j].x, ra = rec[p][j].z;
                    if constexpr (PRE && TAIL) {
                        const bool live = t0 + j < T;
                        wa = live ? wa : -2;
                        ra = live ? ra : -1;
                        rec[p][j].w = live ? rec[p][j].w : 0;
                    }
                    if constexpr (RANGE) {
                        // events on slots outside the resident range act on
                        // the dummy rows (the no-op slots -2, -1 stay outside)
                        const int lw = wa - r0, lr = ra - r0;
                        const bool iw = static_cast<unsigned>(lw) < static_cast<unsigned>(AL);
                        const bool ir = static_cast<unsigned>(lr) < static_cast<unsigned>(AL);
                        wa = iw ? lw : -2;
                        ra = ir ? lr : -1;
                        rec[p][j].w = ir ? rec[p][j].w : 0;
                    }
                    rec[p][j].x = mad24(wa, amul[p], awb[p]);
                    rec[p][j].z = mad24(ra, amul[p], arb[p]);
                }
        };
        auto row = [&](int a) { return lds_at(static_cast<uint32_t>(a)); };
        auto load_rows = [&](int j, FVec<VEC> (&s)[NP]) {
#pragma unroll
            for (int p = 0; p < NP; ++p)
                s[p] = lds_load<VEC>(row(rec[p][j].x));
        };
        // writes s <- s + g (x - s) of token j, then the loads of its read rows
        auto write_read = [&](int j, const FVec<VEC> (&s)[NP], FVec<VEC> (&rv)[NP]) {
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                const float g = __int_as_float(rec[p][j].y);
                FVec<VEC> o, d;
#pragma unroll
                for (int v = 0; v < VEC; ++v) {
                    d.v[v] = x_at(v, j) - s[p].v[v];
                    o.v[v] = fmaf(g, d.v[v], s[p].v[v]);
                }
                lds_store<VEC>(row(rec[p][j].x), o);
                if constexpr (SAVE)
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(d.v[0]), svw, svo[p], (t0 + j) * sv_tok, 0);
            }
#pragma unroll
            for (int p = 0; p < NP; ++p)
                rv[p] = lds_load<VEC>(row(rec[p][j].z));
        };
        // weighted read sum of token j, kept in the lanes that store its y:
        // the lane's partial of every token of a run of EPP, then one
        // reduce-scatter per run (BFLY), else a sum over the event lanes per
        // token
        float part[VEC][BFLY ? EPP : 1];
        auto reduce = [&](int j, const FVec<VEC> (&rv)[NP]) {
            if constexpr (SAVE) {
#pragma unroll
                for (int p = 0; p < NP; ++p)
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(rv[p].v[0]), svr, svo[p], (t0 + j) * sv_tok, 0);
            }
            FVec<VEC> acc;
#pragma unroll
            for (int v = 0; v < VEC; ++v)
                acc.v[v] = __int_as_float(rec[0][j].w) * rv[0].v[v];
#pragma unroll
            for (int p = 1; p < NP; ++p) {
                const float wgt = __int_as_float(rec[p][j].w);
#pragma unroll
                for (int v = 0; v < VEC; ++v)
                    acc.v[v] = fmaf(wgt, rv[p].v[v], acc.v[v]);
            }
            if constexpr (BFLY) {
                // (opaque: the first exchange's DPP add would otherwise be
                // contracted with the product into a DPP move and an fma)
#pragma unroll
                for (int v = 0; v < VEC; ++v)
                    part[v][j % EPP] = __uint_as_float(opaque(__float_as_uint(acc.v[v])));
                if (j % EPP == EPP - 1) {
#pragma unroll
                    for (int v = 0; v < VEC; ++v) {
                        event_scatter<LOGE - 1, SH, EPP>(part[v], hi);
                        ykeep[j / EPP].v[v] = part[v][0];
                    }
                }
            } else {
#pragma unroll
                for (int v = 0; v < VEC; ++v)
                    acc.v[v] = CFL ? strided_sum<LPE>(acc.v[v]) : event_sum<EPP>(acc.v[v]);
                const bool mine = ev % CH == j;
#pragma unroll
                for (int v = 0; v < VEC; ++v)
                    ykeep[0].v[v] = mine ? acc.v[v] : ykeep[0].v[v];
            }
        };
        // Groups of four tokens: the rows of all four are loaded before the
        // first token's writes, and a token's rows are loaded again when its
        // writes may meet an earlier token's of the group (reload mask). The
        // read sums of a group are reduced after the next group's row loads
        // are issued, so the only LDS round trip on the token chain is one
        // row load per group. The reload path drains LDS itself (a rare
        // branch); otherwise the wait merged at its join would also cover the
        // earlier tokens' read rows.
        constexpr int G = 4;
        static_assert(CH % G == 0, "chunks hold whole token groups");
        FVec<VEC> rp[G][NP];
#pragma unroll
        for (int i = 0; i < G; ++i)
            addresses(i);
#pragma unroll
        for (int j0 = 0; j0 < CH; j0 += G) {
            FVec<VEC> sv[G][NP];
#pragma unroll
            for (int i = 0; i < G; ++i)
                load_rows(j0 + i, sv[i]);
            if (j0 > 0) {
#pragma unroll
                for (int i = 0; i < G; ++i)
                    reduce(j0 - G + i, rp[i]);
            }
            if (j0 + G < CH) {
#pragma unroll
                for (int i = 0; i < G; ++i)
                    addresses(j0 + G + i);
            }
            // Up to 8 events per token, a group whose tokens meet none of
            // their group's earlier ones skips the per-token checks (config
            // 2: 0.78 -> 0.77 ms; at 16 events, config 4, the extra branch
            // cost more than it saved: 1.42 -> 1.46 ms).
            if (E <= 8 && __builtin_expect(((fm >> j0) & ((1u << G) - 1)) == 0, 1)) {
#pragma unroll
                for (int i = 0; i < G; ++i)
                    write_read(j0 + i, sv[i], rp[i]);
            } else {
                write_read(j0, sv[0], rp[0]);
#pragma unroll
                for (int i = 1; i < G; ++i) {
                    if (__builtin_expect(flag(j0 + i), 0)) {
                        load_rows(j0 + i, sv[i]);
                        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
                    }
                    write_read(j0 + i, sv[i], rp[i]);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < G; ++i)
            reduce(CH - G + i, rp[i]);
        // y of this chunk: lane stores tokens q * EPP + ev (or ev % 16)
#pragma unroll
        for (int q = 0; q < NSL; ++q) {
            const int j = EPP <= CH ? q * EPP + ev : ev % CH;
            const int t = t0 + j;
            Scalar *yp = gy + static_cast<int64_t>(t) * C + c0 + cl;
            if constexpr (RANGE) {
                // slot ranges: the read sums of the ranges so far stay fp32
                // in yacc; the last range adds its own and stores y
                if (t < T) {
                    float *ap = job.yacc + (static_cast<int64_t>(bh) * T + t) * C + c0 + cl;
#pragma unroll
                    for (int v = 0; v < VEC; ++v) {
                        if (FAST || c0 + cl + v < C) {
                            const float sum = (first_range ? 0.f : ap[v]) + ykeep[q].v[v];
                            if (last_range)
                                store_out(yp + v, sum);
                            else
                                ap[v] = sum;
                        }
                    }
                }
            } else if constexpr (FAST) {
                if (!TAIL || t < T)
                    store_act_vec<Scalar, VEC>(yp, ykeep[q]);
            } else if (t < T) {
#pragma unroll
                for (int v = 0; v < VEC; ++v)
                    if (c0 + cl + v < C)
                        store_out(yp + v, ykeep[q].v[v]);
            }
        }
    };

    // ---- pipeline. Iteration ci: the state waves run chunk ci (stage
    // ci & 1) while the mass wave stages chunk ci + 1 (records fetched one
    // iteration earlier) and fetches chunk ci + 2. Chunks wholly inside T
    // run the unguarded state body; at most one chunk at the end reaches
    // past T.
    using Full = std::false_type;
    using Tail = std::true_type;
    const int nc = (T + CH - 1) / CH;
    const int n_full = T / CH;
    auto clampc = [&](int c) { return (c < nc ? c : nc - 1) * CH; };
    RawRegs rg;
    Bits xb[XI];
    if constexpr (PRE) {
        // Iteration ci: chunk ci runs from the private stage (deposited at
        // the end of chunk ci - 1) while the registers of chunk ci + 2 fill;
        // after it, chunk ci + 1 (fetched two chunks earlier) is deposited.
        // The overlap flags become a scalar mask at deposit, so no loaded
        // vector value is live across the next fetch into its registers (the
        // copy that would keep it waits for every outstanding memory
        // operation, the chunk's y stores included).
        Fetch fa, fb;
        uint64_t fm = 0;  // flags of the chunk in the stage
        __syncthreads();  // state slice loaded
        if (nc > 0) {
            pre_fetch(0, fa);
            pre_fetch(clampc(1), fb);
            pre_deposit(fa);
            fm = flag_mask(fa.flag);
        }
        // SAVE: one chunk body for every chunk. Around a choice between two
        // bodies the compiler keeps an edge that skips both, and its memory
        // waits then assume that none of a chunk's row stores are in flight:
        // each deposit would wait for the whole chunk's stores.
        auto run = [&](int ci, uint64_t m) {
            Recs rc;
            stage_recs(priv, rc);
            if (!SAVE && ci < n_full)
                state_chunk(priv_x, ci * CH, Full{}, rc, m);
            else
                state_chunk(priv_x, ci * CH, Tail{}, rc, m);
        };
        for (int ci = 0; ci < nc; ci += 2) {
            pre_fetch(clampc(ci + 2), fa);
            __builtin_amdgcn_sched_barrier(0);
            run(ci, fm);
            __builtin_amdgcn_sched_barrier(0);
            pre_deposit(fb);
            fm = flag_mask(fb.flag);
            if (ci + 1 >= nc)
                break;
            pre_fetch(clampc(ci + 3), fb);
            __builtin_amdgcn_sched_barrier(0);
            run(ci + 1, fm);
            __builtin_amdgcn_sched_barrier(0);
            pre_deposit(fa);
            fm = flag_mask(fa.flag);
        }
        __syncthreads();
    } else {
        __syncthreads();  // masses initialised before the mass wave starts
        if (nc > 0) {
            if (!mass_wave) {
                raw_fetch(0, rg);
                raw_deposit(0, rg);
                raw_fetch(clampc(1), rg);
                raw_deposit(1, rg);
                x_fetch(0, xb);
                x_deposit(0, xb);
            }
            __syncthreads();
            if (mass_wave)
                mass_chunk(0);
        }
        __syncthreads();
        // Iteration ci: the state waves run chunk ci (stage ci & 1), fetch x of
        // chunk ci + 1 and the raw records of chunk ci + 2; the mass wave stages
        // chunk ci + 1 from the raw records deposited one iteration earlier.
        for (int ci = 0; ci < nc; ++ci) {
            if (mass_wave) {
                if (ci + 1 < nc)
                    mass_chunk((ci + 1) & 1);
            } else {
                // scheduling fences keep the loads at the top and their use at
                // the bottom, so a whole chunk of work covers their latency
                x_fetch(clampc(ci + 1), xb);
                raw_fetch(clampc(ci + 2), rg);
                __builtin_amdgcn_sched_barrier(0);
                Recs rc;
                stage_recs(stage_e(ci & 1), rc);
                const uint64_t fm = flag_mask(stage_f(ci & 1)[min(lane, CH - 1)]);
                if (ci < n_full)
                    state_chunk(stage_x(ci & 1), ci * CH, Full{}, rc, fm);
                else
                    state_chunk(stage_x(ci & 1), ci * CH, Tail{}, rc, fm);
                __builtin_amdgcn_sched_barrier(0);
                x_deposit((ci + 1) & 1, xb);
                raw_deposit(ci & 1, rg);
            }
            __syncthreads();
        }
    }

    // ---- LDS -> post state (whole workgroup); the masses from slice 0
    {
        float *dst = job.slot_out + (static_cast<int64_t>(bh) * A + r0) * C;
        for (int i = tid; i < AL * CS; i += kWave * NWT) {
            const int a = i / CS, c = i - a * CS;
            if (c0 + c < C)
                dst[static_cast<int64_t>(a) * C + c0 + c] = st[a * RS + c];
        }
        if (!PRE && c0 == 0) {
            float *mdst = job.mass_out + static_cast<int64_t>(bh) * A;
            for (int a = tid; a < A; a += kWave * NWT)
                mdst[a] = ms[a];
        }
    }
}

template<typename Scalar, int VEC, int EPP, int NP, int NW, bool MA, bool FAST, bool PRE, bool SAVE = false>
__global__ __launch_bounds__(kWave * (NW + (PRE ? 0 : 1))) void segment_scan_kernel(const SegmentJob job,
                                                                                     const ScanGeom geo) {
    segment_scan_body<Scalar, VEC, EPP, NP, NW, MA, FAST, PRE, false, SAVE>(job, geo);
}

template<typename Scalar, int VEC, int EPP, int NP, int NW, bool MA, bool FAST>
__global__ __launch_bounds__(kWave * NW) void segment_scan_range_kernel(const SegmentJob job, const ScanGeom geo) {
    segment_scan_body<Scalar, VEC, EPP, NP, NW, MA, FAST, true, true>(job, geo);
}

template<typename Scalar, int VEC, int EPP, int NP, int NW, bool MA, bool FAST, bool PRE, bool SAVE = false>
hipError_t launch_scan(const SegmentJob &job, const ScanGeom &geo, hipStream_t stream) {
    const unsigned blocks = static_cast<unsigned>(((geo.n_units + 7) / 8) * 8);
    if constexpr (SAVE) {
        hipLaunchKernelGGL((segment_scan_kernel<Scalar, VEC, EPP, NP, NW, MA, FAST, true, true>), dim3(blocks),
                           dim3(kWave * NW),
                           scan_lds_bytes(geo.n_local, VEC, EPP, NP, NW, static_cast<int>(sizeof(Scalar)), true), stream,
                           job, geo);
        return hipGetLastError();
    }
    if constexpr (PRE) {
        if (geo.n_local != job.A) {
            hipLaunchKernelGGL((segment_scan_range_kernel<Scalar, VEC, EPP, NP, NW, MA, FAST>), dim3(blocks),
                               dim3(kWave * NW),
                               scan_lds_bytes(geo.n_local, VEC, EPP, NP, NW, static_cast<int>(sizeof(Scalar)), true),
                               stream, job, geo);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((segment_scan_kernel<Scalar, VEC, EPP, NP, NW, MA, FAST, PRE>), dim3(blocks),
                       dim3(kWave * (NW + (PRE ? 0 : 1))),
                       scan_lds_bytes(geo.n_local, VEC, EPP, NP, NW, static_cast<int>(sizeof(Scalar)), PRE), stream, job,
                       geo);
    return hipGetLastError();
}

// Layouts compiled for every activation dtype: (VEC, EPP, NP, NW).
#define RAMNET_SCAN_LAYOUTS(X)                                                                       \
    X(1, 4, 1, 1) X(1, 8, 1, 1) X(1, 16, 1, 1) X(1, 32, 1, 1) X(1, 64, 1, 1) X(1, 64, 2, 1)         \
    X(1, 8, 1, 2) X(1, 8, 1, 4) X(1, 8, 2, 1) X(1, 8, 2, 2) X(1, 8, 2, 4) X(1, 16, 1, 2) X(1, 16, 1, 4) \
    X(2, 8, 1, 1) X(2, 8, 1, 2) X(2, 8, 1, 4) X(2, 16, 1, 1) X(2, 16, 1, 2)                          \
    X(4, 8, 1, 1) X(4, 8, 1, 2) X(4, 16, 1, 1)
// Layouts also compiled in the precomputed-gain (PRE) form: the wide
// slot spaces, where dropping the mass column lets a slice hold twice the
// channels.
#define RAMNET_SCAN_PRE_LAYOUTS(X)                                                                   \
    X(1, 8, 1, 2) X(1, 8, 1, 4) X(1, 16, 1, 2) X(1, 16, 1, 4) X(1, 32, 1, 2) X(1, 64, 1, 2) X(1, 64, 2, 1)

// A scan that saves rows (job.save.w set) runs a precomputed-gain layout
// over the whole slot space with whole slices (FAST); the host checks this.
template<typename Scalar>
hipError_t scan_dispatch(const SegmentJob &job, const ScanGeom &geo, int vec, int epp, int np, int nw, bool pre,
                         hipStream_t stream) {
    const int cs = nw * (kWave / epp) * vec;
    const bool fast = job.C % cs == 0;
    if (job.save.w != nullptr) {
        if (!pre || !fast || vec != 1 || geo.n_local != job.A)
            return hipErrorInvalidValue;
#define RAMNET_SCAN_CASE_SAVE(V, E, N, W)                                                            \
        if (V == 1 && epp == E && np == N && nw == W)                                                \
            return job.mass_aware ? launch_scan<Scalar, 1, E, N, W, true, true, true, true>(job, geo, stream) \
                                  : launch_scan<Scalar, 1, E, N, W, false, true, true, true>(job, geo, stream);
        RAMNET_SCAN_PRE_LAYOUTS(RAMNET_SCAN_CASE_SAVE)
#undef RAMNET_SCAN_CASE_SAVE
        return hipErrorInvalidValue;
    }
#define RAMNET_SCAN_CASE(V, E, N, W, P)                                                              \
    if (pre == P && vec == V && epp == E && np == N && nw == W) {                                    \
        if (job.mass_aware)                                                                          \
            return fast ? launch_scan<Scalar, V, E, N, W, true, true, P>(job, geo, stream)           \
                        : launch_scan<Scalar, V, E, N, W, true, false, P>(job, geo, stream);         \
        return fast ? launch_scan<Scalar, V, E, N, W, false, true, P>(job, geo, stream)              \
                    : launch_scan<Scalar, V, E, N, W, false, false, P>(job, geo, stream);            \
    }
#define RAMNET_SCAN_CASE_MASS(V, E, N, W) RAMNET_SCAN_CASE(V, E, N, W, false)
#define RAMNET_SCAN_CASE_PRE(V, E, N, W) RAMNET_SCAN_CASE(V, E, N, W, true)
    RAMNET_SCAN_LAYOUTS(RAMNET_SCAN_CASE_MASS)
    RAMNET_SCAN_PRE_LAYOUTS(RAMNET_SCAN_CASE_PRE)
#undef RAMNET_SCAN_CASE_PRE
#undef RAMNET_SCAN_CASE_MASS
#undef RAMNET_SCAN_CASE
    return hipErrorInvalidValue;
}

// Whether (vec, epp, np, nw) is one of the compiled layouts (in PRE form if pre).
inline bool scan_layout_compiled(int vec, int epp, int np, int nw, bool pre = false) {
#define RAMNET_SCAN_HAS(V, E, N, W) if (vec == V && epp == E && np == N && nw == W) return true;
    if (pre) {
        RAMNET_SCAN_PRE_LAYOUTS(RAMNET_SCAN_HAS)
    } else {
        RAMNET_SCAN_LAYOUTS(RAMNET_SCAN_HAS)
    }
#undef RAMNET_SCAN_HAS
    return false;
}

// One definition per activation dtype, each in its own translation unit.
hipError_t launch_scan_f32(const SegmentJob &, const ScanGeom &, int, int, int, int, bool, hipStream_t);
hipError_t launch_scan_f16(const SegmentJob &, const ScanGeom &, int, int, int, int, bool, hipStream_t);
hipError_t launch_scan_bf16(const SegmentJob &, const ScanGeom &, int, int, int, int, bool, hipStream_t);

}  // namespace ramnet
