// Time-ordered segment scan kernel (gated sparse update + top-K read).
//
// One 64-lane wave owns one (b, h, channel slice) unit and walks the whole
// sequence with the unit's A x CS slot slice and the slot masses resident in
// LDS. The lane layout is fixed at compile time:
//   EPP events per pass (lane % EPP), LPE = 64 / EPP lanes per event,
//   VEC channels per lane, CS = LPE * VEC channels per unit,
//   NP passes cover up to NP * EPP write and NP * EPP read events per token.
// Per-event records ({slot, w, alpha} for writes, {slot, r} for reads; see
// ramnet_kernels.hpp) and the lane's x channels are loaded straight from
// global memory into registers one kScanChunk-token chunk ahead of use, so
// the token loop touches LDS only for the slot state. The chunk body is
// fully unrolled and branch-free: events that must not act point at two
// dummy LDS rows in front of the state (slot -2 for writes, -1 for reads),
// so every load and store is unconditional. LDS executes a wave's accesses
// in program order, which carries the read-modify-write dependency from one
// token to the next.
#pragma once

#include "ramnet_device.hpp"
#include "ramnet_kernels.hpp"

#include <type_traits>

namespace ramnet {

constexpr int kChunk = kScanChunk;

struct ScanGeom {
    int n_units;  // B * H * n_slices
    int n_slices; // ceil(C / CS)
    int n_chunks; // T_pad / kChunk (even)
    int t_pad;    // T rounded up to kScanPad
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
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (EPP >= 2) v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    if constexpr (EPP >= 4) v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    if constexpr (EPP >= 8) v += dpp_f<0x141>(v);  // row_half_mirror
    if constexpr (EPP >= 16) v += dpp_f<0x140>(v); // row_mirror
    if constexpr (EPP >= 32) v += __shfl_xor(v, 16);
    if constexpr (EPP >= 64) v += __shfl_xor(v, 32);
    return v;
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
constexpr int scan_row_stride(int vec, int cs) { return cs + (vec == 1 ? 1 : vec); }
// Per-wave mass block: two dummy masses, A masses, then one sink float per
// lane that takes the mass stores of lanes that do not own the event.
constexpr int scan_mass_stride(int A) { return A + 2 + kWave; }

// LDS bytes of a workgroup with NW waves of lane layout (vec, epp).
inline size_t scan_lds_bytes(int A, int vec, int epp, int nw) {
    const int cs = nw * (kWave / epp) * vec;
    return (static_cast<size_t>(A + 2) * scan_row_stride(vec, cs) + static_cast<size_t>(nw) * scan_mass_stride(A)) * 4;
}

// NW waves share one (b, h, CS-channel slice) unit: wave w owns channels
// [w * CSW, (w + 1) * CSW) of the slice and walks the whole sequence on its
// own (no barriers in the token loop), with its own copy of the slot masses.
// FAST: C is a multiple of CS, so every lane owns VEC real channels.
template<typename Scalar, int VEC, int EPP, int NP, int NW, bool MA, bool FAST>
__global__ __launch_bounds__(kWave * NW) void segment_scan_kernel(const SegmentJob job, const ScanGeom geo) {
    constexpr int LPE = kWave / EPP;
    constexpr int CSW = LPE * VEC;
    constexpr int CS = NW * CSW;
    constexpr int RS = scan_row_stride(VEC, CS);
    extern __shared__ __align__(16) float lds[];
    // Workgroups are dealt round-robin to the 8 XCDs; give each XCD a
    // contiguous run of units so the slices of one (b, h) share an L2.
    const int per_xcd = (geo.n_units + 7) / 8;
    const int unit = static_cast<int>(blockIdx.x % 8) * per_xcd + static_cast<int>(blockIdx.x / 8);
    if (unit >= geo.n_units)
        return;
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    const int lane = static_cast<int>(threadIdx.x) % kWave;
    const int bh = unit / geo.n_slices;
    const int c0 = (unit - bh * geo.n_slices) * CS;
    const int T = job.T, A = job.A, C = job.C, Kw = job.Kw, Kr = job.Kr, Tp = geo.t_pad;
    const int MSW = scan_mass_stride(A);
    const float eps = job.eps;

    // LDS: [dummy write row][dummy read row][A rows] x RS floats, then NW
    // mass blocks. st points at slot 0; ms at this wave's mass of slot 0.
    float *st = lds + 2 * RS;
    float *ms = lds + (A + 2) * RS + wave * MSW + 2;

    const int ev = lane % EPP;                // event slot within a pass
    const int cg = lane / EPP;                // channel group within the wave
    const int cl = wave * CSW + cg * VEC;     // first channel of this lane within the slice
    const int sink = A + lane;                // mass sink of this lane

    // ---- state slice -> LDS (whole workgroup), masses per wave
    {
        const float *src = job.init_slot + static_cast<int64_t>(bh) * A * C;
        for (int i = threadIdx.x; i < A * CS; i += kWave * NW) {
            const int a = i / CS, c = i - a * CS;
            const bool ok = c0 + c < C;
            const float v = src[static_cast<int64_t>(a) * C + (ok ? c0 + c : 0)];
            st[a * RS + c] = ok ? v : 0.f;
        }
        for (int i = threadIdx.x; i < 2 * RS; i += kWave * NW)
            lds[i] = 0.f;
        const float *msrc = job.init_mass + static_cast<int64_t>(bh) * A;
        for (int a = lane; a < A; a += kWave)
            ms[a] = msrc[a];
        if (lane < 2)
            ms[lane - 2] = 1.f;
    }
    __syncthreads();

    // per-lane record rows; lanes beyond top-K read the no-op chunk
    const WriteRec *wbase[NP];
    const ReadRec *rbase[NP];
    bool wreal[NP], rreal[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        const int e = p * EPP + ev;
        wreal[p] = e < Kw;
        rreal[p] = e < Kr;
        wbase[p] = job.wrec + (static_cast<int64_t>(bh) * Kw + (wreal[p] ? e : 0)) * Tp;
        rbase[p] = job.rrec + (static_cast<int64_t>(bh) * Kr + (rreal[p] ? e : 0)) * Tp;
    }
    const Scalar *gx = static_cast<const Scalar *>(job.x) + static_cast<int64_t>(bh) * T * C;
    Scalar *gy = static_cast<Scalar *>(job.y) + static_cast<int64_t>(bh) * T * C;
    const int xc = FAST ? c0 + cl : (c0 + cl < C ? c0 + cl : 0);  // clamped first channel

    struct Raw {
        int4 w[NP][kChunk];
        int2 r[NP][kChunk];
        XBits<Scalar, VEC> x[kChunk];
    };
    // Lanes beyond top-K read the no-op chunk at the end of the workspace;
    // both candidates derive from kernel arguments, so the loads stay global.
    auto load = [&](int t0, Raw &raw) {
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            const WriteRec *wp = wreal[p] ? wbase[p] + t0 : job.noop_w;
            const ReadRec *rp = rreal[p] ? rbase[p] + t0 : job.noop_r;
#pragma unroll
            for (int j = 0; j < kChunk; ++j) {
                raw.w[p][j] = *reinterpret_cast<const int4 *>(wp + j);
                raw.r[p][j] = *reinterpret_cast<const int2 *>(rp + j);
            }
        }
#pragma unroll
        for (int j = 0; j < kChunk; ++j) {
            const int t = t0 + j < T ? t0 + j : T - 1;
            raw.x[j] = load_x_bits<Scalar, VEC, FAST>(gx + static_cast<int64_t>(t) * C, FAST ? xc : c0 + cl, C);
        }
    };

    // One chunk of tokens. The body is one basic block when FAST and not
    // TAIL: the mass store of lanes that do not own the event goes to their
    // sink, and all EPP lanes of a channel group store the (bitwise equal)
    // read sum to the same y elements, so no store is predicated and the
    // scheduler can overlap one token's read phase with the next token's
    // write phase.
    auto scan_chunk = [&](const Raw &cur, int t0, auto tail_tag) {
        constexpr bool TAIL = decltype(tail_tag)::value;
#pragma unroll
        for (int j = 0; j < kChunk; ++j) {
            const FVec<VEC> xj = x_bits_to_f<Scalar, VEC>(cur.x[j]);
            // writes: read-modify-write of the slot rows and masses
            float m[NP];
            FVec<VEC> s[NP];
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                const int a = cur.w[p][j].x;
                m[p] = ms[a];
                s[p] = lds_load<VEC>(st + a * RS + cl);
            }
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                const int a = cur.w[p][j].x;
                const float w = __int_as_float(cur.w[p][j].y);
                const float al = __int_as_float(cur.w[p][j].z);
                const float m2 = fmaf(al, m[p], w);
                const float g = scan_gain(w, m2 + eps);
                FVec<VEC> o;
#pragma unroll
                for (int v = 0; v < VEC; ++v)
                    o.v[v] = fmaf(g, xj.v[v] - s[p].v[v], s[p].v[v]);
                lds_store<VEC>(st + a * RS + cl, o);
                ms[cg == 0 ? a : sink] = m2;
            }
            // reads of the post-write state
            FVec<VEC> acc;
#pragma unroll
            for (int v = 0; v < VEC; ++v)
                acc.v[v] = 0.f;
            float sr = 0.f, srm = 0.f;
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                const int a = cur.r[p][j].x;
                const float r = __int_as_float(cur.r[p][j].y);
                float wgt = r;
                if constexpr (MA) {
                    wgt = r * ms[a];
                    sr += r;
                    srm += wgt;
                }
                const FVec<VEC> rv = lds_load<VEC>(st + a * RS + cl);
#pragma unroll
                for (int v = 0; v < VEC; ++v)
                    acc.v[v] = fmaf(wgt, rv.v[v], acc.v[v]);
            }
#pragma unroll
            for (int v = 0; v < VEC; ++v)
                acc.v[v] = group_sum<EPP>(acc.v[v]);
            if constexpr (MA) {
                sr = group_sum<EPP>(sr);
                srm = group_sum<EPP>(srm);
                const float scale = sr / (srm + eps);
#pragma unroll
                for (int v = 0; v < VEC; ++v)
                    acc.v[v] *= scale;
            }
            const int t = t0 + j;
            Scalar *yp = gy + static_cast<int64_t>(t) * C + c0 + cl;
            if constexpr (FAST) {
                if (!TAIL || t < T)
                    store_act_vec<Scalar, VEC>(yp, acc);
            } else if (t < T) {
#pragma unroll
                for (int v = 0; v < VEC; ++v)
                    if (c0 + cl + v < C)
                        store_out(yp + v, acc.v[v]);
            }
        }
    };

    // Two register buffers in alternation: the loads of chunk ci + 1 are in
    // flight while chunk ci runs, with no copy between the buffers. The chunk
    // count is even (T is padded to kScanPad), so every prefetch is issued
    // unconditionally -- a skipped prefetch would make the compiler's wait
    // counts assume the worst at the join. Chunk pairs that lie wholly inside
    // T run the branch-free body; the last pair, if it reaches past T, runs
    // after the loop with guarded stores.
    const int nc = geo.n_chunks;
    const int n_full = (T / kScanPad) * 2;  // chunks of whole pairs inside T
    using Full = std::false_type;
    using Tail = std::true_type;
    if (nc > 0) {
        Raw buf0, buf1;
        load(0, buf0);
        int ci = 0;
        for (; ci < n_full; ci += 2) {
            load((ci + 1) * kChunk, buf1);
            scan_chunk(buf0, ci * kChunk, Full{});
            load((ci + 2 < nc ? ci + 2 : nc - 1) * kChunk, buf0);
            scan_chunk(buf1, (ci + 1) * kChunk, Full{});
        }
        if (ci < nc) {
            load((ci + 1) * kChunk, buf1);
            scan_chunk(buf0, ci * kChunk, Tail{});
            scan_chunk(buf1, (ci + 1) * kChunk, Tail{});
        }
    }
    __syncthreads();

    // ---- LDS -> post state (whole workgroup). Every wave computes identical
    // masses; wave 0 of slice 0 stores them.
    {
        float *dst = job.slot_out + static_cast<int64_t>(bh) * A * C;
        for (int i = threadIdx.x; i < A * CS; i += kWave * NW) {
            const int a = i / CS, c = i - a * CS;
            if (c0 + c < C)
                dst[static_cast<int64_t>(a) * C + c0 + c] = st[a * RS + c];
        }
        if (c0 == 0 && wave == 0) {
            float *mdst = job.mass_out + static_cast<int64_t>(bh) * A;
            for (int a = lane; a < A; a += kWave)
                mdst[a] = ms[a];
        }
    }
}

template<typename Scalar, int VEC, int EPP, int NP, int NW, bool MA, bool FAST>
hipError_t launch_scan(const SegmentJob &job, const ScanGeom &geo, hipStream_t stream) {
    const unsigned blocks = static_cast<unsigned>(((geo.n_units + 7) / 8) * 8);
    hipLaunchKernelGGL((segment_scan_kernel<Scalar, VEC, EPP, NP, NW, MA, FAST>), dim3(blocks), dim3(kWave * NW),
                       scan_lds_bytes(job.A, VEC, EPP, NW), stream, job, geo);
    return hipGetLastError();
}

// Layouts compiled for every activation dtype: (VEC, EPP, NP, NW).
#define RAMNET_SCAN_LAYOUTS(X)                                                                       \
    X(1, 4, 1, 1) X(1, 8, 1, 1) X(1, 16, 1, 1) X(1, 32, 1, 1) X(1, 64, 1, 1) X(1, 64, 2, 1)         \
    X(1, 8, 1, 2) X(1, 8, 1, 4) X(1, 8, 2, 1) X(1, 8, 2, 2) X(1, 8, 2, 4) X(1, 16, 1, 2) X(1, 16, 1, 4) \
    X(2, 8, 1, 1) X(2, 8, 1, 2) X(2, 8, 1, 4) X(2, 16, 1, 1) X(2, 16, 1, 2)                          \
    X(4, 8, 1, 1) X(4, 8, 1, 2) X(4, 16, 1, 1)

template<typename Scalar>
hipError_t scan_dispatch(const SegmentJob &job, const ScanGeom &geo, int vec, int epp, int np, int nw,
                         hipStream_t stream) {
    const int cs = nw * (kWave / epp) * vec;
    const bool fast = job.C % cs == 0;
#define RAMNET_SCAN_CASE(V, E, N, W)                                                                 \
    if (vec == V && epp == E && np == N && nw == W) {                                                \
        if (job.mass_aware)                                                                          \
            return fast ? launch_scan<Scalar, V, E, N, W, true, true>(job, geo, stream)              \
                        : launch_scan<Scalar, V, E, N, W, true, false>(job, geo, stream);            \
        return fast ? launch_scan<Scalar, V, E, N, W, false, true>(job, geo, stream)                 \
                    : launch_scan<Scalar, V, E, N, W, false, false>(job, geo, stream);               \
    }
    RAMNET_SCAN_LAYOUTS(RAMNET_SCAN_CASE)
#undef RAMNET_SCAN_CASE
    return hipErrorInvalidValue;
}

// Whether (vec, epp, np, nw) is one of the compiled layouts.
inline bool scan_layout_compiled(int vec, int epp, int np, int nw) {
#define RAMNET_SCAN_HAS(V, E, N, W) if (vec == V && epp == E && np == N && nw == W) return true;
    RAMNET_SCAN_LAYOUTS(RAMNET_SCAN_HAS)
#undef RAMNET_SCAN_HAS
    return false;
}

// One definition per activation dtype, each in its own translation unit.
hipError_t launch_scan_f32(const SegmentJob &, const ScanGeom &, int, int, int, int, hipStream_t);
hipError_t launch_scan_f16(const SegmentJob &, const ScanGeom &, int, int, int, int, hipStream_t);
hipError_t launch_scan_bf16(const SegmentJob &, const ScanGeom &, int, int, int, int, hipStream_t);

}  // namespace ramnet
