// Segment-parallel prefill: gated sparse update (GSU) + weighted top-K read.
//
// Semantics follow the reference GSU (torch_impl.py:7-75 and
// csrc/ram_attn_segment_parallel.cu:240-416, cuda_utils.cuh:295-308): per
// token t, first every write slot a with weight w > 0 is updated
//     alpha = (1 - w) / (1 - w + e^gamma_t w)
//     m_a  <- alpha m_a + w
//     g    =  w / (m_a + eps)
//     s_a  <- s_a + g (x_t - s_a)
// then y_t = sum_k r_k s_{a_k} over the read slots (post-write state); with
// mass_aware the read weights become (sum r) (m r) / (sum m r + eps).
// Masked tokens neither write nor read and get y_t = 0.
//
// MI355X mapping. The reference walks per-slot event lists after a global
// sort and accumulates y with float atomics. Here one wave owns one
// (b, h, channel-slice) unit and walks the sequence in time order with the
// slice of the slot state (A x CS fp32) and the slot masses (A fp32)
// resident in LDS for the whole call. Channels of the GSU are independent,
// so slicing C gives every unit the complete read sum for its channels:
// no sort, no atomics, deterministic y, and the state crosses HBM exactly
// once in each direction. Token metadata (slot, weight, x slice, gamma,
// mask) is staged chunk by chunk through registers into LDS; the next
// chunk's global loads are in flight while the current chunk is processed.
#include "ramnet_device.hpp"
#include "ramnet_kernels.hpp"

#include <algorithm>

namespace ramnet {

namespace {

constexpr int kMetaPerLane = 16;  // staged (slot, weight) pairs per lane per chunk
constexpr int kXPerLane = 16;     // staged x-slice values per lane per chunk
constexpr int kMaxChunk = 64;     // tokens per chunk (<= one per lane for gamma/mask)

struct SegGeom {
    int n_units, ns, cs, L, n_chunks;
    int st_off, ms_off, ma_off, mv_off, al_off, xs_off, gm_off, mk_off;  // LDS offsets in 4-byte words
};

// 1/d refined by one Newton step; gain = w / (m + eps) to ~1 ulp.
__device__ __forceinline__ float gsu_gain(float w, float d) {
    float r = __builtin_amdgcn_rcpf(d);
    r = fmaf(r, fmaf(-d, r, 1.f), r);
    return w * r;
}

template<typename Scalar, int VEC, bool MASS_AWARE>
__global__ __launch_bounds__(64) void segment_forward_kernel(const SegmentJob job, const SegGeom geo) {
    extern __shared__ float lds[];
    // Workgroups are dealt round-robin to the 8 XCDs; give each XCD a
    // contiguous run of units so the slices of one (b, h) share an L2.
    const int per_xcd = (geo.n_units + 7) / 8;
    const int unit = static_cast<int>(blockIdx.x % 8) * per_xcd + static_cast<int>(blockIdx.x / 8);
    if (unit >= geo.n_units)
        return;
    const int lane = threadIdx.x;
    const int ns = geo.ns, CS = geo.cs, L = geo.L;
    const int bh = unit / ns;
    const int c0 = (unit % ns) * CS;
    const int b = bh / job.H;
    const int T = job.T, A = job.A, C = job.C, Kw = job.Kw, Kr = job.Kr;
    const int Kt = Kw + Kr;
    const float eps = job.eps;

    float *st = lds + geo.st_off;                                // A * CS
    float *ms = lds + geo.ms_off;                                // A
    int *ma = reinterpret_cast<int *>(lds + geo.ma_off);         // L * Kt
    float *mv = lds + geo.mv_off;                                // L * Kt
    float *al = lds + geo.al_off;                                // L * Kw
    float *xs = lds + geo.xs_off;                                // L * CS
    float *gm = lds + geo.gm_off;                                // L
    int *mk = reinterpret_cast<int *>(lds + geo.mk_off);         // L

    // ---- state slice -> LDS
    {
        const float *src = job.init_slot + static_cast<int64_t>(bh) * A * C;
        for (int i = lane; i < A * CS; i += kWave) {
            const int a = i / CS, c = i - a * CS;
            st[i] = c0 + c < C ? src[static_cast<int64_t>(a) * C + c0 + c] : 0.f;
        }
        const float *msrc = job.init_mass + static_cast<int64_t>(bh) * A;
        for (int a = lane; a < A; a += kWave)
            ms[a] = msrc[a];
    }

    const int32_t *gidx = job.addr_idx + static_cast<int64_t>(bh) * Kt * T;
    const float *gval = job.addr_val + static_cast<int64_t>(bh) * Kt * T;
    const Scalar *gx = static_cast<const Scalar *>(job.x) + static_cast<int64_t>(bh) * T * C;
    const Scalar *gg = static_cast<const Scalar *>(job.gamma) + static_cast<int64_t>(bh) * T;
    Scalar *gy = static_cast<Scalar *>(job.y) + static_cast<int64_t>(bh) * T * C;
    const int slot_base = bh * A;

    // ---- chunk staging registers
    int r_idx[kMetaPerLane];
    float r_val[kMetaPerLane];
    float r_x[kXPerLane];
    float r_g = 0.f;
    int r_mk = 0;

    auto load_chunk = [&](int t0) {
#pragma unroll
        for (int q = 0; q < kMetaPerLane; ++q) {
            const int j = lane + q * kWave;
            const int kk = j / L, tt = j - kk * L;
            const bool ok = j < L * Kt && t0 + tt < T;
            const int64_t g = static_cast<int64_t>(kk) * T + t0 + tt;
            r_idx[q] = ok ? gidx[g] : -1;
            r_val[q] = ok ? gval[g] : 0.f;
        }
#pragma unroll
        for (int q = 0; q < kXPerLane; ++q) {
            const int j = lane + q * kWave;
            const int tt = j / CS, c = j - tt * CS;
            const bool ok = j < L * CS && t0 + tt < T && c0 + c < C;
            r_x[q] = ok ? load_f32(gx + static_cast<int64_t>(t0 + tt) * C + c0 + c) : 0.f;
        }
        const bool tok = lane < L && t0 + lane < T;
        r_g = tok ? load_f32(gg + t0 + lane) : 0.f;
        r_mk = tok ? (job.mask ? static_cast<int>(job.mask[static_cast<int64_t>(b) * T + t0 + lane] != 0) : 1) : 0;
    };

    auto store_chunk = [&]() {
#pragma unroll
        for (int q = 0; q < kMetaPerLane; ++q) {
            const int j = lane + q * kWave;
            if (j < L * Kt) {
                const int kk = j / L, tt = j - kk * L;
                const int a = r_idx[q] - slot_base;
                const bool ok = a >= 0 && a < A;
                ma[tt * Kt + kk] = ok ? a : 0;
                // reads are stored negated by the decoder; keep positive weights
                mv[tt * Kt + kk] = ok ? (kk < Kw ? r_val[q] : -r_val[q]) : 0.f;
            }
        }
#pragma unroll
        for (int q = 0; q < kXPerLane; ++q) {
            const int j = lane + q * kWave;
            if (j < L * CS)
                xs[j] = r_x[q];
        }
        if (lane < L) {
            gm[lane] = r_g;
            mk[lane] = r_mk;
        }
    };

    const int LPE = CS / VEC;      // lanes per event
    const int EPP = kWave / LPE;   // events per pass
    const int ev = lane / LPE;     // event slot of this lane within a pass
    const int cg = lane - ev * LPE;
    const int cl = cg * VEC;       // first channel of this lane within the slice

    load_chunk(0);
    for (int ci = 0; ci < geo.n_chunks; ++ci) {
        const int t0 = ci * L;
        __syncthreads();
        store_chunk();
        __syncthreads();
        // forget coefficients of the chunk's write events
        for (int j = lane; j < L * Kw; j += kWave) {
            const int tt = j / Kw, e = j - tt * Kw;
            al[j] = gsu_alpha(mv[tt * Kt + e], gm[tt]);
        }
        __syncthreads();
        if (ci + 1 < geo.n_chunks)
            load_chunk(t0 + L);

        const int n_tok = min(L, T - t0);
        for (int tt = 0; tt < n_tok; ++tt) {
            const int t = t0 + tt;
            Scalar *yrow = gy + static_cast<int64_t>(t) * C + c0 + cl;
            if (!mk[tt]) {
                if (lane < LPE) {
#pragma unroll
                    for (int v = 0; v < VEC; ++v)
                        if (c0 + cl + v < C)
                            store_f32(yrow + v, 0.f);
                }
                continue;
            }
            float xv[VEC];
#pragma unroll
            for (int v = 0; v < VEC; ++v)
                xv[v] = xs[tt * CS + cl + v];
            // writes (distinct slots within a token)
            for (int e0 = 0; e0 < Kw; e0 += EPP) {
                const int e = e0 + ev;
                if (e < Kw) {
                    const float w = mv[tt * Kt + e];
                    if (w != 0.f) {
                        const int a = ma[tt * Kt + e];
                        const float alpha = al[tt * Kw + e];
                        float *row = st + a * CS + cl;
                        const float m2 = fmaf(alpha, ms[a], w);
                        float s[VEC];
#pragma unroll
                        for (int v = 0; v < VEC; ++v)
                            s[v] = row[v];
                        const float g = gsu_gain(w, m2 + eps);
#pragma unroll
                        for (int v = 0; v < VEC; ++v)
                            row[v] = fmaf(g, xv[v] - s[v], s[v]);
                        if (cg == 0)
                            ms[a] = m2;
                    }
                }
            }
            // reads of the post-write state
            float acc[VEC];
#pragma unroll
            for (int v = 0; v < VEC; ++v)
                acc[v] = 0.f;
            float sr = 0.f, srm = 0.f;
            for (int e0 = 0; e0 < Kr; e0 += EPP) {
                const int e = e0 + ev;
                if (e < Kr) {
                    const float r = mv[tt * Kt + Kw + e];
                    if (r != 0.f) {
                        const int a = ma[tt * Kt + Kw + e];
                        const float *row = st + a * CS + cl;
                        float wgt = r;
                        if constexpr (MASS_AWARE) {
                            wgt = r * ms[a];
                            sr += r;
                            srm += wgt;
                        }
#pragma unroll
                        for (int v = 0; v < VEC; ++v)
                            acc[v] = fmaf(wgt, row[v], acc[v]);
                    }
                }
            }
            for (int off = LPE; off < kWave; off <<= 1) {
#pragma unroll
                for (int v = 0; v < VEC; ++v)
                    acc[v] += __shfl_xor(acc[v], off);
                if constexpr (MASS_AWARE) {
                    sr += __shfl_xor(sr, off);
                    srm += __shfl_xor(srm, off);
                }
            }
            if constexpr (MASS_AWARE) {
                const float scale = sr / (srm + eps);
#pragma unroll
                for (int v = 0; v < VEC; ++v)
                    acc[v] *= scale;
            }
            if (lane < LPE) {
#pragma unroll
                for (int v = 0; v < VEC; ++v)
                    if (c0 + cl + v < C)
                        store_f32(yrow + v, acc[v]);
            }
        }
    }
    __syncthreads();

    // ---- LDS -> post state. Every slice of a (b, h) computes identical
    // masses; slice 0 stores them.
    {
        float *dst = job.slot_out + static_cast<int64_t>(bh) * A * C;
        for (int i = lane; i < A * CS; i += kWave) {
            const int a = i / CS, c = i - a * CS;
            if (c0 + c < C)
                dst[static_cast<int64_t>(a) * C + c0 + c] = st[i];
        }
        if (c0 == 0) {
            float *mdst = job.mass_out + static_cast<int64_t>(bh) * A;
            for (int a = lane; a < A; a += kWave)
                mdst[a] = ms[a];
        }
    }
}

int pow2_floor(int x) {
    int p = 1;
    while (p * 2 <= x)
        p <<= 1;
    return p;
}

int pow2_ceil(int x) {
    int p = 1;
    while (p < x)
        p <<= 1;
    return p;
}

// LDS words for a given slice width and chunk length.
int64_t lds_words(int A, int cs, int L, int Kw, int Kr) {
    const int Kt = Kw + Kr;
    return static_cast<int64_t>(A) * cs + A + 2LL * L * Kt + static_cast<int64_t>(L) * Kw + static_cast<int64_t>(L) * cs + 2LL * L;
}

bool make_geom(const SegmentJob &job, SegGeom *g, int *vec) {
    const int Kt = job.Kw + job.Kr;
    const int64_t budget2 = 78 * 1024;   // two units per CU
    const int64_t budget1 = 150 * 1024;  // one unit per CU
    const int cs_max = job.C >= 32 ? 32 : pow2_ceil(job.C);
    for (int pass = 0; pass < 2; ++pass) {
        const int64_t budget = pass == 0 ? budget2 : budget1;
        for (int cs = cs_max; cs >= 1; cs >>= 1) {
            int L = kMaxChunk;
            L = std::min(L, kMetaPerLane * kWave / Kt);
            L = std::min(L, kXPerLane * kWave / cs);
            if (L < 1)
                return false;
            // smaller chunks trade staging for LDS room
            while (L > 8 && lds_words(job.A, cs, L, job.Kw, job.Kr) * 4 > budget)
                L >>= 1;
            if (lds_words(job.A, cs, L, job.Kw, job.Kr) * 4 > budget)
                continue;
            // lanes per event: as many events per pass as top-K needs
            const int kmax = std::max(job.Kw, job.Kr);
            const int epp_want = std::min(kWave, pow2_ceil(std::max(kmax, 1)));
            int v = cs * epp_want / kWave;
            v = std::max(1, std::min(v, 4));
            v = std::min(v, cs);
            g->cs = cs;
            g->L = L;
            g->ns = (job.C + cs - 1) / cs;
            g->n_units = job.B * job.H * g->ns;
            g->n_chunks = (job.T + L - 1) / L;
            int off = 0;
            g->st_off = off; off += job.A * cs;
            g->ms_off = off; off += job.A;
            g->ma_off = off; off += L * Kt;
            g->mv_off = off; off += L * Kt;
            g->al_off = off; off += L * job.Kw;
            g->xs_off = off; off += L * cs;
            g->gm_off = off; off += L;
            g->mk_off = off; off += L;
            *vec = v;
            return true;
        }
    }
    return false;
}

template<typename T, int VEC>
hipError_t launch_vec(const SegmentJob &job, const SegGeom &g, hipStream_t stream) {
    const size_t lds = static_cast<size_t>(lds_words(job.A, g.cs, g.L, job.Kw, job.Kr)) * 4;
    const unsigned blocks = static_cast<unsigned>(((g.n_units + 7) / 8) * 8);
    if (job.mass_aware)
        hipLaunchKernelGGL((segment_forward_kernel<T, VEC, true>), dim3(blocks), dim3(kWave), lds, stream, job, g);
    else
        hipLaunchKernelGGL((segment_forward_kernel<T, VEC, false>), dim3(blocks), dim3(kWave), lds, stream, job, g);
    return hipGetLastError();
}

template<typename T>
hipError_t launch_typed(const SegmentJob &job, const SegGeom &g, int vec, hipStream_t stream) {
    switch (vec) {
        case 1: return launch_vec<T, 1>(job, g, stream);
        case 2: return launch_vec<T, 2>(job, g, stream);
        default: return launch_vec<T, 4>(job, g, stream);
    }
}

}  // namespace

int segment_plan(int A, int C, int Kw, int Kr, int *cs, int *lds_bytes) {
    SegmentJob job{};
    job.A = A;
    job.C = C;
    job.Kw = Kw;
    job.Kr = Kr;
    job.B = job.H = job.T = 1;
    SegGeom g{};
    int vec = 0;
    if (!make_geom(job, &g, &vec))
        return 0;
    if (cs)
        *cs = g.cs;
    if (lds_bytes)
        *lds_bytes = static_cast<int>(lds_words(A, g.cs, g.L, Kw, Kr) * 4);
    return 1;
}

hipError_t launch_segment_forward(const SegmentJob &job, hipStream_t stream, const char **why) {
    if (static_cast<int64_t>(job.B) * job.H == 0)
        return hipSuccess;
    SegGeom g{};
    int vec = 0;
    if (!make_geom(job, &g, &vec)) {
        *why = "segment forward: slot count A too large for the LDS-resident state (needs A*2*4 bytes + staging <= 150 KiB)";
        return hipErrorInvalidValue;
    }
    if (job.T == 0) {
        // nothing to scan: post state is the initial state
        g.n_chunks = 0;
    }
    switch (job.dtype) {
        case kF32: return launch_typed<float>(job, g, vec, stream);
        case kF16: return launch_typed<_Float16>(job, g, vec, stream);
        case kBF16: return launch_typed<bf16_t>(job, g, vec, stream);
        default: *why = "segment forward: unsupported dtype"; return hipErrorInvalidValue;
    }
}

}  // namespace ramnet
