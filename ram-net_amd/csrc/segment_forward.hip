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
constexpr int kMaxChunk = 64;     // tokens per chunk (one gamma per lane)

struct SegGeom {
    int n_units, ns, cs, L, n_chunks;
    int lpe, epp;                  // lanes per event, events per pass (lpe * epp = 64)
    int st_off, ms_off, ev_off, al_off, xs_off, gm_off, mk_off;  // LDS offsets in 4-byte words
};

// 1/d refined by one Newton step; gain = w / (m + eps) to ~1 ulp.
__device__ __forceinline__ float gsu_gain(float w, float d) {
    float r = __builtin_amdgcn_rcpf(d);
    r = fmaf(r, fmaf(-d, r, 1.f), r);
    return w * r;
}

template<int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum over the `epp` consecutive lanes of an event group; every lane of the
// group receives the same value. Within a 16-lane row the exchange uses DPP
// (quad permutes, half-row and row mirrors); wider groups add lane shuffles.
__device__ __forceinline__ float group_sum(float v, int epp) {
    if (epp >= 2) v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
    if (epp >= 4) v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
    if (epp >= 8) v += dpp<0x141>(v);  // row_half_mirror
    if (epp >= 16) v += dpp<0x140>(v); // row_mirror
    if (epp >= 32) v += __shfl_xor(v, 16);
    if (epp >= 64) v += __shfl_xor(v, 32);
    return v;
}

// Token loop state of one lane: its write and read events (one per pass)
// and its channels of the token's value.
template<int VEC, int NP>
struct TokenMeta {
    int aw[NP];
    float w[NP];
    float al[NP];
    int ar[NP];
    float r[NP];
    float x[VEC];
};

template<typename Scalar, int VEC, int NP>
__global__ __launch_bounds__(64) void segment_forward_kernel(const SegmentJob job, const SegGeom geo) {
    extern __shared__ float lds[];
    // Workgroups are dealt round-robin to the 8 XCDs; give each XCD a
    // contiguous run of units so the slices of one (b, h) share an L2.
    const int per_xcd = (geo.n_units + 7) / 8;
    const int unit = static_cast<int>(blockIdx.x % 8) * per_xcd + static_cast<int>(blockIdx.x / 8);
    if (unit >= geo.n_units)
        return;
    const int lane = threadIdx.x;
    const int ns = geo.ns, CS = geo.cs, L = geo.L, EPP = geo.epp;
    const int bh = unit / ns;
    const int c0 = (unit % ns) * CS;
    const int b = bh / job.H;
    const int T = job.T, A = job.A, C = job.C, Kw = job.Kw, Kr = job.Kr;
    const int Kt = Kw + Kr;
    const float eps = job.eps;
    const bool mass_aware = job.mass_aware != 0;

    float *st = lds + geo.st_off;                              // A * CS   slot slice
    float *ms = lds + geo.ms_off;                              // A        masses
    int2 *evm = reinterpret_cast<int2 *>(lds + geo.ev_off);    // L * Kt   (slot, weight) per event
    float *al = lds + geo.al_off;                              // L * Kw   forget coefficient per write
    float *xs = lds + geo.xs_off;                              // L * CS   x slice
    float *gm = lds + geo.gm_off;                              // L        gamma
    int *mk = reinterpret_cast<int *>(lds + geo.mk_off);       // L        token valid

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

    // ---- chunk staging registers (next chunk's loads are in flight while
    // the current chunk is processed)
    int r_idx[kMetaPerLane];
    float r_val[kMetaPerLane];
    float r_x[kXPerLane];
    float r_g = 0.f;
    int r_mk = 0;

    // Staging writes masked tokens and out-of-range slots with weight 0,
    // which makes every event of the token a no-op and its read sum 0.
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

    const int ev = lane & (EPP - 1);   // event slot of this lane within a pass
    const int cg = lane / EPP;         // channel group
    const int cl = cg * VEC;           // first channel of this lane within the slice

    auto fetch = [&](int tt, TokenMeta<VEC, NP> &m) {
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            const int e = p * EPP + ev;
            const bool okw = e < Kw, okr = e < Kr;
            const int2 we = evm[tt * Kt + (okw ? e : 0)];
            const int2 re = evm[tt * Kt + Kw + (okr ? e : 0)];
            m.aw[p] = we.x;
            m.w[p] = okw ? __int_as_float(we.y) : 0.f;
            m.al[p] = okw ? al[tt * Kw + e] : 1.f;
            m.ar[p] = re.x;
            m.r[p] = okr ? __int_as_float(re.y) : 0.f;
        }
#pragma unroll
        for (int v = 0; v < VEC; ++v)
            m.x[v] = xs[tt * CS + cl + v];
    };

    // deferred read of the previous token
    bool pend = false;
    int pend_t = 0;
    float prs[NP][VEC], pr[NP], prm[NP];

    auto flush = [&]() {
        float acc[VEC];
#pragma unroll
        for (int v = 0; v < VEC; ++v)
            acc[v] = 0.f;
        float sr = 0.f, srm = 0.f;
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            const float wgt = mass_aware ? pr[p] * prm[p] : pr[p];
            sr += pr[p];
            srm += wgt;
#pragma unroll
            for (int v = 0; v < VEC; ++v)
                acc[v] = fmaf(wgt, prs[p][v], acc[v]);
        }
#pragma unroll
        for (int v = 0; v < VEC; ++v)
            acc[v] = group_sum(acc[v], EPP);
        if (mass_aware) {
            sr = group_sum(sr, EPP);
            srm = group_sum(srm, EPP);
            const float scale = sr / (srm + eps);
#pragma unroll
            for (int v = 0; v < VEC; ++v)
                acc[v] *= scale;
        }
        if (ev == 0) {
            Scalar *yrow = gy + static_cast<int64_t>(pend_t) * C + c0 + cl;
#pragma unroll
            for (int v = 0; v < VEC; ++v)
                if (c0 + cl + v < C)
                    store_f32(yrow + v, acc[v]);
        }
    };

    load_chunk(0);
    for (int ci = 0; ci < geo.n_chunks; ++ci) {
        const int t0 = ci * L;
        __syncthreads();
        // ---- stage the chunk
#pragma unroll
        for (int q = 0; q < kMetaPerLane; ++q) {
            const int j = lane + q * kWave;
            if (j < L * Kt) {
                const int kk = j / L, tt = j - kk * L;
                const int a = r_idx[q] - slot_base;
                const bool ok = a >= 0 && a < A;
                // reads are stored negated by the decoder; keep positive weights
                const float wv = ok ? (kk < Kw ? r_val[q] : -r_val[q]) : 0.f;
                evm[tt * Kt + kk] = make_int2(ok ? a : 0, __float_as_int(wv));
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
        __syncthreads();
        // forget coefficients; masked tokens lose all their events
        for (int j = lane; j < L * Kt; j += kWave) {
            const int tt = j / Kt, e = j - tt * Kt;
            const float g = gm[tt];
            const bool masked = mk[tt] == 0;
            int2 evv = evm[j];
            if (masked)
                evv.y = __float_as_int(0.f);
            if (e < Kw)
                al[tt * Kw + e] = masked ? 1.f : gsu_alpha(__int_as_float(evv.y), g);
            evm[j] = evv;
        }
        __syncthreads();
        if (ci + 1 < geo.n_chunks)
            load_chunk(t0 + L);

        const int n_tok = min(L, T - t0);
        TokenMeta<VEC, NP> cur, nxt;
        fetch(0, cur);
        for (int tt = 0; tt < n_tok; ++tt) {
            // state rows of this token's writes
            float m[NP], s[NP][VEC];
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                m[p] = ms[cur.aw[p]];
                const float *row = st + cur.aw[p] * CS + cl;
#pragma unroll
                for (int v = 0; v < VEC; ++v)
                    s[p][v] = row[v];
            }
            // finish the previous token's read while those loads fly
            if (pend)
                flush();
            if (tt + 1 < n_tok)
                fetch(tt + 1, nxt);
            // gated sparse update of the write slots
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                const float w = cur.w[p];
                const float m2 = fmaf(cur.al[p], m[p], w);
                const float g = gsu_gain(w, m2 + eps);
                if (w != 0.f) {
                    float *row = st + cur.aw[p] * CS + cl;
#pragma unroll
                    for (int v = 0; v < VEC; ++v)
                        row[v] = fmaf(g, cur.x[v] - s[p][v], s[p][v]);
                    if (cg == 0)
                        ms[cur.aw[p]] = m2;
                }
            }
            // read rows of the post-write state (consumed next iteration)
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                const float *row = st + cur.ar[p] * CS + cl;
#pragma unroll
                for (int v = 0; v < VEC; ++v)
                    prs[p][v] = row[v];
                prm[p] = mass_aware ? ms[cur.ar[p]] : 1.f;
                pr[p] = cur.r[p];
            }
            pend = true;
            pend_t = t0 + tt;
            cur = nxt;
        }
    }
    if (pend)
        flush();
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

int pow2_ceil(int x) {
    int p = 1;
    while (p < x)
        p <<= 1;
    return p;
}

// LDS words for a given slice width and chunk length.
int64_t lds_words(int A, int cs, int L, int Kw, int Kr) {
    const int Kt = Kw + Kr;
    return static_cast<int64_t>(A) * cs + A + 2LL * L * Kt + static_cast<int64_t>(L) * Kw +
           static_cast<int64_t>(L) * cs + 2LL * L + 1;
}

// Choose the channel-slice width (LDS-resident state of A x CS fp32 per
// wave, two waves per CU when possible), the chunk length, and the lane
// layout: EPP events per pass x LPE lanes per event, VEC channels per lane.
bool make_geom(const SegmentJob &job, SegGeom *g, int *vec, int *npass) {
    const int Kt = job.Kw + job.Kr;
    const int kmax = std::max(job.Kw, job.Kr);
    const int64_t budget2 = 78 * 1024;   // two units per CU
    const int64_t budget1 = 150 * 1024;  // one unit per CU
    const int cs_max = job.C >= 32 ? 32 : pow2_ceil(job.C);
    for (int pass = 0; pass < 2; ++pass) {
        const int64_t budget = pass == 0 ? budget2 : budget1;
        for (int cs = cs_max; cs >= 1; cs >>= 1) {
            // events per pass: enough for top-K in at most two passes, VEC <= 4
            int epp = std::min(kWave, pow2_ceil(std::max(kmax, 1)));
            int v = std::max(1, cs * epp / kWave);
            if (v > 4)
                continue;  // slice too wide for this K: try a narrower one
            const int lpe = cs / v;
            epp = kWave / lpe;
            const int np = (kmax + epp - 1) / epp;
            if (np > 2)
                continue;
            int L = kMaxChunk;
            L = std::min(L, kMetaPerLane * kWave / Kt);
            L = std::min(L, kXPerLane * kWave / cs);
            if (L < 1)
                return false;
            while (L > 8 && lds_words(job.A, cs, L, job.Kw, job.Kr) * 4 > budget)
                L >>= 1;
            if (lds_words(job.A, cs, L, job.Kw, job.Kr) * 4 > budget)
                continue;
            g->cs = cs;
            g->L = L;
            g->lpe = lpe;
            g->epp = epp;
            g->ns = (job.C + cs - 1) / cs;
            g->n_units = job.B * job.H * g->ns;
            g->n_chunks = (job.T + L - 1) / L;
            int off = 0;
            g->st_off = off; off += job.A * cs;
            g->ms_off = off; off += job.A;
            off = (off + 1) & ~1;  // 8-byte alignment of the event pairs
            g->ev_off = off; off += 2 * L * Kt;
            g->al_off = off; off += L * job.Kw;
            g->xs_off = off; off += L * cs;
            g->gm_off = off; off += L;
            g->mk_off = off; off += L;
            *vec = v;
            *npass = np;
            return true;
        }
    }
    return false;
}

size_t lds_bytes_of(const SegmentJob &job, const SegGeom &g) {
    return static_cast<size_t>(g.mk_off + g.L) * 4;
}

template<typename T, int VEC, int NP>
hipError_t launch_vec(const SegmentJob &job, const SegGeom &g, hipStream_t stream) {
    const unsigned blocks = static_cast<unsigned>(((g.n_units + 7) / 8) * 8);
    hipLaunchKernelGGL((segment_forward_kernel<T, VEC, NP>), dim3(blocks), dim3(kWave), lds_bytes_of(job, g), stream,
                       job, g);
    return hipGetLastError();
}

template<typename T>
hipError_t launch_typed(const SegmentJob &job, const SegGeom &g, int vec, int np, hipStream_t stream) {
    if (np == 1) {
        switch (vec) {
            case 1: return launch_vec<T, 1, 1>(job, g, stream);
            case 2: return launch_vec<T, 2, 1>(job, g, stream);
            default: return launch_vec<T, 4, 1>(job, g, stream);
        }
    }
    switch (vec) {
        case 1: return launch_vec<T, 1, 2>(job, g, stream);
        case 2: return launch_vec<T, 2, 2>(job, g, stream);
        default: return launch_vec<T, 4, 2>(job, g, stream);
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
    int vec = 0, np = 0;
    if (!make_geom(job, &g, &vec, &np))
        return 0;
    if (cs)
        *cs = g.cs;
    if (lds_bytes)
        *lds_bytes = static_cast<int>(lds_bytes_of(job, g));
    return 1;
}

hipError_t launch_segment_forward(const SegmentJob &job, hipStream_t stream, const char **why) {
    if (static_cast<int64_t>(job.B) * job.H == 0)
        return hipSuccess;
    SegGeom g{};
    int vec = 0, np = 0;
    if (!make_geom(job, &g, &vec, &np)) {
        *why = "segment forward: shape outside the LDS-resident scan (needs A*2*4 bytes + staging <= 150 KiB and "
               "top_k <= 128)";
        return hipErrorInvalidValue;
    }
    switch (job.dtype) {
        case kF32: return launch_typed<float>(job, g, vec, np, stream);
        case kF16: return launch_typed<_Float16>(job, g, vec, np, stream);
        case kBF16: return launch_typed<bf16_t>(job, g, vec, np, stream);
        default: *why = "segment forward: unsupported dtype"; return hipErrorInvalidValue;
    }
}

}  // namespace ramnet
