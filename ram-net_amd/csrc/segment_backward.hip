// Segment backward: gradients of the gated sparse update (GSU) and top-K
// read over a whole sequence (reference: csrc/ram_attn_segment_parallel.cu:
// 418-606, the "backward by state reconstruction" of the segment op, and its
// host op ram_attn_ops.cpp:267-310).
//
// Forward, per (b, h) and token t: every write event (slot a, weight w > 0)
//     alpha = (1 - w) / (1 - w + e^gamma w),  m' = alpha m + w,
//     g = w / (m' + eps),                     s_a <- s_a + g (x_t - s_a),
// then y_t = sum_j r_j s_{a_j} with r_j the effective read weights (with
// mass_aware r_j = R m_j rho_j / (Z + eps), R = sum rho, Z = sum m rho, for
// the raw weights rho and the post-write masses m).
//
// Backward, walking time in reverse with Ds = dL/ds and Dm = dL/dm:
//   read j:  Ds_{a_j} += r_j Dy_t,   d_j = <Dy_t, s_{a_j}(t)>;
//            dL/drho_j = d_j, or with mass_aware, for Q = sum_i d_i m_i rho_i / (Z + eps)
//            and c = R / (Z + eps): dL/drho_j = Q + c m_j (d_j - Q),
//            Dm_{a_j} += c rho_j (d_j - Q);
//   write:   Dg = <Ds_a, x_t - s_a(before)>,  Dx_t += g Ds_a,  Ds_a <- (1 - g) Ds_a,
//            Dm_tot = Dm_a - Dg g / (m' + eps),
//            dL/dw = Dg / (m' + eps) + Dm_tot (1 + m dalpha/dw),
//            dL/dgamma_t += Dm_tot m dalpha/dgamma,   Dm_a <- alpha Dm_tot,
// with dalpha/dw = -q / den^2 and dalpha/dgamma = -(1 - w) w q / den^2, where
// q = e^-|gamma| and den = q (1 - w) + w (gamma >= 0) or (1 - w) + q w.
// Events that do not act (masked tokens, zero weights, inactive addresses)
// get zero gradients, as in the reference, which skips them.
//
// MI355X mapping. Given the gains and effective read weights, the channels
// of Ds are independent: the slot-state part runs like the forward scan, one
// wave per (b, h, channel slice) with the slice resident in LDS, and only
// the scalar mass chain needs the full-channel dot products. Passes:
//   1. the forward mass replay (the mass pre-pass in record-keeping mode):
//      per event its slot, gain, masses and effective read weight;
//   2. segment_bwd_scan_kernel, per (b, h, slice): forward over t with s in
//      LDS, saving x - s before every write and the read dot products d_j;
//      then backward over t with Ds in LDS: Dx, the per-slice Dg and
//      dL/d init_slot. The saved rows replace the reference's state roll-back
//      by subtraction, so no slot value is ever reconstructed;
//   3. segment_bwd_sum_kernel: per-slice dot products -> totals (in slice 0),
//      in a fixed order, so the gradients are deterministic;
//   4. segment_bwd_mass_kernel, per (b, h): backward over t with Dm in LDS:
//      dL/dw, dL/drho, dL/dgamma and dL/d init_mass.
#include "ramnet_device.hpp"
#include "ramnet_kernels.hpp"
#include "segment_scan.hpp"

#include <algorithm>

namespace ramnet {

namespace {

constexpr int64_t kBwdLdsLimit = 160 * 1024;
constexpr int kBwdMaxSlices = 16;

int pow2_at_least(int x) {
    int p = 1;
    while (p < x)
        p <<= 1;
    return p;
}

struct BwdPlan {
    int epp, np, vec, csw, n_sub;
    int64_t lds;
};

// Lane layout of the slice kernel: EPP events per pass (NP passes), LPE =
// 64 / EPP lanes per event, VEC channels per lane, CSW = LPE * VEC channels
// per wave. VEC grows until at most 16 slices cover C (bounding the partial
// sums), and shrinks again if the slice does not fit in LDS.
bool bwd_plan(int A, int C, int Kw, int Kr, BwdPlan *p) {
    const int kmax = std::max(Kw, Kr);
    if (kmax > 2 * kWave || A <= 0 || C <= 0)
        return false;
    const int epp = std::min(kWave, std::max(8, pow2_at_least(kmax)));
    const int np = (kmax + epp - 1) / epp;
    const int lpe = kWave / epp;
    int vec = 1;
    while (vec < 4 && static_cast<int64_t>(lpe) * vec * kBwdMaxSlices < C)
        vec *= 2;
    while (vec > 1 && static_cast<int64_t>(A + 2) * lpe * vec * 4 > kBwdLdsLimit)
        vec /= 2;
    const int64_t lds = static_cast<int64_t>(A + 2) * lpe * vec * 4;
    if (lds > kBwdLdsLimit)
        return false;
    *p = {epp, np, vec, lpe * vec, (C + lpe * vec - 1) / (lpe * vec), lds};
    return true;
}

// Sum over the lanes of one event (the LPE lanes with equal lane % EPP).
template<int EPP>
__device__ __forceinline__ float chan_sum(float v) {
#pragma unroll
    for (int o = EPP; o < kWave; o <<= 1)
        v += __shfl_xor(v, o);
    return v;
}

// One token's loads for a lane of the slice kernel.
template<int NP, int VEC, bool FWD>
struct BwdTok {
    int2 w[NP];             // write event {slot, gain bits}
    int2 r[NP];             // read event {slot, effective weight bits}
    float dy[VEC];          // Dy_t on the lane's channels
    float xd[FWD ? VEC : NP * VEC];  // forward: x_t; backward: saved x - s per write pass
};

template<typename Scalar, int EPP, int NP, int VEC>
__global__ __launch_bounds__(kWave) void segment_bwd_scan_kernel(const SegmentBwdJob job, int n_sub) {
    constexpr int LPE = kWave / EPP;
    constexpr int CSW = LPE * VEC;
    constexpr int CH = NP * VEC >= 4 ? 4 : 8;  // tokens per prefetch chunk
    extern __shared__ __align__(16) float st[];  // (A + 2) rows of CSW: rows -2 and -1 are the no-op rows
    const SegmentJob &fj = job.fwd;
    const int A = fj.A, C = fj.C, T = fj.T, Kw = fj.Kw, Kr = fj.Kr;
    const int BH = fj.B * fj.H;
    const int unit = static_cast<int>(blockIdx.x);
    const int bh = unit / n_sub, sub = unit - bh * n_sub;
    const int lane = static_cast<int>(threadIdx.x);
    const int e = lane % EPP, q = lane / EPP;
    const int c0 = sub * CSW + q * VEC;  // first channel of this lane
    float *rows = st + 2 * CSW;
    const Scalar *xs = static_cast<const Scalar *>(fj.x);
    const Scalar *dys = static_cast<const Scalar *>(job.grad_y);

    auto load_tok = [&](int t, auto &k, auto fwd_tag) {
        constexpr bool F = decltype(fwd_tag)::value;
        const int64_t tb = static_cast<int64_t>(bh) * T + t;
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            const int kw = p * EPP + e, kr = p * EPP + e;
            k.w[p] = kw < Kw ? job.aux.wev[tb * Kw + kw] : make_int2(-2, 0);
            k.r[p] = kr < Kr ? job.aux.rev[tb * Kr + kr] : make_int2(-1, 0);
        }
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
            const int c = c0 + v;
            k.dy[v] = c < C ? load_f32(dys + tb * C + c) : 0.f;
            if constexpr (F)
                k.xd[v] = c < C ? load_f32(xs + tb * C + c) : 0.f;
        }
        if constexpr (!F) {
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                const int kw = p * EPP + e;
                const float *src = job.delta + ((static_cast<int64_t>(unit) * T + t) * Kw + (kw < Kw ? kw : 0)) * CSW +
                                   q * VEC;
                const FVec<VEC> d = lds_load<VEC>(src);  // plain vector load (global here)
#pragma unroll
                for (int v = 0; v < VEC; ++v)
                    k.xd[p * VEC + v] = d.v[v];
            }
        }
    };

    // ---- forward over t: s in LDS; save x - s before each write, d_j per read
    for (int i = lane; i < (A + 2) * CSW; i += kWave) {
        const int a = i / CSW - 2, c = sub * CSW + i % CSW;
        st[i] = (a >= 0 && c < C) ? fj.init_slot[(static_cast<int64_t>(bh) * A + a) * C + c] : 0.f;
    }
    __syncthreads();
    {
        using Tok = BwdTok<NP, VEC, true>;
        using Tag = std::true_type;
        Tok cur[CH], nxt[CH];
#pragma unroll
        for (int j = 0; j < CH; ++j)
            load_tok(min(j, T - 1), cur[j], Tag{});
        const int nck = (T + CH - 1) / CH;
        for (int ci = 0; ci < nck; ++ci) {
#pragma unroll
            for (int j = 0; j < CH; ++j)
                load_tok(min((ci + 1) * CH + j, T - 1), nxt[j], Tag{});
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                const int t = ci * CH + j;
                if (t >= T)
                    break;
                const Tok &k = cur[j];
#pragma unroll
                for (int p = 0; p < NP; ++p) {
                    const int kw = p * EPP + e;
                    const float g = __int_as_float(k.w[p].y);
                    float *row = rows + k.w[p].x * CSW + q * VEC;
                    FVec<VEC> s = lds_load<VEC>(row);
                    FVec<VEC> d;
#pragma unroll
                    for (int v = 0; v < VEC; ++v) {
                        d.v[v] = k.xd[v] - s.v[v];
                        s.v[v] = fmaf(g, d.v[v], s.v[v]);
                    }
                    lds_store<VEC>(row, s);
                    if (kw < Kw)
                        lds_store<VEC>(job.delta + ((static_cast<int64_t>(unit) * T + t) * Kw + kw) * CSW + q * VEC, d);
                }
#pragma unroll
                for (int p = 0; p < NP; ++p) {
                    const int kr = p * EPP + e;
                    const FVec<VEC> s = lds_load<VEC>(rows + k.r[p].x * CSW + q * VEC);
                    float part = 0.f;
#pragma unroll
                    for (int v = 0; v < VEC; ++v)
                        part = fmaf(s.v[v], k.dy[v], part);
                    part = chan_sum<EPP>(part);
                    if (kr < Kr && q == 0)
                        job.dr_part[((static_cast<int64_t>(sub) * BH + bh) * T + t) * Kr + kr] = part;
                }
            }
#pragma unroll
            for (int j = 0; j < CH; ++j)
                cur[j] = nxt[j];
        }
    }
    __syncthreads();

    // ---- backward over t: Ds in LDS
    for (int i = lane; i < (A + 2) * CSW; i += kWave) {
        const int a = i / CSW - 2, c = sub * CSW + i % CSW;
        st[i] = (a >= 0 && c < C && job.grad_slot) ? job.grad_slot[(static_cast<int64_t>(bh) * A + a) * C + c] : 0.f;
    }
    __syncthreads();
    {
        using Tok = BwdTok<NP, VEC, false>;
        using Tag = std::false_type;
        Tok cur[CH], nxt[CH];
#pragma unroll
        for (int j = 0; j < CH; ++j)
            load_tok(max(T - 1 - j, 0), cur[j], Tag{});
        const int nck = (T + CH - 1) / CH;
        for (int ci = 0; ci < nck; ++ci) {
#pragma unroll
            for (int j = 0; j < CH; ++j)
                load_tok(max(T - 1 - (ci + 1) * CH - j, 0), nxt[j], Tag{});
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                const int t = T - 1 - ci * CH - j;
                if (t < 0)
                    break;
                const Tok &k = cur[j];
#pragma unroll
                for (int p = 0; p < NP; ++p) {
                    const float r = __int_as_float(k.r[p].y);
                    float *row = rows + k.r[p].x * CSW + q * VEC;
                    FVec<VEC> D = lds_load<VEC>(row);
#pragma unroll
                    for (int v = 0; v < VEC; ++v)
                        D.v[v] = fmaf(r, k.dy[v], D.v[v]);
                    lds_store<VEC>(row, D);
                }
                float dx[VEC];
#pragma unroll
                for (int v = 0; v < VEC; ++v)
                    dx[v] = 0.f;
#pragma unroll
                for (int p = 0; p < NP; ++p) {
                    const int kw = p * EPP + e;
                    const float g = __int_as_float(k.w[p].y);
                    float *row = rows + k.w[p].x * CSW + q * VEC;
                    FVec<VEC> D = lds_load<VEC>(row);
                    float part = 0.f;
#pragma unroll
                    for (int v = 0; v < VEC; ++v) {
                        part = fmaf(D.v[v], k.xd[p * VEC + v], part);
                        dx[v] = fmaf(g, D.v[v], dx[v]);
                        D.v[v] = fmaf(-g, D.v[v], D.v[v]);
                    }
                    lds_store<VEC>(row, D);
                    part = chan_sum<EPP>(part);
                    if (kw < Kw && q == 0)
                        job.dg_part[((static_cast<int64_t>(sub) * BH + bh) * T + t) * Kw + kw] = part;
                }
                const int64_t tb = static_cast<int64_t>(bh) * T + t;
#pragma unroll
                for (int v = 0; v < VEC; ++v) {
                    const float s = event_sum<EPP>(dx[v]);
                    if (e == 0 && c0 + v < C)
                        job.grad_x[tb * C + c0 + v] = s;
                }
            }
#pragma unroll
            for (int j = 0; j < CH; ++j)
                cur[j] = nxt[j];
        }
    }
    __syncthreads();
    for (int i = lane; i < A * CSW; i += kWave) {
        const int a = i / CSW, c = sub * CSW + i % CSW;
        if (c < C)
            job.grad_init_slot[(static_cast<int64_t>(bh) * A + a) * C + c] = rows[i];
    }
}

// Per-slice partial sums -> totals in slice 0, summed in slice order.
__global__ __launch_bounds__(256) void segment_bwd_sum_kernel(float *part, int n_sub, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n)
        return;
    float s = part[i];
    for (int k = 1; k < n_sub; ++k)
        s += part[static_cast<int64_t>(k) * n + i];
    part[i] = s;
}

// One token's loads for a lane of the mass kernel: lanes 0..31 take write
// events p * 32 + lane, lanes 32..63 read events p * 32 + lane - 32.
template<int MP>
struct MassTok {
    int2 ev[MP];   // {slot, gain or effective weight}
    float m[MP];   // write: mass before; read: post-write mass
    float v[MP];   // write: w; read: raw weight rho (positive)
    float dd[MP];  // write: Dg; read: d_j
    float gam;
};

template<typename Scalar, bool MA, int MP>
__global__ __launch_bounds__(kWave) void segment_bwd_mass_kernel(const SegmentBwdJob job) {
    constexpr int CH = MP == 1 ? 8 : MP == 2 ? 4 : 2;
    extern __shared__ __align__(16) float lds[];
    const SegmentJob &fj = job.fwd;
    const int A = fj.A, T = fj.T, Kw = fj.Kw, Kr = fj.Kr, Kt = Kw + Kr;
    const float eps = fj.eps;
    const int bh = static_cast<int>(blockIdx.x);
    const int lane = static_cast<int>(threadIdx.x);
    const int hl = lane & 31;
    const bool wlane = lane < 32;
    float *dm = lds + 2;  // dm[-2], dm[-1]: the no-op slots
    for (int a = lane; a < A; a += kWave)
        dm[a] = job.grad_mass ? job.grad_mass[static_cast<int64_t>(bh) * A + a] : 0.f;
    if (lane < 2)
        lds[lane] = 0.f;
    __syncthreads();
    const Scalar *gs = static_cast<const Scalar *>(job.gamma) + static_cast<int64_t>(bh) * T;
    const float *val = job.addr_val + static_cast<int64_t>(bh) * Kt * T;
    float *gval = job.grad_val + static_cast<int64_t>(bh) * Kt * T;

    auto load_tok = [&](int t, MassTok<MP> &k) {
        const int64_t tb = static_cast<int64_t>(bh) * T + t;
#pragma unroll
        for (int p = 0; p < MP; ++p) {
            const int ev = p * 32 + hl;
            const bool on = wlane ? ev < Kw : ev < Kr;
            const int ec = on ? ev : 0;
            if (wlane) {
                k.ev[p] = on ? job.aux.wev[tb * Kw + ec] : make_int2(-2, 0);
                k.m[p] = job.aux.wm[tb * Kw + ec];
                k.v[p] = val[static_cast<int64_t>(ec) * T + t];
                k.dd[p] = job.dg_part[tb * Kw + ec];
            } else {
                k.ev[p] = on ? job.aux.rev[tb * Kr + ec] : make_int2(-1, 0);
                k.m[p] = MA ? job.aux.rm[tb * Kr + ec] : 0.f;
                k.v[p] = -val[static_cast<int64_t>(Kw + ec) * T + t];
                k.dd[p] = job.dr_part[tb * Kr + ec];
            }
        }
        k.gam = load_f32(gs + t);
    };

    MassTok<MP> cur[CH], nxt[CH];
#pragma unroll
    for (int j = 0; j < CH; ++j)
        load_tok(max(T - 1 - j, 0), cur[j]);
    const int nck = (T + CH - 1) / CH;
    for (int ci = 0; ci < nck; ++ci) {
#pragma unroll
        for (int j = 0; j < CH; ++j)
            load_tok(max(T - 1 - (ci + 1) * CH - j, 0), nxt[j]);
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            const int t = T - 1 - ci * CH - j;
            if (t < 0)
                break;
            const MassTok<MP> &k = cur[j];
            // reads of token t (they follow its writes in the forward)
            float dr[MP];
            if constexpr (MA) {
                float sr = 0.f, srm = 0.f, sdm = 0.f;
#pragma unroll
                for (int p = 0; p < MP; ++p) {
                    const bool act = !wlane && k.ev[p].x >= 0;
                    const float rho = act ? k.v[p] : 0.f;
                    sr += rho;
                    srm = fmaf(rho, k.m[p], srm);
                    sdm = fmaf(rho * k.m[p], act ? k.dd[p] : 0.f, sdm);
                }
                sr = event_sum<32>(sr);
                srm = event_sum<32>(srm);
                sdm = event_sum<32>(sdm);
                const float inv = 1.f / (srm + eps);
                const float c = sr * inv, Q = sdm * inv;
#pragma unroll
                for (int p = 0; p < MP; ++p) {
                    const bool act = !wlane && k.ev[p].x >= 0;
                    const float diff = k.dd[p] - Q;
                    dr[p] = act ? fmaf(c * k.m[p], diff, Q) : 0.f;
                    if (act)
                        dm[k.ev[p].x] += c * k.v[p] * diff;
                }
            } else {
#pragma unroll
                for (int p = 0; p < MP; ++p)
                    dr[p] = (!wlane && k.ev[p].x >= 0) ? k.dd[p] : 0.f;
            }
            __syncthreads();
            // writes of token t
            float dgam = 0.f;
            float dw[MP];
#pragma unroll
            for (int p = 0; p < MP; ++p) {
                dw[p] = 0.f;
                const bool act = wlane && k.ev[p].x >= 0;
                if (act) {
                    const float w = k.v[p], m = k.m[p], gm = k.gam, Dg = k.dd[p];
                    const float g = __int_as_float(k.ev[p].y);
                    const float al = gsu_alpha(w, gm);
                    const float den = fmaf(al, m, w) + eps;
                    const int a = k.ev[p].x;
                    const float dtot = dm[a] - Dg * g / den;
                    const float qd = expf(-fabsf(gm));
                    const float cw = 1.f - w;
                    const float dn = gm >= 0.f ? fmaf(qd, cw, w) : fmaf(qd, w, cw);
                    const float t2 = qd / (dn * dn);
                    dw[p] = Dg / den + dtot * fmaf(-m, t2, 1.f);
                    dgam = fmaf(-dtot * m, cw * w * t2, dgam);
                    dm[a] = dtot * al;
                }
            }
            dgam = event_sum<32>(dgam);
            if (lane == 0)
                job.grad_gamma[static_cast<int64_t>(bh) * T + t] = dgam;
#pragma unroll
            for (int p = 0; p < MP; ++p) {
                const int ev = p * 32 + hl;
                if (wlane && ev < Kw)
                    gval[static_cast<int64_t>(ev) * T + t] = dw[p];
                if (!wlane && ev < Kr)
                    gval[static_cast<int64_t>(Kw + ev) * T + t] = dr[p];
            }
            __syncthreads();
        }
#pragma unroll
        for (int j = 0; j < CH; ++j)
            cur[j] = nxt[j];
    }
    for (int a = lane; a < A; a += kWave)
        job.grad_init_mass[static_cast<int64_t>(bh) * A + a] = dm[a];
}

template<typename Scalar, int EPP, int NP>
hipError_t launch_bwd_scan_vec(const SegmentBwdJob &job, const BwdPlan &p, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(job.fwd.B * job.fwd.H * p.n_sub));
    const size_t lds = static_cast<size_t>(p.lds);
    switch (p.vec) {
        case 1: hipLaunchKernelGGL((segment_bwd_scan_kernel<Scalar, EPP, NP, 1>), grid, dim3(kWave), lds, stream, job, p.n_sub); break;
        case 2: hipLaunchKernelGGL((segment_bwd_scan_kernel<Scalar, EPP, NP, 2>), grid, dim3(kWave), lds, stream, job, p.n_sub); break;
        default: hipLaunchKernelGGL((segment_bwd_scan_kernel<Scalar, EPP, NP, 4>), grid, dim3(kWave), lds, stream, job, p.n_sub); break;
    }
    return hipGetLastError();
}

template<typename Scalar>
hipError_t launch_bwd_scan(const SegmentBwdJob &job, const BwdPlan &p, hipStream_t stream) {
    switch (p.epp) {
        case 8: return launch_bwd_scan_vec<Scalar, 8, 1>(job, p, stream);
        case 16: return launch_bwd_scan_vec<Scalar, 16, 1>(job, p, stream);
        case 32: return launch_bwd_scan_vec<Scalar, 32, 1>(job, p, stream);
        default:
            return p.np == 1 ? launch_bwd_scan_vec<Scalar, 64, 1>(job, p, stream)
                             : launch_bwd_scan_vec<Scalar, 64, 2>(job, p, stream);
    }
}

template<typename Scalar, bool MA>
hipError_t launch_bwd_mass(const SegmentBwdJob &job, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(job.fwd.B * job.fwd.H));
    const size_t lds = static_cast<size_t>(job.fwd.A + 2) * 4;
    const int kmax = std::max(job.fwd.Kw, job.fwd.Kr);
    if (kmax <= 32)
        hipLaunchKernelGGL((segment_bwd_mass_kernel<Scalar, MA, 1>), grid, dim3(kWave), lds, stream, job);
    else if (kmax <= 64)
        hipLaunchKernelGGL((segment_bwd_mass_kernel<Scalar, MA, 2>), grid, dim3(kWave), lds, stream, job);
    else
        hipLaunchKernelGGL((segment_bwd_mass_kernel<Scalar, MA, 4>), grid, dim3(kWave), lds, stream, job);
    return hipGetLastError();
}

template<typename Scalar>
hipError_t launch_typed(const SegmentBwdJob &job, const BwdPlan &p, hipStream_t stream) {
    hipError_t err = launch_bwd_scan<Scalar>(job, p, stream);
    if (err != hipSuccess)
        return err;
    const SegmentJob &fj = job.fwd;
    const int64_t nw = static_cast<int64_t>(fj.B) * fj.H * fj.T * fj.Kw;
    const int64_t nr = static_cast<int64_t>(fj.B) * fj.H * fj.T * fj.Kr;
    if (p.n_sub > 1) {
        hipLaunchKernelGGL(segment_bwd_sum_kernel, dim3(static_cast<unsigned>((nw + 255) / 256)), dim3(256), 0, stream,
                           job.dg_part, p.n_sub, nw);
        hipLaunchKernelGGL(segment_bwd_sum_kernel, dim3(static_cast<unsigned>((nr + 255) / 256)), dim3(256), 0, stream,
                           job.dr_part, p.n_sub, nr);
        if ((err = hipGetLastError()) != hipSuccess)
            return err;
    }
    return fj.mass_aware ? launch_bwd_mass<Scalar, true>(job, stream) : launch_bwd_mass<Scalar, false>(job, stream);
}

// dst = src, or 0 when src is null (a kernel, not a memset, so that callers
// may capture the call in a graph).
__global__ __launch_bounds__(256) void copy_or_zero_kernel(float *dst, const float *src, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n)
        dst[i] = src ? src[i] : 0.f;
}

int64_t align256(int64_t n) { return (n + 255) / 256 * 256; }

}  // namespace

int64_t segment_backward_layout(int B, int H, int T, int A, int C, int Kw, int Kr, char *base, SegmentBwdJob *job) {
    BwdPlan p{};
    if (!bwd_plan(A, C, Kw, Kr, &p))
        return -1;
    const int64_t bh = static_cast<int64_t>(B) * H;
    const int64_t nw = bh * T * Kw, nr = bh * T * Kr;
    int64_t off = 0;
    auto take = [&](int64_t bytes) {
        char *ptr = base ? base + off : nullptr;
        off += align256(bytes);
        return ptr;
    };
    char *wev = take(nw * 8), *wm = take(nw * 4), *rev = take(nr * 8), *rm = take(nr * 4);
    char *mass = take(bh * A * 4);
    const int64_t maps_bytes = mass_replay_scratch_bytes(B, H, T, A);
    char *maps = take(maps_bytes);
    char *delta = take(bh * p.n_sub * T * Kw * p.csw * 4);
    char *dr = take(p.n_sub * nr * 4), *dg = take(p.n_sub * nw * 4);
    if (job) {
        job->aux = MassAux{reinterpret_cast<int2 *>(wev), reinterpret_cast<float *>(wm), reinterpret_cast<int2 *>(rev),
                           reinterpret_cast<float *>(rm)};
        job->mass_scratch = reinterpret_cast<float *>(mass);
        job->maps = maps;
        job->maps_bytes = static_cast<size_t>(maps_bytes);
        job->delta = reinterpret_cast<float *>(delta);
        job->dr_part = reinterpret_cast<float *>(dr);
        job->dg_part = reinterpret_cast<float *>(dg);
    }
    return off;
}

hipError_t launch_segment_backward(const SegmentBwdJob &job, hipStream_t stream, const char **why) {
    const SegmentJob &fj = job.fwd;
    if (static_cast<int64_t>(fj.B) * fj.H == 0)
        return hipSuccess;
    BwdPlan p{};
    if (!bwd_plan(fj.A, fj.C, fj.Kw, fj.Kr, &p)) {
        *why = "segment backward: shape outside the LDS-resident scan (top_k <= 128 and (A + 2) * 4 * slice "
               "channels <= 160 KiB)";
        return hipErrorInvalidValue;
    }
    if (fj.T == 0) {
        // no events: the gradients of the initial state are those of the final state
        const int64_t ns = static_cast<int64_t>(fj.B) * fj.H * fj.A;
        hipLaunchKernelGGL(copy_or_zero_kernel, dim3(static_cast<unsigned>((ns * fj.C + 255) / 256)), dim3(256), 0,
                           stream, job.grad_init_slot, job.grad_slot, ns * fj.C);
        hipLaunchKernelGGL(copy_or_zero_kernel, dim3(static_cast<unsigned>((ns + 255) / 256)), dim3(256), 0, stream,
                           job.grad_init_mass, job.grad_mass, ns);
        return hipGetLastError();
    }
    SegmentJob mj = fj;
    mj.mass_out = job.mass_scratch;
    hipError_t err = launch_mass_replay(mj, job.aux, job.maps, job.maps_bytes, stream);
    if (err != hipSuccess)
        return err;
    switch (fj.dtype) {
        case kF32: return launch_typed<float>(job, p, stream);
        case kF16: return launch_typed<_Float16>(job, p, stream);
        case kBF16: return launch_typed<bf16_t>(job, p, stream);
        default: *why = "segment backward: unsupported dtype"; return hipErrorInvalidValue;
    }
}

}  // namespace ramnet
