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
//   3. segment_bwd_sum_kernel: per-slice dot products -> totals, summed in
//      slice order, so the gradients are deterministic;
//   4. segment_bwd_mass_kernel, per (b, h, time chunk): the Dm chain is
//      affine in Dm, so it runs as chunk maps, a scan over chunks
//      (segment_bwd_mass_scan_kernel) and chunk replays that write dL/dw,
//      dL/drho and dL/dgamma; the scan gives dL/d init_mass.
#include "ramnet_device.hpp"
#include "ramnet_kernels.hpp"
#include "ramnet_search.hpp"
#include "segment_scan.hpp"

#include <algorithm>

namespace ramnet {

namespace {

constexpr int64_t kBwdLdsLimit = 160 * 1024;
constexpr int kBwdMaxSlices = 16;
// The Dm chain keeps one float per slot in LDS ((A + 2) * 4 bytes); the
// forward mass replay runs in slot ranges where its tag tables do not fit.
constexpr int64_t kBwdMaxMassSlots = kBwdLdsLimit / 4 - 2;

int pow2_at_least(int x) {
    int p = 1;
    while (p < x)
        p <<= 1;
    return p;
}

struct BwdPlan {
    int epp, np, vec, csw, n_sub;
    int64_t lds;  // dynamic LDS (the slot rows); the chunk stage is static
};

// Tokens per staged chunk of the slice kernel, and the stage's LDS bytes:
// write records (16 B) and read records (8 B) per event slot, x and Dy per
// channel, per token.
__host__ __device__ constexpr int bwd_chunk(int epp, int np, int vec) { return epp * np >= 64 || np * vec >= 2 ? 8 : 16; }
constexpr int64_t bwd_stage_bytes(int epp, int np, int vec) {
    return static_cast<int64_t>(bwd_chunk(epp, np, vec)) * (epp * np * (16 + 8) + 2 * (kWave / epp) * vec * 4);
}

// Lane layout of the slice kernel: EPP events per pass (NP passes), LPE =
// 64 / EPP lanes per event, VEC channels per lane, CSW = LPE * VEC channels
// per wave. VEC grows until at most 16 slices cover C (bounding the partial
// sums), and shrinks again if the slice does not fit in LDS; wide slot spaces
// then take more event lanes per pass (fewer channels per wave).
bool bwd_plan(int A, int C, int Kw, int Kr, BwdPlan *p) {
    const int kmax = std::max(Kw, Kr);
    // the Dm chain keeps one float per slot in LDS
    if (kmax > 2 * kWave || A <= 0 || C <= 0 || A > kBwdMaxMassSlots)
        return false;
    for (int epp = std::min(kWave, std::max(8, pow2_at_least(kmax))); epp <= kWave; epp *= 2) {
        const int np = (kmax + epp - 1) / epp;
        const int lpe = kWave / epp;
        auto total = [&](int v) { return static_cast<int64_t>(A + 2) * lpe * v * 4 + bwd_stage_bytes(epp, np, v); };
        int vec = 1;
        while (vec < 4 && static_cast<int64_t>(lpe) * vec * kBwdMaxSlices < C)
            vec *= 2;
        while (vec > 1 && total(vec) > kBwdLdsLimit)
            vec /= 2;
        if (total(vec) > kBwdLdsLimit)
            continue;
        *p = {epp, np, vec, lpe * vec, (C + lpe * vec - 1) / (lpe * vec), static_cast<int64_t>(A + 2) * lpe * vec * 4};
        return true;
    }
    return false;
}

// 1 / d as v_rcp_f32 refined by one Newton step.
__device__ __forceinline__ float recip_nr(float d) {
    const float r = __builtin_amdgcn_rcpf(d);
    return fmaf(r, fmaf(-d, r, 1.f), r);
}

// v where the mask is all ones, +0 where it is zero (also for a v that is
// not finite); an integer AND, which the compiler does not turn into a branch
__device__ __forceinline__ float keep_if(float v, uint32_t mask) {
    return __uint_as_float(__float_as_uint(v) & mask);
}

// Sum over the lanes whose indices differ only in bits LO .. HI/2 (powers of
// two): a butterfly of DPP and permlane exchanges, with no LDS traffic.
template<int LO, int HI>
__device__ __forceinline__ float xor_sum(float v) {
    if constexpr (LO < HI)
        return xor_sum<LO * 2, HI>(v + lane_xor_f<LO>(v));
    else
        return v;
}

// Raw bits of one activation element (converted at use, so that a prefetch
// needs no wait when it is issued).
template<typename Scalar>
__device__ __forceinline__ uint32_t raw_load(const Scalar *p) {
    if constexpr (sizeof(Scalar) == 4)
        return *reinterpret_cast<const uint32_t *>(p);
    else
        return *reinterpret_cast<const uint16_t *>(p);
}

// SAVED: the forward saved the rows x - s and the read rows (job.delta,
// job.saved_r), so the forward pass over t is skipped and the backward pass
// also forms the read dot products d_j from the saved read rows.
template<typename Scalar, int EPP, int NP, int VEC, bool SAVED>
__global__ __launch_bounds__(kWave) void segment_bwd_scan_kernel(const SegmentBwdJob job, int n_sub) {
    constexpr int LPE = kWave / EPP;               // lanes per event (consecutive: channel groups)
    constexpr int CSW = LPE * VEC;
    constexpr int KP = NP * EPP;                   // event slots per token (padded)
    constexpr int CH = bwd_chunk(EPP, NP, VEC);         // tokens per staged chunk
    constexpr int NREC = CH * KP;                  // records of each kind per chunk
    constexpr int RPL = (NREC + kWave - 1) / kWave;
    constexpr int NXE = CH * CSW;                  // x (and Dy) elements per chunk
    constexpr int XPL = (NXE + kWave - 1) / kWave;
    constexpr int GX = EPP < CH ? EPP : CH;        // tokens per batched grad_x store
    // Reductions by reduce-scatter over the tokens of a group (one exchange
    // per token instead of an all-reduce and a select per token): over the
    // LPE channel lanes of an event (lane bits 0 .. log2(LPE) - 1) for the
    // read dots and Dg, over the EPP event lanes (the bits above) for Dx
    // when a chunk holds EPP tokens.
    constexpr int LOGL = __builtin_ctz(LPE);
    constexpr bool XSC = EPP <= CH;
    constexpr int NXS = XSC ? EPP : 1;
    // The chunk's event records and activations, loaded once per chunk
    // (one element per lane) and read back per token as LDS broadcasts.
    __shared__ int4 stw[NREC];   // write records {slot, g, matched read weight, mass}
    __shared__ int2 str[NREC];   // read records {slot, effective weight}
    __shared__ float stx[NXE];   // x_t (forward) on the slice's channels
    __shared__ float sdy[NXE];   // Dy_t on the slice's channels
    extern __shared__ __align__(16) float st[];  // (A + 2) rows of CSW: rows -2 and -1 are the no-op rows
    const SegmentJob &fj = job.fwd;
    const int A = fj.A, C = fj.C, T = fj.T, Kw = fj.Kw, Kr = fj.Kr;
    const int BH = fj.B * fj.H;
    const int t_pad = (T + CH - 1) / CH * CH;
    // Workgroups are dealt round-robin to the 8 XCDs; give each XCD a
    // contiguous run of units so the slices of one (b, h), which read the
    // same records and activations, share an L2.
    const int n_units = BH * n_sub;
    const int per_xcd = (n_units + 7) / 8;
    const int unit = static_cast<int>(blockIdx.x % 8) * per_xcd + static_cast<int>(blockIdx.x / 8);
    if (unit >= n_units)
        return;
    const int bh = unit / n_sub, sub = unit - bh * n_sub;
    const int lane = static_cast<int>(threadIdx.x);
    const int e = lane / LPE, q = lane % LPE;
    const int c0 = sub * CSW + q * VEC;  // first channel of this lane
    uint32_t hi[6];
    hi[0] = bit_mask<1>(lane);
    hi[1] = bit_mask<2>(lane);
    hi[2] = bit_mask<4>(lane);
    hi[3] = bit_mask<8>(lane);
    hi[4] = bit_mask<16>(lane);
    hi[5] = bit_mask<32>(lane);
    auto opq = [](float v) { return __uint_as_float(opaque(__float_as_uint(v))); };
    float *rows = st + 2 * CSW;
    const Scalar *xs = static_cast<const Scalar *>(fj.x);
    const Scalar *dys = static_cast<const Scalar *>(job.grad_y);
    const int2 *rev2 = reinterpret_cast<const int2 *>(job.aux.rev);  // {slot, weight} of each 16-byte record
    // per-slice partial sums of this unit: [t][KP]
    float *drp = job.dr_part + (static_cast<int64_t>(sub) * BH + bh) * t_pad * KP;
    float *dgp = job.dg_part + (static_cast<int64_t>(sub) * BH + bh) * t_pad * KP;
    // the rows x - s: (unit, T_pad, KP, CSW), the forward's padded token count
    // the rows x - s: (unit, T_pad, KP, CSW), the forward's padded token count
    const int64_t unit_rows = static_cast<int64_t>(unit) * scan_t_pad(T) * KP * CSW;
    float *dlt = job.delta + unit_rows + e * CSW + q * VEC;  // + (t * KP + p * EPP) * CSW
    // They are read back through buffer resources over the unit's rows: a
    // byte offset per lane and pass, and the token's as a scalar offset, so
    // the loads need no per-lane address arithmetic.
    const int unit_bytes = scan_t_pad(T) * KP * CSW * 4;
    const auto rsd = __builtin_amdgcn_make_buffer_rsrc(job.delta + unit_rows, 0, unit_bytes, kBufWord3);
    [[maybe_unused]] const auto rsr = __builtin_amdgcn_make_buffer_rsrc(
        SAVED ? const_cast<float *>(job.saved_r) + unit_rows : nullptr, 0, SAVED ? unit_bytes : 0, kBufWord3);
    int svo[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p)
        svo[p] = ((p * EPP + e) * CSW + q * VEC) * 4;

    struct Pre {
        int4 w[RPL];
        int2 r[RPL];
        uint32_t x[XPL];
        uint32_t dy[XPL];
    };
    // token j of chunk ci, clamped into [0, T)
    auto token = [&](int ci, int j, auto fwd_tag) {
        const int t = decltype(fwd_tag)::value ? ci * CH + j : T - 1 - ci * CH - j;
        return min(max(t, 0), T - 1);
    };
    // Offsets within the head are 32-bit (T * K and T * C fit an int: the
    // host checks B * H * T * C and B * H * T_pad * (Kw + Kr)), from bases
    // per head, so a load costs no 64-bit index arithmetic.
    const int4 *wev_h = job.aux.wev + static_cast<int64_t>(bh) * T * Kw;
    const int2 *rev_h = rev2 + 2 * static_cast<int64_t>(bh) * T * Kr;
    const Scalar *dy_h = dys + static_cast<int64_t>(bh) * T * C;
    const Scalar *x_h = xs + static_cast<int64_t>(bh) * T * C;
    auto prefetch = [&](int ci, Pre &pf, auto fwd_tag) {
#pragma unroll
        for (int i = 0; i < RPL; ++i) {
            const int idx = min(lane + kWave * i, NREC - 1);
            const int k = idx % KP;
            const int t = token(ci, idx / KP, fwd_tag);
            pf.w[i] = wev_h[static_cast<uint32_t>(t * Kw + min(k, Kw - 1))];
            pf.r[i] = rev_h[2u * static_cast<uint32_t>(t * Kr + min(k, Kr - 1))];
        }
#pragma unroll
        for (int i = 0; i < XPL; ++i) {
            const int idx = min(lane + kWave * i, NXE - 1);
            const int c = min(sub * CSW + idx % CSW, C - 1);
            const uint32_t o = static_cast<uint32_t>(token(ci, idx / CSW, fwd_tag) * C + c);
            pf.dy[i] = raw_load(dy_h + o);
            if constexpr (decltype(fwd_tag)::value)
                pf.x[i] = raw_load(x_h + o);
        }
    };
    auto stage = [&](const Pre &pf, auto fwd_tag) {
#pragma unroll
        for (int i = 0; i < RPL; ++i) {
            const int idx = lane + kWave * i;
            if (NREC % kWave == 0 || idx < NREC) {
                // padding slots get the no-op records; selected bitwise, as a
                // branch around the copy would wait for every outstanding access
                const int k = idx % KP;
                const uint32_t mw = k < Kw ? ~0u : 0u;
                const int4 w = pf.w[i];
                stw[idx] = make_int4(static_cast<int>(bfi(mw, w.x, static_cast<uint32_t>(-2))), static_cast<int>(bfi(mw, w.y, 0)),
                                     static_cast<int>(bfi(mw, w.z, 0)), static_cast<int>(bfi(mw, w.w, 0)));
                str[idx] = k < Kr ? pf.r[i] : make_int2(-1, 0);
            }
        }
#pragma unroll
        for (int i = 0; i < XPL; ++i) {
            const int idx = lane + kWave * i;
            if (NXE % kWave == 0 || idx < NXE) {
                const bool real = sub * CSW + idx % CSW < C;
                sdy[idx] = real ? half_bits_to_f<Scalar>(pf.dy[i]) : 0.f;
                if constexpr (decltype(fwd_tag)::value)
                    stx[idx] = real ? half_bits_to_f<Scalar>(pf.x[i]) : 0.f;
            }
        }
    };
    auto lds_vec = [&](const float *p) { return lds_load<VEC>(p); };
    const int nck = (T + CH - 1) / CH;

    // A chunk's results stay in registers and are stored at the start of the
    // next chunk, before its prefetch, so a wait for prefetched data never
    // waits on stores just issued; and the chunk loop runs two chunks per
    // iteration with swapped buffers, as a copy of a register with a load
    // pending waits for every outstanding access.
    constexpr int NG = CH / LPE;   // groups of LPE tokens per chunk (read dots, Dg)
    constexpr int NGX = CH / GX;   // groups of GX tokens per chunk (Dx)
    static_assert(CH % LPE == 0 && CH % GX == 0, "a chunk holds whole groups");
    // Wide lanes at two passes (more than 32 saved floats per chunk) would
    // spill with the held-back saved rows and the paired chunk buffers: those
    // store the saved rows as they go and loop over single chunks.
    constexpr bool HOLD = CH * NP * VEC <= 32;

    // ---- forward over t: s in LDS; save x - s before each write, d_j per read
    if constexpr (!SAVED) {
    for (int i = lane; i < (A + 2) * CSW; i += kWave) {
        const int a = i / CSW - 2, c = sub * CSW + i % CSW;
        st[i] = (a >= 0 && c < C) ? fj.init_slot[(static_cast<int64_t>(bh) * A + a) * C + c] : 0.f;
    }
    __syncthreads();
    {
        using Tag = std::true_type;
        struct Out {
            FVec<VEC> d[HOLD ? CH : 1][NP];  // x - s of each write row, per token
            float dr[NG][NP];     // d_j of token (group start + q)
        };
        Out out;
        auto flush = [&](int ci) {
            const int n = min(CH, T - ci * CH);
            float *dc = dlt + static_cast<int64_t>(ci) * CH * KP * CSW;
            float *rc = drp + (static_cast<int64_t>(ci) * CH + q) * KP + e;  // rows padded to whole chunks
            auto put = [&](auto full_tag) {
                constexpr bool FULL = decltype(full_tag)::value;
                if constexpr (HOLD) {
#pragma unroll
                    for (int j = 0; j < CH; ++j)
                        if (FULL || j < n) {
#pragma unroll
                            for (int p = 0; p < NP; ++p)
                                lds_store<VEC>(dc + (j * KP + p * EPP) * CSW, out.d[j][p]);
                        }
                }
#pragma unroll
                for (int g = 0; g < NG; ++g)
                    if (FULL || g * LPE < n) {
#pragma unroll
                        for (int p = 0; p < NP; ++p)
                            rc[g * LPE * KP + p * EPP] = out.dr[g][p];
                    }
            };
            if (n == CH)
                put(std::true_type{});
            else
                put(std::false_type{});
        };
        auto chunk = [&](int ci, Pre &cur, Pre &nxt) {
            stage(cur, Tag{});
            if (ci > 0)
                flush(ci - 1);
            prefetch(min(ci + 1, nck - 1), nxt, Tag{});
            // the chunk's records and activations for this lane, read back in
            // one batch, so that each token costs one LDS round trip
            int wsl[CH][NP], rsl[CH][NP];
            float wg[CH][NP], xv[CH][VEC], dyv[CH][VEC];
#pragma unroll
            for (int j = 0; j < CH; ++j) {
#pragma unroll
                for (int p = 0; p < NP; ++p) {
                    const int2 w2 = *reinterpret_cast<const int2 *>(&stw[j * KP + p * EPP + e]);
                    wsl[j][p] = w2.x;
                    wg[j][p] = __int_as_float(w2.y);
                    rsl[j][p] = str[j * KP + p * EPP + e].x;
                }
#pragma unroll
                for (int v = 0; v < VEC; ++v) {
                    xv[j][v] = stx[j * CSW + q * VEC + v];
                    dyv[j][v] = sdy[j * CSW + q * VEC + v];
                }
            }
            // write rows of the current token, loaded one token ahead:
            // after the previous token's writes, with its reads
            FVec<VEC> sw[NP];
#pragma unroll
            for (int p = 0; p < NP; ++p)
                sw[p] = lds_vec(rows + wsl[0][p] * CSW + q * VEC);
            // d_j of token j: the dot of its read rows with Dy_t; the lane's
            // partials of a group of LPE tokens are reduced over the event's
            // lanes at once, leaving token (group start + q) in lane q
            float rdp[NP][LPE];
#pragma unroll
            for (int p = 0; p < NP; ++p)
#pragma unroll
                for (int m = 0; m < LPE; ++m)
                    rdp[p][m] = 0.f;
            auto read_dot = [&](int j, const FVec<VEC> (&sr)[NP]) {
#pragma unroll
                for (int p = 0; p < NP; ++p) {
                    float part = 0.f;
#pragma unroll
                    for (int v = 0; v < VEC; ++v)
                        part = fmaf(sr[p].v[v], dyv[j][v], part);
                    rdp[p][j % LPE] = opq(part);
                }
                if (j % LPE == LPE - 1) {
#pragma unroll
                    for (int p = 0; p < NP; ++p) {
                        event_scatter<LOGL - 1, 0, LPE>(rdp[p], hi);
                        out.dr[j / LPE][p] = rdp[p][0];
                    }
                }
            };
            FVec<VEC> sr[NP];  // read rows of the previous token, reduced one token late
            // Chunks wholly inside T run without the per-token guards, so
            // the token body is one basic block.
            auto tokens = [&](auto tail_tag) {
                constexpr bool TL = decltype(tail_tag)::value;
#pragma unroll
                for (int j = 0; j < CH; ++j) {
                    const int t = ci * CH + j;
                    if (TL && t >= T)
                        break;
#pragma unroll
                    for (int p = 0; p < NP; ++p) {
                        FVec<VEC> s = sw[p], d;
#pragma unroll
                        for (int v = 0; v < VEC; ++v) {
                            d.v[v] = xv[j][v] - s.v[v];
                            s.v[v] = fmaf(wg[j][p], d.v[v], s.v[v]);
                        }
                        lds_store<VEC>(rows + wsl[j][p] * CSW + q * VEC, s);
                        if constexpr (HOLD)
                            out.d[j][p] = d;
                        else
                            lds_store<VEC>(dlt + (static_cast<int64_t>(t) * KP + p * EPP) * CSW, d);
                    }
                    FVec<VEC> srn[NP];
#pragma unroll
                    for (int p = 0; p < NP; ++p)
                        srn[p] = lds_vec(rows + rsl[j][p] * CSW + q * VEC);
                    if (j + 1 < CH) {
#pragma unroll
                        for (int p = 0; p < NP; ++p)
                            sw[p] = lds_vec(rows + wsl[j + 1][p] * CSW + q * VEC);
                    }
                    if (j > 0)
                        read_dot(j - 1, sr);
#pragma unroll
                    for (int p = 0; p < NP; ++p)
                        sr[p] = srn[p];
                    if (j == CH - 1 || (TL && t == T - 1))
                        read_dot(j, sr);
                }
            };
            if ((ci + 1) * CH <= T)
                tokens(std::false_type{});
            else
                tokens(std::true_type{});
            if constexpr (LPE > 1) {
                if (T - ci * CH < CH && (T - ci * CH) % LPE != 0) {  // ragged last group
                    const int gl = (T - ci * CH) / LPE;
#pragma unroll
                    for (int p = 0; p < NP; ++p) {
                        event_scatter<LOGL - 1, 0, LPE>(rdp[p], hi);
#pragma unroll
                        for (int g = 0; g < NG; ++g)
                            if (g == gl)
                                out.dr[g][p] = rdp[p][0];
                    }
                }
            }
        };
        Pre pa, pb;
        prefetch(0, pa, Tag{});
        for (int ci = 0; ci < nck; ci += HOLD ? 2 : 1) {
            chunk(ci, pa, pb);
            if constexpr (HOLD) {
                if (ci + 1 < nck)
                    chunk(ci + 1, pb, pa);
            } else {
                pa = pb;
            }
        }
        flush(nck - 1);
    }
    __syncthreads();
    }

    // ---- backward over t: Ds in LDS
    for (int i = lane; i < (A + 2) * CSW; i += kWave) {
        const int a = i / CSW - 2, c = sub * CSW + i % CSW;
        st[i] = (a >= 0 && c < C && job.grad_slot) ? job.grad_slot[(static_cast<int64_t>(bh) * A + a) * C + c] : 0.f;
    }
    __syncthreads();
    {
        using Tag = std::false_type;
        // the saved rows x - s of this lane's write events (and with SAVED the
        // read rows of its read events), per token of a chunk
        constexpr int NSR = SAVED ? CH : 1;
        struct Saved {
            uint32_t v[CH][NP * VEC];
            uint32_t r[NSR][NP * VEC];
        };
        auto buf_vec = [&](__amdgpu_buffer_rsrc_t rs, int vo, int so, uint32_t *out) {
            if constexpr (VEC == 4) {
                const auto q4 = __builtin_amdgcn_raw_buffer_load_b128(rs, vo, so, 0);
                out[0] = q4[0]; out[1] = q4[1]; out[2] = q4[2]; out[3] = q4[3];
            } else if constexpr (VEC == 2) {
                const auto q2 = __builtin_amdgcn_raw_buffer_load_b64(rs, vo, so, 0);
                out[0] = q2[0]; out[1] = q2[1];
            } else {
                out[0] = __builtin_amdgcn_raw_buffer_load_b32(rs, vo, so, 0);
            }
        };
        auto load_saved = [&](int ci, Saved &sv) {
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                const int so = __builtin_amdgcn_readfirstlane(token(ci, j, Tag{})) * (KP * CSW * 4);
#pragma unroll
                for (int p = 0; p < NP; ++p) {
                    buf_vec(rsd, svo[p], so, sv.v[j] + p * VEC);
                    if constexpr (SAVED)
                        buf_vec(rsr, svo[p], so, sv.r[j] + p * VEC);
                }
            }
        };
        struct Out {
            float dg[NG][NP];    // Dg of token (group start - q)
            float gx[NGX][VEC];  // Dx of token (group start - e)
            float dr[SAVED ? NG : 1][NP];  // SAVED: d_j of token (group start - q)
        };
        Out out;
        float *gx = job.grad_x + static_cast<int64_t>(bh) * T * C;
        auto flush = [&](int ci) {
            const int n = min(CH, T - ci * CH);
            const int t0 = T - 1 - ci * CH;  // the chunk's first token; group g's in this lane: t0 - g * LPE - q (Dg), t0 - g * GX - e (Dx)
            auto put = [&](auto full_tag) {
                constexpr bool FULL = decltype(full_tag)::value;
#pragma unroll
                for (int g = 0; g < NG; ++g)
                    if (FULL || g * LPE + q < n) {
                        const int64_t tg = t0 - g * LPE - q;
#pragma unroll
                        for (int p = 0; p < NP; ++p) {
                            dgp[tg * KP + p * EPP + e] = out.dg[g][p];
                            if constexpr (SAVED)
                                drp[tg * KP + p * EPP + e] = out.dr[g][p];
                        }
                    }
                if (e < GX) {
#pragma unroll
                    for (int g = 0; g < NGX; ++g)
                        if (FULL || g * GX + e < n) {
                            const int64_t tg = t0 - g * GX - e;
#pragma unroll
                            for (int v = 0; v < VEC; ++v)
                                if (c0 + v < C)
                                    gx[tg * C + c0 + v] = out.gx[g][v];
                        }
                }
            };
            if (n == CH)
                put(std::true_type{});
            else
                put(std::false_type{});
        };
        auto chunk = [&](int ci, Pre &cur, Pre &nxt, Saved &scur, Saved &snxt) {
            stage(cur, Tag{});
            if (ci > 0)
                flush(ci - 1);
            prefetch(min(ci + 1, nck - 1), nxt, Tag{});
            load_saved(min(ci + 1, nck - 1), snxt);
            int wsl[CH][NP], rsl[CH][NP];
            float wg[CH][NP], wrm[CH][NP], rw[CH][NP], dyv[CH][VEC];
#pragma unroll
            for (int j = 0; j < CH; ++j) {
#pragma unroll
                for (int p = 0; p < NP; ++p) {
                    const int4 w4 = stw[j * KP + p * EPP + e];
                    const int2 r2 = str[j * KP + p * EPP + e];
                    wsl[j][p] = w4.x;
                    wg[j][p] = __int_as_float(w4.y);
                    wrm[j][p] = __int_as_float(w4.z);
                    rsl[j][p] = r2.x;
                    rw[j][p] = __int_as_float(r2.y);
                }
#pragma unroll
                for (int v = 0; v < VEC; ++v)
                    dyv[j][v] = sdy[j * CSW + q * VEC + v];
            }
            float dgp_[NP][LPE];  // Dg partials of a group of LPE tokens (token group start - m)
            float rdp_[SAVED ? NP : 1][LPE];  // SAVED: d_j partials, grouped as Dg's
            float dxp[VEC][NXS];  // Dx partials of a group of EPP tokens (reduce-scatter form)
            float keep_x[VEC];    // Dx of token (group start - e) (all-reduce form)
#pragma unroll
            for (int p = 0; p < NP; ++p)
#pragma unroll
                for (int m = 0; m < LPE; ++m) {
                    dgp_[p][m] = 0.f;
                    if constexpr (SAVED)
                        rdp_[p][m] = 0.f;
                }
#pragma unroll
            for (int v = 0; v < VEC; ++v) {
                keep_x[v] = 0.f;
#pragma unroll
                for (int m = 0; m < NXS; ++m)
                    dxp[v][m] = 0.f;
            }
            // rows of the current token, loaded before the previous token's
            // reductions (after its stores)
            FVec<VEC> dr[NP], dw[NP];
#pragma unroll
            for (int p = 0; p < NP; ++p)
                dr[p] = lds_vec(rows + rsl[0][p] * CSW + q * VEC);
#pragma unroll
            for (int p = 0; p < NP; ++p)
                dw[p] = lds_vec(rows + wsl[0][p] * CSW + q * VEC);
            // chunks wholly inside T run without the per-token guards
            auto tokens = [&](auto tail_tag) {
                constexpr bool TL = decltype(tail_tag)::value;
#pragma unroll
                for (int j = 0; j < CH; ++j) {
                    const int t = T - 1 - ci * CH - j;
                    if (TL && t < 0)
                        break;
                    // a write takes the read of its own slot (same token) from its
                    // matched weight, and its store lands after that read's
#pragma unroll
                    for (int p = 0; p < NP; ++p) {
#pragma unroll
                        for (int v = 0; v < VEC; ++v)
                            dr[p].v[v] = fmaf(rw[j][p], dyv[j][v], dr[p].v[v]);
                        lds_store<VEC>(rows + rsl[j][p] * CSW + q * VEC, dr[p]);
                    }
                    float dx[VEC], part[NP];
#pragma unroll
                    for (int v = 0; v < VEC; ++v)
                        dx[v] = 0.f;
#pragma unroll
                    for (int p = 0; p < NP; ++p) {
                        const float g = wg[j][p];
                        FVec<VEC> D = dw[p];
                        part[p] = 0.f;
#pragma unroll
                        for (int v = 0; v < VEC; ++v) {
                            D.v[v] = fmaf(wrm[j][p], dyv[j][v], D.v[v]);
                            part[p] = fmaf(D.v[v], __uint_as_float(scur.v[j][p * VEC + v]), part[p]);
                            dx[v] = fmaf(g, D.v[v], dx[v]);
                            D.v[v] = fmaf(-g, D.v[v], D.v[v]);
                        }
                        lds_store<VEC>(rows + wsl[j][p] * CSW + q * VEC, D);
                    }
                    if (j + 1 < CH) {
#pragma unroll
                        for (int p = 0; p < NP; ++p)
                            dr[p] = lds_vec(rows + rsl[j + 1][p] * CSW + q * VEC);
#pragma unroll
                        for (int p = 0; p < NP; ++p)
                            dw[p] = lds_vec(rows + wsl[j + 1][p] * CSW + q * VEC);
                    }
#pragma unroll
                    for (int p = 0; p < NP; ++p)
                        dgp_[p][j % LPE] = opq(part[p]);
                    if constexpr (SAVED) {
                        // d_j of this token: its saved read rows with Dy_t
#pragma unroll
                        for (int p = 0; p < NP; ++p) {
                            float pr = 0.f;
#pragma unroll
                            for (int v = 0; v < VEC; ++v)
                                pr = fmaf(__uint_as_float(scur.r[j][p * VEC + v]), dyv[j][v], pr);
                            rdp_[p][j % LPE] = opq(pr);
                        }
                    }
                    if (j % LPE == LPE - 1 || (TL && t == 0)) {
#pragma unroll
                        for (int p = 0; p < NP; ++p) {
                            event_scatter<LOGL - 1, 0, LPE>(dgp_[p], hi);
                            out.dg[j / LPE][p] = dgp_[p][0];
                            if constexpr (SAVED) {
                                event_scatter<LOGL - 1, 0, LPE>(rdp_[p], hi);
                                out.dr[j / LPE][p] = rdp_[p][0];
                            }
                        }
                    }
                    if constexpr (XSC) {
#pragma unroll
                        for (int v = 0; v < VEC; ++v)
                            dxp[v][j % GX] = opq(dx[v]);
                        if (j % GX == GX - 1 || (TL && t == 0)) {
#pragma unroll
                            for (int v = 0; v < VEC; ++v) {
                                event_scatter<__builtin_ctz(NXS) - 1, LOGL, NXS>(dxp[v], hi);
                                out.gx[j / GX][v] = dxp[v][0];
                            }
                        }
                    } else {
#pragma unroll
                        for (int v = 0; v < VEC; ++v) {
                            const float sx = strided_sum<LPE>(dx[v]);
                            keep_x[v] = e == j % GX ? sx : keep_x[v];
                        }
                        if (j % GX == GX - 1 || (TL && t == 0)) {
#pragma unroll
                            for (int v = 0; v < VEC; ++v)
                                out.gx[j / GX][v] = keep_x[v];
                        }
                    }
                }
            };
            if ((ci + 1) * CH <= T)
                tokens(std::false_type{});
            else
                tokens(std::true_type{});
        };
        Pre pa, pb;
        Saved sa, sb;
        prefetch(0, pa, Tag{});
        load_saved(0, sa);
        for (int ci = 0; ci < nck; ci += HOLD ? 2 : 1) {
            chunk(ci, pa, pb, sa, sb);
            if constexpr (HOLD) {
                if (ci + 1 < nck)
                    chunk(ci + 1, pb, pa, sb, sa);
            } else {
                pa = pb;
                sa = sb;
            }
        }
        flush(nck - 1);
    }
    __syncthreads();
    for (int i = lane; i < A * CSW; i += kWave) {
        const int a = i / CSW, c = sub * CSW + i % CSW;
        if (c < C)
            job.grad_init_slot[(static_cast<int64_t>(bh) * A + a) * C + c] = rows[i];
    }
}

// Per-slice partial sums [sub][bh][t_pad][KP] -> totals [bh][t][K], summed in
// slice order.
__global__ __launch_bounds__(256) void segment_bwd_sum_kernel(const float *part, float *out, int n_sub, int BH, int T,
                                                              int t_pad, int KP, int K) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t n = static_cast<int64_t>(BH) * T * K;
    if (i >= n)
        return;
    const int k = static_cast<int>(i % K);
    const int64_t bt = i / K;
    const int t = static_cast<int>(bt % T);
    const int64_t bh = bt / T;
    const int64_t stride = static_cast<int64_t>(BH) * t_pad * KP;
    const float *src = part + (bh * t_pad + t) * KP + k;
    // eight loads in flight at a time (clamped into range, so unconditional),
    // added in slice order
    float s = 0.f;
    for (int u0 = 0; u0 < n_sub; u0 += 8) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            v[j] = src[static_cast<int64_t>(min(u0 + j, n_sub - 1)) * stride];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int u = u0 + j;
            s = u == 0 ? v[j] : u < n_sub ? s + v[j] : s;
        }
    }
    out[i] = s;
}

// ---- the mass chain, chunked over time
//
// Walking back in time, each slot's Dm evolves affinely with coefficients
// that do not depend on Dm: a write maps Dm to alpha (Dm - Dg g / den), a
// mass-aware read adds c rho (d - Q). So, as in the forward mass pre-pass:
//   1. MAP: per (b, h, chunk), every slot's composed map
//      Dm(chunk start) = a Dm(chunk end) + b;
//   2. segment_bwd_mass_scan_kernel: per (b, h, slot), Dm at every chunk's
//      end from the final-state gradient and the maps (last chunk first), and
//      dL/d init_mass;
//   3. REPLAY: per (b, h, chunk), the chunk walked back from its end values,
//      writing dL/dw, dL/drho and dL/dgamma.
// Lanes 0..31 take write events p * 32 + lane, lanes 32..63 read events.

// One token's loads for a lane of the mass kernels.
template<int MP>
struct MassTok {
    int4 ev[MP];   // the event's record (write: {slot, g, matched read weight, mass before};
                   // read: {slot, effective weight, post-write mass, 0})
    float v[MP];   // write: w; read: the stored (negated) weight
    float dd[MP];  // write: Dg; read: d_j
};

// The token body is branch-free: every quantity that does not depend on the
// slot values (alpha, the reciprocals, the read-side sums) is computed for
// all lanes, and an event that is off acts on its kind's no-op slot (-2 for
// writes, -1 for reads), so the only dependent chain from token to token is
// the slot's LDS read-modify-write, and the scheduler can overlap the rest of
// neighbouring tokens with it. The no-op slots' values are never used.
template<typename Scalar, bool MA, int MP, bool REPLAY>
__global__ __launch_bounds__(kWave) void segment_bwd_mass_kernel(const SegmentBwdJob job, float2 *maps,
                                                                int chunk_len) {
    constexpr int CH = MP == 1 ? 16 : MP == 2 ? 8 : 4;
    extern __shared__ __align__(16) float lds[];
    const SegmentJob &fj = job.fwd;
    const int A = fj.A, T = fj.T, Kw = fj.Kw, Kr = fj.Kr, Kt = Kw + Kr;
    const float eps = fj.eps;
    const int bh = static_cast<int>(blockIdx.x), ck = static_cast<int>(blockIdx.y), nck = static_cast<int>(gridDim.y);
    const int lane = static_cast<int>(threadIdx.x);
    const int hl = lane & 31;
    const bool wlane = lane < 32;
    float *dm = lds + 2;                              // REPLAY: Dm per slot; dm[-2], dm[-1] the no-op slots
    float2 *mp = reinterpret_cast<float2 *>(lds) + 2;  // MAP: (a, b) per slot
    const float2 *ends = maps + (static_cast<int64_t>(bh) * nck + ck) * A;
    if constexpr (REPLAY) {
        for (int a = lane; a < A; a += kWave)
            dm[a] = nck > 1 ? ends[a].x : (job.grad_mass ? job.grad_mass[static_cast<int64_t>(bh) * A + a] : 0.f);
        if (lane < 2)
            lds[lane] = 0.f;
    } else {
        for (int a = lane - 2; a < A; a += kWave)
            mp[a] = make_float2(1.f, 0.f);
    }
    __syncthreads();
    const Scalar *gs = static_cast<const Scalar *>(job.gamma) + static_cast<int64_t>(bh) * T;
    const float *val = job.addr_val + static_cast<int64_t>(bh) * Kt * T;
    float *gval = job.grad_val + static_cast<int64_t>(bh) * Kt * T;
    bool on[MP];
    int ec[MP];
#pragma unroll
    for (int p = 0; p < MP; ++p) {
        const int ev = p * 32 + hl;
        on[p] = wlane ? ev < Kw : ev < Kr;
        ec[p] = min(ev, (wlane ? Kw : Kr) - 1);
    }
    const int4 *evp = wlane ? job.aux.wev : job.aux.rev;
    const float *ddp = wlane ? job.dg_sum : job.dr_sum;
    const int kl = wlane ? Kw : Kr, koff = wlane ? 0 : Kw;
    // per-lane bases of this head's records, Dg / d sums and weights; a
    // token adds t * kl records (t * 1 weights). Loads a lane does not use
    // repeat write lane hl's addresses (same cache lines, no extra traffic):
    // without mass-aware reads, the chunk maps use only the write events and
    // the replay's read lanes only the records and d sums.
    const bool rd_rec = MA || REPLAY, rd_val = MA;
    const int hw = wlane || rd_rec ? 0 : 1;  // 1: this read lane loads write lane hl's records
    const int hv = wlane || rd_val ? 0 : 1;  // 1: ... and its weights
    const int64_t head = static_cast<int64_t>(bh) * T;
    const int klr = hw ? Kw : kl;
    const int4 *ev_l[MP];
    const float *dd_l[MP], *v_l[MP];
#pragma unroll
    for (int p = 0; p < MP; ++p) {
        const int ecw = min(p * 32 + hl, Kw - 1);
        ev_l[p] = (hw ? job.aux.wev : evp) + head * klr + (hw ? ecw : ec[p]);
        dd_l[p] = (hw ? job.dg_sum : ddp) + head * klr + (hw ? ecw : ec[p]);
        v_l[p] = val + static_cast<int64_t>(hv ? ecw : koff + ec[p]) * T;
    }

    auto load_tok = [&](int t, MassTok<MP> &k) {
        const uint32_t tk = static_cast<uint32_t>(t) * static_cast<uint32_t>(klr);
#pragma unroll
        for (int p = 0; p < MP; ++p) {
            k.ev[p] = ev_l[p][tk];
            k.v[p] = v_l[p][t];
            k.dd[p] = dd_l[p][tk];
        }
    };
    const int t_begin = ck * chunk_len, t_end = min(T, t_begin + chunk_len);
    const int n = t_end - t_begin;
    const int nc = (n + CH - 1) / CH;
    // group ci's tokens t_end - 1 - ci * CH - j, j < CH (clamped to the
    // chunk); gamma of token j in lane j: the exponential of every token of
    // a group is one vector operation, read back per token as a scalar
    auto tok_t = [&](int ci, int j) { return max(t_end - 1 - ci * CH - j, t_begin); };
    auto load_group = [&](int ci, MassTok<MP> (&k)[CH], uint32_t &graw) {
#pragma unroll
        for (int j = 0; j < CH; ++j)
            load_tok(tok_t(ci, j), k[j]);
        graw = raw_load(gs + tok_t(ci, lane % CH));
    };
    // REPLAY: the chunk's gradients per lane (event) and of gamma, stored as
    // runs of consecutive tokens once the chunk is done
    auto store_run = [&](float *row, int t_hi, const float *vals, int stride) {
        const int t_lo = t_hi - (CH - 1);
        if (t_lo >= t_begin && (t_lo & 3) == 0 && (T & 3) == 0) {
#pragma unroll
            for (int i = 0; i < CH; i += 4)
                *reinterpret_cast<float4 *>(row + t_lo + i) =
                    make_float4(vals[(CH - 1 - i) * stride], vals[(CH - 2 - i) * stride],
                                vals[(CH - 3 - i) * stride], vals[(CH - 4 - i) * stride]);
        } else {
#pragma unroll
            for (int j = 0; j < CH; ++j)
                if (t_hi - j >= t_begin)
                    row[t_hi - j] = vals[j * stride];
        }
    };
    auto group = [&](int ci, const MassTok<MP> (&cur)[CH], uint32_t graw) {
        float outv[CH][MP], outg[CH];
        // tokens past the chunk's start (the last group's tail) repeat
        // t_begin's loads; they act on the no-op slots only
        const int left = n - ci * CH;
        const float gmv = half_bits_to_f<Scalar>(graw);
        const float qdv = expf(-fabsf(gmv));
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            const bool tok = j < left;
            const MassTok<MP> &k = cur[j];
            // every field of the record counts as used, so that it stays one
            // 16-byte load: a group's loads then fit the memory counter's 63
            // (3 per token and event, 16 tokens, and gamma), and the wait for
            // this group does not take in the next group's first loads
#pragma unroll
            for (int p = 0; p < MP; ++p)
                asm volatile("" ::"v"(k.ev[p].z));
            // reads of token t (they follow its writes in the forward)
            float dr[MP];
            if constexpr (MA) {
                float sr = 0.f, srm = 0.f, sdm = 0.f;
                bool a_on[MP];
#pragma unroll
                for (int p = 0; p < MP; ++p) {
                    a_on[p] = tok & !wlane & on[p] & (k.ev[p].x >= 0);
                    const float rho = a_on[p] ? -k.v[p] : 0.f;
                    sr += rho;
                    srm = fmaf(rho, __int_as_float(k.ev[p].z), srm);
                    sdm = fmaf(rho * __int_as_float(k.ev[p].z), a_on[p] ? k.dd[p] : 0.f, sdm);
                }
                sr = xor_sum<1, 32>(sr);
                srm = xor_sum<1, 32>(srm);
                sdm = xor_sum<1, 32>(sdm);
                const float inv = 1.f / (srm + eps);
                const float c = sr * inv, Q = sdm * inv;
#pragma unroll
                for (int p = 0; p < MP; ++p) {
                    const uint32_t am = a_on[p] ? ~0u : 0u;
                    const float diff = k.dd[p] - Q;
                    dr[p] = keep_if(fmaf(c * __int_as_float(k.ev[p].z), diff, Q), am);
                    const float kap = keep_if(-c * k.v[p] * diff, am);
                    const int s = a_on[p] ? k.ev[p].x : -1;
                    if constexpr (REPLAY)
                        dm[s] += kap;
                    else
                        mp[s].y += kap;
                }
                // the write lanes' reads of this token's slots come after
                // the read lanes' updates (other lanes, same slots)
                __builtin_amdgcn_wave_barrier();
            } else {
#pragma unroll
                for (int p = 0; p < MP; ++p)
                    dr[p] = keep_if(k.dd[p], (tok & !wlane & on[p] & (k.ev[p].x >= 0)) ? ~0u : 0u);
            }
            // writes of token t: alpha in the stable form of gsu_alpha, with
            // q = e^-|gamma| and reciprocals of its denominator dn and of
            // m' + eps (each v_rcp_f32 and a Newton step)
            float dgam = 0.f;
            float dw[MP];
            const float gm = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gmv), j));
            const float qd = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(qdv), j));
            const bool gpos = gm >= 0.f;
#pragma unroll
            for (int p = 0; p < MP; ++p) {
                // (bitwise: a short-circuit test of a lane condition becomes
                // an exec-mask region, which the scheduler does not cross)
                // (the chunk maps without mass-aware reads: every lane holds a
                // write record, the read lanes and the lanes past Kw a copy of
                // a write lane's, whose update they repeat in the same
                // instruction; no-op records name slot -2 themselves)
                const bool act = (!REPLAY && !MA) ? tok : tok & wlane & on[p] & (k.ev[p].x >= 0);
                const float w = k.v[p], m = __int_as_float(k.ev[p].w), Dg = k.dd[p];
                const float g = __int_as_float(k.ev[p].y);
                const float cw = 1.f - w;
                const float dn = gpos ? fmaf(qd, cw, w) : fmaf(qd, w, cw);
                const float rdn = recip_nr(dn);
                const float al = (gpos ? cw * qd : cw) * rdn;
                const float den = fmaf(al, m, w) + eps;
                const float rden = recip_nr(den);
                const float q0 = Dg * g * rden;
                const int s = act ? k.ev[p].x : -2;
                if constexpr (REPLAY) {
                    const uint32_t am = act ? ~0u : 0u;
                    const float dtot = dm[s] - q0;
                    dm[s] = dtot * al;
                    const float t2 = qd * rdn * rdn;
                    dw[p] = keep_if(fmaf(dtot, fmaf(-m, t2, 1.f), Dg * rden), am);
                    dgam = fmaf(keep_if(-dtot * m, am), keep_if(cw * w * t2, am), dgam);
                } else {
                    const float2 ab = mp[s];
                    mp[s] = make_float2(al * ab.x, al * (ab.y - q0));
                    dw[p] = 0.f;
                }
            }
            if constexpr (REPLAY) {
                outg[j] = xor_sum<1, 32>(dgam);
#pragma unroll
                for (int p = 0; p < MP; ++p)
                    outv[j][p] = wlane ? dw[p] : dr[p];
            }
        }
        if constexpr (REPLAY) {
            const int t_hi = t_end - 1 - ci * CH;
            if (lane == 0)
                store_run(job.grad_gamma + static_cast<int64_t>(bh) * T, t_hi, outg, 1);
#pragma unroll
            for (int p = 0; p < MP; ++p)
                if (on[p])
                    store_run(gval + static_cast<int64_t>(koff + p * 32 + hl) * T, t_hi, &outv[0][p], MP);
        }
    };
    // two groups per iteration with swapped buffers: a copy of registers
    // with loads pending would wait for every outstanding load
    MassTok<MP> ka[CH], kb[CH];
    uint32_t ga, gb;
    load_group(0, ka, ga);
    int ci = 0;
    for (; ci + 1 < nc; ci += 2) {
        load_group(ci + 1, kb, gb);
        __builtin_amdgcn_sched_barrier(0);
        group(ci, ka, ga);
        __builtin_amdgcn_sched_barrier(0);
        load_group(min(ci + 2, nc - 1), ka, ga);
        __builtin_amdgcn_sched_barrier(0);
        group(ci + 1, kb, gb);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (ci < nc)
        group(ci, ka, ga);
    __syncthreads();
    if constexpr (REPLAY) {
        if (nck == 1) {
            for (int a = lane; a < A; a += kWave)
                job.grad_init_mass[static_cast<int64_t>(bh) * A + a] = dm[a];
        }
    } else {
        float2 *dst = maps + (static_cast<int64_t>(bh) * nck + ck) * A;
        for (int a = lane; a < A; a += kWave)
            dst[a] = mp[a];
    }
}

// Per (b, h, slot): Dm at the end of every chunk (last chunk first) in
// place of its map, and the gradient of the initial mass.
__global__ __launch_bounds__(256) void segment_bwd_mass_scan_kernel(const SegmentBwdJob job, float2 *maps, int nck) {
    const int A = job.fwd.A;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<int64_t>(job.fwd.B) * job.fwd.H * A)
        return;
    const int64_t bh = i / A;
    const int a = static_cast<int>(i - bh * A);
    float D = job.grad_mass ? job.grad_mass[i] : 0.f;
    float2 *mp = maps + bh * nck * A + a;
    // eight chunks' maps loaded before their stores (a store could alias a
    // later load as far as the compiler knows)
    for (int c0 = nck - 1; c0 >= 0; c0 -= 8) {
        float2 ab[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            ab[j] = mp[static_cast<int64_t>(max(c0 - j, 0)) * A];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (c0 - j >= 0) {
                mp[static_cast<int64_t>(c0 - j) * A] = make_float2(D, 0.f);
                D = fmaf(ab[j].x, D, ab[j].y);
            }
        }
    }
    job.grad_init_mass[i] = D;
}

template<typename Scalar, int EPP, int NP, bool SAVED>
hipError_t launch_bwd_scan_saved(const SegmentBwdJob &job, const BwdPlan &p, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>((job.fwd.B * job.fwd.H * p.n_sub + 7) / 8 * 8));
    const size_t lds = static_cast<size_t>(p.lds);
    switch (p.vec) {
        case 1: hipLaunchKernelGGL((segment_bwd_scan_kernel<Scalar, EPP, NP, 1, SAVED>), grid, dim3(kWave), lds, stream, job, p.n_sub); break;
        case 2: hipLaunchKernelGGL((segment_bwd_scan_kernel<Scalar, EPP, NP, 2, SAVED>), grid, dim3(kWave), lds, stream, job, p.n_sub); break;
        default: hipLaunchKernelGGL((segment_bwd_scan_kernel<Scalar, EPP, NP, 4, SAVED>), grid, dim3(kWave), lds, stream, job, p.n_sub); break;
    }
    return hipGetLastError();
}

// Saved rows are taken with one pass of events (segment_saved_slices).
template<typename Scalar, int EPP, int NP>
hipError_t launch_bwd_scan_vec(const SegmentBwdJob &job, const BwdPlan &p, hipStream_t stream) {
    if constexpr (NP == 1) {
        if (job.saved_r)
            return launch_bwd_scan_saved<Scalar, EPP, NP, true>(job, p, stream);
    } else if (job.saved_r) {
        return hipErrorInvalidValue;
    }
    return launch_bwd_scan_saved<Scalar, EPP, NP, false>(job, p, stream);
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

template<typename Scalar, bool MA, int MP>
hipError_t launch_bwd_mass_mp(const SegmentBwdJob &job, hipStream_t stream) {
    const SegmentJob &fj = job.fwd;
    int len = 0;
    const int nck = mass_replay_chunks(fj, job.maps_bytes, &len);
    const dim3 grid(static_cast<unsigned>(fj.B * fj.H), static_cast<unsigned>(nck));
    auto *maps = static_cast<float2 *>(job.maps);
    if (nck > 1) {
        hipLaunchKernelGGL((segment_bwd_mass_kernel<Scalar, MA, MP, false>), grid, dim3(kWave),
                           static_cast<size_t>(fj.A + 2) * 8, stream, job, maps, len);
        const int64_t n = static_cast<int64_t>(fj.B) * fj.H * fj.A;
        hipLaunchKernelGGL(segment_bwd_mass_scan_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                           stream, job, maps, nck);
    }
    hipLaunchKernelGGL((segment_bwd_mass_kernel<Scalar, MA, MP, true>), grid, dim3(kWave),
                       static_cast<size_t>(fj.A + 2) * 4, stream, job, maps, len);
    return hipGetLastError();
}

template<typename Scalar, bool MA>
hipError_t launch_bwd_mass(const SegmentBwdJob &job, hipStream_t stream) {
    const int kmax = std::max(job.fwd.Kw, job.fwd.Kr);
    if (kmax <= 32)
        return launch_bwd_mass_mp<Scalar, MA, 1>(job, stream);
    if (kmax <= 64)
        return launch_bwd_mass_mp<Scalar, MA, 2>(job, stream);
    return launch_bwd_mass_mp<Scalar, MA, 4>(job, stream);
}

template<typename Scalar>
hipError_t launch_typed(const SegmentBwdJob &job, const BwdPlan &p, hipStream_t stream) {
    hipError_t err = launch_bwd_scan<Scalar>(job, p, stream);
    if (err != hipSuccess)
        return err;
    const SegmentJob &fj = job.fwd;
    const int BH = fj.B * fj.H, KP = p.epp * p.np;
    const int t_pad = (fj.T + bwd_chunk(p.epp, p.np, p.vec) - 1) / bwd_chunk(p.epp, p.np, p.vec) * bwd_chunk(p.epp, p.np, p.vec);
    const int64_t nw = static_cast<int64_t>(BH) * fj.T * fj.Kw;
    const int64_t nr = static_cast<int64_t>(BH) * fj.T * fj.Kr;
    hipLaunchKernelGGL(segment_bwd_sum_kernel, dim3(static_cast<unsigned>((nw + 255) / 256)), dim3(256), 0, stream,
                       job.dg_part, job.dg_sum, p.n_sub, BH, fj.T, t_pad, KP, fj.Kw);
    hipLaunchKernelGGL(segment_bwd_sum_kernel, dim3(static_cast<unsigned>((nr + 255) / 256)), dim3(256), 0, stream,
                       job.dr_part, job.dr_sum, p.n_sub, BH, fj.T, t_pad, KP, fj.Kr);
    if ((err = hipGetLastError()) != hipSuccess)
        return err;
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

int64_t segment_backward_layout(int B, int H, int T, int A, int C, int Kw, int Kr, char *base, SegmentBwdJob *job,
                                bool saved) {
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
    char *wev = take(nw * 16), *rev = take(nr * 16);
    char *mass = take(bh * A * 4);
    const int64_t maps_bytes = mass_replay_scratch_bytes(B, H, T, A);
    char *maps = take(maps_bytes);
    const int64_t kp = p.epp * p.np, ch = bwd_chunk(p.epp, p.np, p.vec), t_pad = (T + ch - 1) / ch * ch;
    char *delta = saved ? nullptr : take(bh * p.n_sub * scan_t_pad64(T) * kp * p.csw * 4);
    char *dr = take(p.n_sub * bh * t_pad * kp * 4), *dg = take(p.n_sub * bh * t_pad * kp * 4);
    char *drs = take(nr * 4), *dgs = take(nw * 4);
    if (job) {
        job->aux = MassAux{reinterpret_cast<int4 *>(wev), reinterpret_cast<int4 *>(rev)};
        job->mass_scratch = reinterpret_cast<float *>(mass);
        job->maps = maps;
        job->maps_bytes = static_cast<size_t>(maps_bytes);
        if (!saved)
            job->delta = reinterpret_cast<float *>(delta);
        job->dr_part = reinterpret_cast<float *>(dr);
        job->dg_part = reinterpret_cast<float *>(dg);
        job->dr_sum = reinterpret_cast<float *>(drs);
        job->dg_sum = reinterpret_cast<float *>(dgs);
    }
    return off;
}

bool segment_saved_slices(int A, int C, int Kw, int Kr, SavedRows *geo) {
    BwdPlan p{};
    // whole slices only (the forward stores every channel of a slice), and one
    // pass of events (two-pass layouts would spill the saved read rows)
    if (!bwd_plan(A, C, Kw, Kr, &p) || C % p.csw != 0 || p.np != 1)
        return false;
    geo->w = geo->r = nullptr;
    geo->n_sub = p.n_sub;
    geo->kp = p.epp * p.np;
    geo->csw = p.csw;
    return true;
}

hipError_t launch_segment_backward(const SegmentBwdJob &job, hipStream_t stream, const char **why) {
    const SegmentJob &fj = job.fwd;
    if (static_cast<int64_t>(fj.B) * fj.H == 0)
        return hipSuccess;
    BwdPlan p{};
    if (!bwd_plan(fj.A, fj.C, fj.Kw, fj.Kr, &p)) {
        *why = "segment backward: shape outside the LDS-resident scan (top_k <= 128 and a slot slice in LDS: "
               "A <= 37870, or 34798 beyond 64 events)";
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
    if (!job.aux_saved) {
        SegmentJob mj = fj;
        mj.mass_out = job.mass_scratch;
        const hipError_t err = launch_mass_replay(mj, job.aux, job.maps, job.maps_bytes, stream);
        if (err != hipSuccess)
            return err;
    }
    switch (fj.dtype) {
        case kF32: return launch_typed<float>(job, p, stream);
        case kF16: return launch_typed<_Float16>(job, p, stream);
        case kBF16: return launch_typed<bf16_t>(job, p, stream);
        default: *why = "segment backward: unsupported dtype"; return hipErrorInvalidValue;
    }
}

}  // namespace ramnet
