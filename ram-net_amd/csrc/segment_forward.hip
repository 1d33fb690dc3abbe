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
// resident in LDS for the whole call (segment_scan.hpp). Channels of the GSU
// are independent, so slicing C gives every unit the complete read sum for
// its channels: no sort, no atomics, deterministic y, and the state crosses
// HBM exactly once in each direction.
//
// This file holds the planner: it picks the lane layout (events per pass,
// channels per lane) for top-K and the slice width that lets the most units
// share a CU's LDS, then dispatches to the per-dtype kernels. For wide slot
// spaces it can first run the mass pre-pass (segment_mass_kernel): the mass
// recurrence once per (b, h) instead of once per channel slice, which frees
// the LDS mass column so each slice holds twice the channels.
#include "ramnet_device.hpp"
#include "ramnet_kernels.hpp"
#include "segment_scan.hpp"
#include "segment_scan_pair.hpp"

#include <algorithm>
#include <atomic>
#include <climits>
#include <cstdio>
#include <cstdlib>

namespace ramnet {

namespace {

constexpr int64_t kLdsPerCu = 160 * 1024;
constexpr int64_t kLdsGranule = 512;

int pow2_ceil(int x) {
    int p = 1;
    while (p < x)
        p <<= 1;
    return p;
}

// CU count of the current device, looked up once per device. Concurrent
// first calls may both query the runtime; they store the same value.
constexpr int kCuCacheDevices = 64;
std::atomic<int> g_cu_count[kCuCacheDevices];

int cu_count() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0)
        return 256;
    const bool cacheable = dev < kCuCacheDevices;
    if (cacheable) {
        const int c = g_cu_count[dev].load(std::memory_order_relaxed);
        if (c > 0)
            return c;
    }
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
        return 256;
    if (cacheable)
        g_cu_count[dev].store(n, std::memory_order_relaxed);
    return n;
}

int dtype_bytes(int dtype) { return dtype == kF32 ? 4 : 2; }

struct Plan {
    int vec, epp, np, nw, cs;
    size_t lds;
    bool pre;     // mass pre-pass + precomputed-gain scan
    int nr = 1;   // slot ranges, scanned one launch each (precomputed-gain form)
    int tp = 1;   // tokens per wave step: 2 = the paired scan (precomputed-gain form, one range)
};

// Cost model of one layout, in cycles per token of one round of resident
// workgroups: a wave's token loop is bound by its dependency chain (LDS
// read -> update -> LDS write, ~kChainCycles) or by the issue of its VALU
// work (~10 + 6 * VEC * NP instructions, 4 cycles each, shared by the waves
// on one SIMD), whichever is longer. Total = T * rounds * per-token cycles.
// In the mass-wave form the mass wave's own chain (mass update, gain,
// staging: ~kMassWaveCycles per token) paces the state waves; the
// precomputed-gain form instead pays for its pre-pass, chunked over time
// across the GPU (~kPrePassCycles per token), plus its three extra launches
// (~kPrePassLaunchCycles, which decide short calls). Measured on MI355X.
constexpr int64_t kChainCycles = 160;
// The paired scan (two tokens per wave step, segment_scan_pair.hpp): its
// chain per pair, hazard steps included, per token, with one wave per SIMD
// and one channel per lane; a second channel per lane adds kPairVecCycles,
// each further wave sharing a SIMD kPairSharedCycles (they contend for the
// LDS, whose bank conflicts grow with the rows a pass touches), and the
// pre-pass's read-after-write flags kPairFlagCycles. Measured on MI355X, in
// the units of kChainCycles (one-token scan: ~190 cycles per token and
// round): config 4, 2 one-token waves per CU or 4 paired, scan 1.33 -> 1.06
// ms; config 2, 4 one-token waves per CU or 8 paired, 0.654 -> 0.67 ms, or 4
// paired with two channels per lane, 0.70 ms.
constexpr int64_t kPairChainCycles = 130;
constexpr int64_t kPairVecCycles = 40;
constexpr int64_t kPairSharedCycles = 35;
constexpr int64_t kPairFlagCycles = 15;
constexpr int64_t kMassWaveCycles = 230;
constexpr int64_t kPrePassCycles = 60;
constexpr int64_t kPrePassLaunchCycles = 45000;
// The mass pre-pass's replay keeps a head's masses in LDS ((A + 2) * 4
// bytes): up to A = 40958 in one piece, chunked over time; wider slot spaces
// run it per slot range of at most that many slots (segment_mass_range_kernel).
constexpr int64_t kMaxPrePassSlots = kLdsPerCu / 4 - 2;
// Its record-keeping mode (the segment backward) also holds a read tag and
// weight per slot, (A + 2) * 4 + (A + 1) * 8 bytes: A <= 13652 in one piece,
// slot ranges beyond.
constexpr int64_t kMaxAuxSlots = (kLdsPerCu - 16) / 12;
// Slot ranges of one scan: at most this many launches.
constexpr int kMaxScanRanges = 4096;
// The paired scan's pre-pass also keeps a tag per slot for its read-after-
// write flags: (A + 2) * 4 + (A + 3) * 4 bytes.
constexpr int64_t kMaxPairSlots = (kLdsPerCu - 20) / 8;
// The paired scan reads a head's gain records through a buffer resource of
// at most 2^31 - 1 bytes.
static bool pair_records_fit(int kmax, int T) {
    return static_cast<int64_t>(kmax) * scan_t_pad(std::max(T, 0)) * 16 <= INT_MAX;
}

// A forward that saves rows for the backward (SavedRows sv) runs a one-token
// precomputed-gain layout with one channel per lane and whole slices, whose
// event lanes fit in the backward's kp slots; a head's saved rows are
// addressed with 32-bit byte offsets.
static bool save_fits(const SavedRows &sv, int T) {
    return static_cast<int64_t>(sv.n_sub) * scan_t_pad(std::max(T, 1)) * sv.kp * sv.csw * 4 <= INT_MAX;
}
static bool save_layout_ok(const SavedRows *sv, int vec, int epp, int np, int cs, int C) {
    return !sv || (vec == 1 && epp * np <= sv->kp && C % cs == 0);
}

// The best layout for slot ranges of AL slots (the whole space when AL == A);
// forms: mass wave allowed (mass_ok), precomputed gains allowed (pre_ok);
// sv: the layout saves rows in those slices.
static bool plan_layout(int B, int H, int AL, int A_full, int C, int kmax, int elem, int n_cu, int T, bool mass_ok,
                        bool pre_ok, Plan *out, int64_t *best_cost, const SavedRows *sv = nullptr) {
    const int64_t tt = std::max(1, T);
    const int epp0 = std::min(kWave, std::max(4, pow2_ceil(kmax)));
    bool found = false;
    int64_t best = 0;
    // paired scan: the precomputed-gain form over the whole slot space, one
    // pass of events
    if (!sv && pre_ok && AL == A_full && AL <= kMaxPairSlots && pair_records_fit(kmax, T)) {
        for (int epp = 2; epp <= kWave / 2; epp <<= 1) {
            if (epp < kmax)
                continue;
            for (int nw = 8; nw >= 1; nw >>= 1) {
                for (int vec = 4; vec >= 1; vec >>= 1) {
                    if (!scan_pair_layout_compiled(vec, epp, nw))
                        continue;
                    const int cs = nw * (kWave / 2 / epp) * vec;
                    const size_t lds = scan_pair_lds_bytes(AL, vec, epp, nw, elem);
                    const int64_t gran = (static_cast<int64_t>(lds) + kLdsGranule - 1) / kLdsGranule * kLdsGranule;
                    if (gran > kLdsPerCu)
                        continue;
                    const int64_t units = static_cast<int64_t>(B) * H * ((C + cs - 1) / cs);
                    const int64_t per_cu = std::min<int64_t>(kLdsPerCu / gran, std::max(1, 16 / nw));
                    const int64_t rounds = (units + per_cu * n_cu - 1) / (per_cu * n_cu);
                    const int64_t resident = std::min<int64_t>(per_cu, (units + n_cu - 1) / n_cu);
                    const int64_t waves_per_simd = (resident * nw + 3) / 4;
                    // per token: half a pair's chain, or half its issue
                    const int64_t issue = 4 * (12 + 6 * vec) * waves_per_simd / 2;
                    const int64_t chain =
                        kPairChainCycles + kPairVecCycles * (vec - 1) + kPairSharedCycles * (waves_per_simd - 1);
                    int64_t cost = tt * rounds * std::max(chain, issue);
                    if (C % cs != 0)
                        cost = cost * 3 / 2;
                    cost += tt * (kPrePassCycles + kPairFlagCycles) + kPrePassLaunchCycles;
                    if (!found || cost < best) {
                        *out = {vec, epp, 1, nw, cs, lds, true};
                        out->tp = 2;
                        best = cost;
                        found = true;
                    }
                }
            }
        }
    }
    for (int pre = mass_ok ? 0 : 1; pre <= (pre_ok ? 1 : 0); ++pre) {
        for (int epp = 4; epp <= kWave; epp <<= 1) {
            const int np = (kmax + epp - 1) / epp;
            if (np > 2 || (np == 2 && epp * 2 < epp0))
                continue;
            for (int nw = 4; nw >= 1; nw >>= 1) {
                for (int vec = 4; vec >= 1; vec >>= 1) {
                    if (!scan_layout_compiled(vec, epp, np, nw, pre))
                        continue;
                    const int cs = nw * (kWave / epp) * vec;
                    if (!save_layout_ok(sv, vec, epp, np, cs, C))
                        continue;
                    const size_t lds = scan_lds_bytes(AL, vec, epp, np, nw, elem, pre);
                    const int64_t gran = (static_cast<int64_t>(lds) + kLdsGranule - 1) / kLdsGranule * kLdsGranule;
                    if (gran > kLdsPerCu)
                        continue;
                    const int64_t units = static_cast<int64_t>(B) * H * ((C + cs - 1) / cs);
                    const int64_t per_cu = std::min<int64_t>(kLdsPerCu / gran, std::max(1, 8 / nw));
                    const int64_t rounds = (units + per_cu * n_cu - 1) / (per_cu * n_cu);
                    const int64_t resident = std::min<int64_t>(per_cu, (units + n_cu - 1) / n_cu);
                    const int64_t waves_per_simd = (resident * nw + 3) / 4;
                    const int64_t issue = 4 * (10 + 6 * vec * np) * waves_per_simd;
                    int64_t cost = tt * rounds * std::max(pre ? kChainCycles : kMassWaveCycles, issue);
                    if (C % cs != 0)
                        cost = cost * 3 / 2;  // partial slices take the guarded path
                    if (pre)
                        cost += tt * kPrePassCycles + kPrePassLaunchCycles;
                    // ties: fewer channels per lane (less work per wave), then
                    // more waves, then wider slices
                    const bool better =
                        !found || cost < best ||
                        (cost == best && (vec < out->vec || (vec == out->vec && (nw > out->nw ||
                                                                                 (nw == out->nw && cs > out->cs)))));
                    if (better) {
                        *out = {vec, epp, np, nw, cs, lds, pre != 0};
                        out->tp = 1;
                        best = cost;
                        found = true;
                    }
                }
            }
        }
    }
    *best_cost = best;
    return found;
}

bool make_plan(int B, int H, int A, int C, int Kw, int Kr, int elem, int n_cu, int T, Plan *out,
               const SavedRows *sv = nullptr) {
    const int kmax = std::max(Kw, Kr);
    if (kmax > 2 * kWave || A < 1)
        return false;
    int64_t cost = 0;
    if (sv)  // saving rows: the precomputed-gain form over the whole slot space
        return A <= kMaxPrePassSlots && save_fits(*sv, T) &&
               plan_layout(B, H, A, A, C, kmax, elem, n_cu, T, false, true, out, &cost, sv);
    if (plan_layout(B, H, A, A, C, kmax, elem, n_cu, T, true, true, out, &cost))
        return true;
    // Too wide for one resident slice: split the slot space into the fewest
    // ranges that fit (precomputed-gain form), one launch per range. A slice
    // row holds at least one channel plus a pad (8 bytes), so no range is
    // wider than kLdsPerCu / 8 slots: the search starts at that bound.
    for (int nr = std::max(2, static_cast<int>(static_cast<int64_t>(A) * 8 / kLdsPerCu)); nr <= kMaxScanRanges;
         ++nr) {
        const int al = (A + nr - 1) / nr;
        if (plan_layout(B, H, al, A, C, kmax, elem, n_cu, T, false, true, out, &cost)) {
            out->nr = nr;
            return true;
        }
    }
    return false;
}

// Scan records from decoder outputs: one thread per (b*H + h, event, t) with
// t < T_pad. Writes keep positive weights; reads were stored negated. KF:
// write events compared per token for the overlap flags (8 or 16, >= Kw).
template<typename Scalar, int KF>
__global__ __launch_bounds__(256) void pack_records_kernel(const PackJob job, int t_pad) {
    // 32-bit index arithmetic: the host checks that B*H*T_pad*(Kw + Kr) fits
    // an int (a 64-bit division costs far more than the rest of a thread)
    const uint32_t Kt = static_cast<uint32_t>(job.Kw + job.Kr);
    const uint32_t n = static_cast<uint32_t>(job.B) * static_cast<uint32_t>(job.H) * Kt * static_cast<uint32_t>(t_pad);
    const uint32_t gid0 = blockIdx.x * blockDim.x + threadIdx.x;
    const bool in = gid0 < n;
    const uint32_t gid = in ? gid0 : n - 1;  // lanes past the end follow along (in the ballot)
    const uint32_t rest = gid / static_cast<uint32_t>(t_pad);
    const int t = static_cast<int>(gid - rest * static_cast<uint32_t>(t_pad));
    const uint32_t bhu = rest / Kt;
    const int k = static_cast<int>(rest - bhu * Kt);
    const int bh = static_cast<int>(bhu);
    const int b = bh / job.H;
    const int T = job.T, A = job.A;
    const int tl = t < T ? t : T - 1;
    const int64_t src = (static_cast<int64_t>(bh) * Kt + k) * T + tl;
    const int a = job.addr_idx[src] - bh * A;
    const float v = job.addr_val[src];
    const float g = load_f32(static_cast<const Scalar *>(job.gamma) + static_cast<int64_t>(bh) * T + tl);
    const uint8_t *mp = job.mask ? job.mask + static_cast<int64_t>(b) * T + tl : &kScanAllValid;
    const bool live = t < T && *mp != 0 && static_cast<unsigned>(a) < static_cast<unsigned>(A);
    // Event 0 carries the token's overlap flags, which the scan reads: bit
    // d - 1 set if a slot this token writes is also written by token t - d
    // (d = 1, 2, 3). Computed exactly for top-K up to 16 (assumed for wider
    // top-K), by whole waves: each lane reads the write slots of its own
    // token and of the three before it. Every load is issued
    // unconditionally from clamped indices (neighbouring lanes read the same
    // records, from cache): a load under a lane condition would be waited
    // for inside its branch, one round trip at a time.
    int ov = 7;
    if (__ballot(in && k == 0 && job.Kw <= 16) != 0) {
        // slot written by write event kk of token tt, or -1
        auto written = [&](int tt, int kk) {
            const int64_t s = (static_cast<int64_t>(bh) * Kt + kk) * T + tt;
            const int aa = job.addr_idx[s] - bh * A;
            return static_cast<unsigned>(aa) < static_cast<unsigned>(A) && job.addr_val[s] != 0.f ? aa : -1;
        };
        auto unmasked = [&](int tt) {
            const uint8_t *m = job.mask ? job.mask + static_cast<int64_t>(b) * T + tt : &kScanAllValid;
            return *m != 0;
        };
        const int kl = job.Kw - 1;
        int cur[KF];
        const bool mine = t < T && unmasked(tl);
#pragma unroll
        for (int i = 0; i < KF; ++i) {
            const int x = written(tl, min(i, kl));
            cur[i] = i < job.Kw && mine ? x : -1;
        }
        ov = 0;
#pragma unroll
        for (int d = 1; d <= 3; ++d) {
            const int tq = tl - d > 0 ? tl - d : 0;
            const bool theirs = t < T && t >= d && unmasked(tq);
            bool hit = false;
#pragma unroll
            for (int i = 0; i < KF; ++i) {
                int x = written(tq, min(i, kl));
                x = i < job.Kw && theirs ? x : -1;
#pragma unroll
                for (int j = 0; j < KF; ++j)
                    hit = hit || (x >= 0 && x == cur[j]);
            }
            if (hit)
                ov |= 1 << (d - 1);
        }
    }
    if (!in)
        return;
    if (k < job.Kw) {
        const bool act = live && v != 0.f;
        const float overlap = __int_as_float(k == 0 && job.Kw <= 16 ? ov : 7);
        WriteRec rec{-2, 0.f, 1.f, overlap};
        if (act)
            rec = WriteRec{a, v, gsu_alpha(v, g), overlap};
        job.wrec[(static_cast<int64_t>(bh) * job.Kw + k) * t_pad + t] = rec;
    } else {
        const float r = -v;
        const bool act = live && r != 0.f;
        job.rrec[(static_cast<int64_t>(bh) * job.Kr + (k - job.Kw)) * t_pad + t] = act ? ReadRec{a, r} : ReadRec{-1, 0.f};
    }
}

// The same records, one thread per (b*H + h, t) with t < T_pad, for top-K up
// to KE (8 or 16) on both sides: every load of a token -- its events, and
// the write events of the three tokens before it for the overlap flags -- is
// issued up front from clamped indices, then its Kw + Kr records are stored.
// A thread per event (above) leaves each thread one load and one store, so
// its waves sit on memory latency (config 2: 88 us a call).
template<typename Scalar, int KE>
__global__ __launch_bounds__(256) void pack_token_records_kernel(const PackJob job, int t_pad) {
    const uint32_t n = static_cast<uint32_t>(job.B) * static_cast<uint32_t>(job.H) * static_cast<uint32_t>(t_pad);
    const uint32_t gid0 = blockIdx.x * blockDim.x + threadIdx.x;
    if (gid0 >= n)
        return;
    const uint32_t bhu = gid0 / static_cast<uint32_t>(t_pad);
    const int t = static_cast<int>(gid0 - bhu * static_cast<uint32_t>(t_pad));
    const int bh = static_cast<int>(bhu);
    const int b = bh / job.H;
    const int T = job.T, A = job.A, Kw = job.Kw, Kr = job.Kr, Kt = Kw + Kr;
    const int tl = t < T ? t : T - 1;
    const int32_t *ip = job.addr_idx + static_cast<int64_t>(bh) * Kt * T;
    const float *vp = job.addr_val + static_cast<int64_t>(bh) * Kt * T;
    // Conditions below are bitwise: a short-circuit test of a lane value
    // becomes an exec-mask region (scalar instructions, and a boundary the
    // scheduler does not cross). Without a mask, the mask loads read bytes
    // of this head's indices instead (always in bounds) and are ignored.
    const bool has_mask = job.mask != nullptr;
    const uint8_t *mrow = has_mask ? job.mask + static_cast<int64_t>(b) * T : reinterpret_cast<const uint8_t *>(ip);
    auto unmasked = [&](int tt) { return !has_mask | (mrow[tt] != 0); };
    // this token's events (write events 0..Kw-1, then read events), clamped
    int ia[2 * KE];
    float va[2 * KE];
#pragma unroll
    for (int e = 0; e < 2 * KE; ++e) {
        // (offsets within the head fit 32 bits: the host checks B * H * T * (Kw + Kr))
        const int k = e < KE ? min(e, Kw - 1) : Kw + min(e - KE, Kr - 1);
        ia[e] = ip[static_cast<uint32_t>(k * T + tl)];
        va[e] = vp[static_cast<uint32_t>(k * T + tl)];
    }
    // the write slots of tokens t - 1, t - 2, t - 3 (clamped to token 0)
    int pa[3][KE];
    bool pon[3];
    float pv[3][KE];
#pragma unroll
    for (int d = 1; d <= 3; ++d) {
        const int tq = tl - d > 0 ? tl - d : 0;
        pon[d - 1] = (t < T) & (t >= d) & unmasked(tq);
#pragma unroll
        for (int e = 0; e < KE; ++e) {
            const int k = min(e, Kw - 1);
            pa[d - 1][e] = ip[static_cast<uint32_t>(k * T + tq)];
            pv[d - 1][e] = vp[static_cast<uint32_t>(k * T + tq)];
        }
    }
    const float g = load_f32(static_cast<const Scalar *>(job.gamma) + static_cast<int64_t>(bh) * T + tl);
    const bool live = (t < T) & unmasked(tl);
    const int base = bh * A;
    // slot written by event e (or `none`): in range, with a nonzero weight
    auto wslot = [&](bool on, int a, float v, int none) {
        const int o = a - base;
        return (on & (static_cast<unsigned>(o) < static_cast<unsigned>(A)) & (v != 0.f)) ? o : none;
    };
    // this token's write slots (-1: none) and, per token before, whether one
    // of them is written there too (its none, -2, never matches)
    int mine[KE];
#pragma unroll
    for (int j = 0; j < KE; ++j)
        mine[j] = wslot((j < Kw) & live, ia[j], va[j], -1);
    int ov = 0;
#pragma unroll
    for (int d = 0; d < 3; ++d) {
        bool hit = false;
#pragma unroll
        for (int i = 0; i < KE; ++i) {
            const int x = wslot((i < Kw) & pon[d], pa[d][i], pv[d][i], -2);
#pragma unroll
            for (int j = 0; j < KE; ++j)
                hit |= x == mine[j];
        }
        ov |= hit ? 1 << d : 0;
    }
    const float overlap = __int_as_float(ov);
    // this thread's records of event 0; event e is e * t_pad records further
    WriteRec *wr0 = job.wrec + static_cast<int64_t>(bh) * Kw * t_pad + t;
    ReadRec *rr0 = job.rrec + static_cast<int64_t>(bh) * Kr * t_pad + t;
#pragma unroll
    for (int e = 0; e < KE; ++e) {
        if (e < Kw) {
            const int a = ia[e] - base;
            const float v = va[e];
            const bool act = live & (static_cast<unsigned>(a) < static_cast<unsigned>(A)) & (v != 0.f);
            // alpha kept through an opaque bit mask (a select of the quotient
            // would be turned back into a branch around the division)
            const uint32_t m = opaque(act ? ~0u : 0u);
            const float al = __uint_as_float((__float_as_uint(gsu_alpha(v, g)) & m) | (__float_as_uint(1.f) & ~m));
            wr0[static_cast<uint32_t>(e * t_pad)] = WriteRec{act ? a : -2, act ? v : 0.f, al, overlap};
        }
    }
#pragma unroll
    for (int e = 0; e < KE; ++e) {
        if (e < Kr) {
            const int a = ia[KE + e] - base;
            const float r = -va[KE + e];  // reads were stored negated
            const bool act = live & (static_cast<unsigned>(a) < static_cast<unsigned>(A)) & (r != 0.f);
            rr0[static_cast<uint32_t>(e * t_pad)] = ReadRec{act ? a : -1, act ? r : 0.f};
        }
    }
}

// Mass pre-pass: the slot-mass recurrence (m <- alpha m + w per write
// event, in token order), once per (b, h) instead of once per channel
// slice. It writes the gain records of the precomputed-gain scan: per token
// and event, the write slot with its gain g = w / (m + eps) and the read
// slot with its weight (mass-aware: the effective weight
// (sum r) (m r) / (sum m r + eps) on the post-write masses). The decoder
// records are only read, so they can be scanned again.
//
// The sequence is cut into NC time chunks run in parallel. The recurrence is
// affine in m with coefficients independent of m, so:
//   1. mass_chunk_map_kernel: per (b, h, chunk), each slot's composed map
//      m_end = a m_start + b over the chunk (slots it does not touch: 1, 0);
//   2. mass_chunk_scan_kernel: per (b, h, slot), m_start of every chunk from
//      the initial mass and the maps in chunk order, and the final mass;
//   3. segment_mass_kernel: per (b, h, chunk), the chunk replayed from its
//      m_start, writing the gains.
// The maps live in a caller buffer (the scan's output y, which the scan
// overwrites afterwards); with NC = 1 step 3 alone runs, from the initial
// mass.
//
// Lanes 0..31 take write events p * 32 + lane, lanes 32..63 read events
// p * 32 + lane - 32; the masses (or maps) live in LDS, whose in-order
// accesses carry the slot dependency from token to token. Tokens go in pairs
// like the scan's mass wave: the second token's masses are read before the
// first token's writes and again only when the two write sets may overlap.
//
// Lanes past max(Kw, Kr) stand in for the last event lane of their half
// (same records, same results, same stores), so that every memory access of
// a token is made by the whole wave: no branch around a load or a store,
// which would make the compiler's memory-counter waits drain everything
// outstanding, the just-issued prefetch and the stores included.
// HALF: lanes per half (write lanes, then read lanes); 32, or fewer when a
// wave carries several (b, h) units, each on 2 * HALF consecutive lanes.
template<int MP, int HALF = 32>
struct MassLanes {
    static_assert(HALF == 32 || MP == 1, "units narrower than a wave take one pass of events");
    static constexpr int CH = MP <= 1 ? 16 : MP == 2 ? 8 : 4;  // tokens per fetch
    int ev[MP];    // this lane's event (clamped for loads)
    int evw[MP];   // its write event and read event, each clamped (every lane loads both)
    int evr[MP];
    bool on[MP];   // whether it is a real event
    bool act[MP];  // whether it acts: a real event, or a stand-in for the half's last event lane
    int es[MP];    // the event it stores (lanes past max(Kw, Kr) repeat the last one's store)
    bool wl;       // a write lane (else a read lane)
    __device__ MassLanes(int lane, int Kw, int Kr) {
        const int hl = lane % HALF;
        wl = (lane / HALF) % 2 == 0;
        const int ek = max(Kw, Kr);
#pragma unroll
        for (int p = 0; p < MP; ++p) {
            const int e = p * 32 + hl;
            es[p] = min(e, ek - 1);
            on[p] = wl ? e < Kw : e < Kr;
            act[p] = wl ? es[p] < Kw : es[p] < Kr;
            evw[p] = min(e, Kw - 1);
            evr[p] = min(e, Kr - 1);
            ev[p] = wl ? evw[p] : evr[p];
        }
    }
};
template<int MP, int CH>
struct MassRecs {
    int4 w[MP][CH];
    int2 r[MP][CH];
};
// The chunk's records from token t0 on: WONLY, the write record in every
// lane; else one 16-byte load per lane and token, the write record in the
// write lanes (c.w) and, in the read lanes, the aligned pair of read records
// holding token t's (c.r; t_pad is even and the rows 16-byte aligned).
template<bool WONLY, int MP, int CH, int HALF>
__device__ __forceinline__ void mass_fetch(const MassLanes<MP, HALF> &ln, const WriteRec *gw, const ReadRec *gr, int t_pad,
                                           int t0, MassRecs<MP, CH> &c) {
#pragma unroll
    for (int p = 0; p < MP; ++p) {
        if constexpr (WONLY) {
            // the chunk's groups start at multiples of CH from a multiple of
            // 16 and end by roundup(T, 8) <= t_pad: no clamp, so the tokens
            // are immediate offsets from one address per group
            const int4 *pw0 = reinterpret_cast<const int4 *>(gw + static_cast<int64_t>(ln.evw[p]) * t_pad + t0);
#pragma unroll
            for (int j = 0; j < CH; ++j)
                c.w[p][j] = pw0[j];
            continue;
        }
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            const int t = min(t0 + j, t_pad - 1);
            const WriteRec *pw = gw + static_cast<int64_t>(ln.evw[p]) * t_pad + t;
            {
                const ReadRec *pr = gr + static_cast<int64_t>(ln.evr[p]) * t_pad + (t & ~1);
                const int4 q = *reinterpret_cast<const int4 *>(ln.wl ? static_cast<const void *>(pw)
                                                                     : static_cast<const void *>(pr));
                c.w[p][j] = q;
                c.r[p][j] = (t & 1) ? make_int2(q.z, q.w) : make_int2(q.x, q.y);
            }
        }
    }
}

// Step 1: one wave per NU (b, h) units of one chunk (NU > 1: lanes as in
// the replay, unit u on lanes [u * 64 / NU, (u + 1) * 64 / NU), the units
// past the last (b, h) repeating it); LDS holds (a, b) per slot and unit.
template<int MP, int NU = 1>
__global__ __launch_bounds__(kWave) void mass_chunk_map_kernel(const SegmentJob job, float2 *maps, int t_pad,
                                                              int chunk_len) {
    static_assert(NU == 1 || MP == 1, "several units per wave: one pass of events");
    constexpr int HALF = kWave / NU / 2;
    using L = MassLanes<MP, HALF>;
    // half the replay's fetch: fewer registers, more resident waves to
    // cover the record loads' latency
    constexpr int CH = L::CH / 2;
    extern __shared__ __align__(16) float2 cm[];
    const int n_bh = job.B * job.H;
    const int ck = blockIdx.y, nck = gridDim.y;
    const int lane = static_cast<int>(threadIdx.x);
    const int bh = min(static_cast<int>(blockIdx.x) * NU + lane / (2 * HALF), n_bh - 1);
    const bool wlane = (lane / HALF) % 2 == 0;
    const int A = job.A, Kw = job.Kw, Kr = job.Kr;
    // unit v's maps at cm + v * (A + 2) + 2; [-2]: the no-op slot of padding records
    float2 *mp = cm + (lane / (2 * HALF)) * (A + 2) + 2;
    for (int a = lane; a < NU * (A + 2); a += kWave)
        cm[a] = make_float2(1.f, 0.f);
    __syncthreads();
    const L ln(lane, Kw, Kr);
    const WriteRec *gw = job.wrec + static_cast<int64_t>(bh) * Kw * t_pad;
    const ReadRec *gr = job.rrec + static_cast<int64_t>(bh) * Kr * t_pad;
    const int t_begin = ck * chunk_len, t_end = min(job.T, t_begin + chunk_len);
    const int nc = (t_end - t_begin + CH - 1) / CH;
    // Every lane of a unit holds a write record here: the read lanes and
    // the lanes past Kw hold a copy of one of the write lanes', so they read
    // and write the same map with the same values in the same instruction,
    // which changes nothing. Only tokens past the chunk's end (its last
    // group) act on the no-op slot.
    auto run = [&](int ci, const MassRecs<MP, CH> &c) {
        auto step = [&](auto tail_tag) {
            constexpr bool TL = decltype(tail_tag)::value;
            const int left = t_end - (t_begin + ci * CH);
#pragma unroll
            for (int j = 0; j < CH; ++j) {
#pragma unroll
                for (int p = 0; p < MP; ++p) {
                    const bool act = !TL || j < left;
                    const int a = act ? c.w[p][j].x : -2;
                    const float w = act ? __int_as_float(c.w[p][j].y) : 0.f;
                    const float al = act ? __int_as_float(c.w[p][j].z) : 1.f;
                    const float2 m = mp[a];
                    mp[a] = make_float2(al * m.x, fmaf(al, m.y, w));
                }
            }
        };
        if (t_begin + (ci + 1) * CH <= t_end)
            step(std::false_type{});
        else
            step(std::true_type{});
    };
    // a ring of three fetch buffers, two fetches ahead of the mass chain
    // (at config 2 the grid leaves half the SIMDs without a wave, so no
    // other wave covers the loads' latency); rotating in an unrolled loop,
    // as a copy of registers with loads pending would wait for every
    // outstanding load. Fetches past the last repeat it.
    auto at = [&](int i) { return t_begin + max(min(i, nc - 1), 0) * CH; };
    MassRecs<MP, CH> ca, cb, cc;
    mass_fetch<true>(ln, gw, gr, t_pad, at(0), ca);
    mass_fetch<true>(ln, gw, gr, t_pad, at(1), cb);
    for (int ci = 0; ci < nc; ci += 3) {
        mass_fetch<true>(ln, gw, gr, t_pad, at(ci + 2), cc);
        __builtin_amdgcn_sched_barrier(0);
        run(ci, ca);
        __builtin_amdgcn_sched_barrier(0);
        if (ci + 1 >= nc)
            break;
        mass_fetch<true>(ln, gw, gr, t_pad, at(ci + 3), ca);
        __builtin_amdgcn_sched_barrier(0);
        run(ci + 1, cb);
        __builtin_amdgcn_sched_barrier(0);
        if (ci + 2 >= nc)
            break;
        mass_fetch<true>(ln, gw, gr, t_pad, at(ci + 4), cb);
        __builtin_amdgcn_sched_barrier(0);
        run(ci + 2, cc);
        __builtin_amdgcn_sched_barrier(0);
    }
    __syncthreads();
#pragma unroll
    for (int v = 0; v < NU; ++v) {
        const int bv = min(static_cast<int>(blockIdx.x) * NU + v, n_bh - 1);
        const float2 *mv = cm + v * (A + 2) + 2;
        float2 *dst = maps + (static_cast<int64_t>(bv) * nck + ck) * A;
        for (int a = lane; a < A; a += kWave)
            dst[a] = mv[a];
    }
}

// Step 2: one thread per (b, h, slot); the map of chunk c is replaced by
// (m_start of chunk c, unused).
__global__ __launch_bounds__(256) void mass_chunk_scan_kernel(const SegmentJob job, float2 *maps, int nck) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int A = job.A;
    if (i >= static_cast<int64_t>(job.B) * job.H * A)
        return;
    const int64_t bh = i / A;
    const int a = static_cast<int>(i - bh * A);
    float m = job.init_mass[i];
    float2 *mp = maps + bh * nck * A + a;
    // eight chunks' maps loaded before their stores (a store could alias a
    // later load as far as the compiler knows, so one at a time each load
    // would wait for the store before it)
    for (int c0 = 0; c0 < nck; c0 += 8) {
        float2 ab[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            ab[j] = mp[static_cast<int64_t>(min(c0 + j, nck - 1)) * A];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (c0 + j < nck) {
                mp[static_cast<int64_t>(c0 + j) * A] = make_float2(m, 0.f);
                m = fmaf(ab[j].x, m, ab[j].y);
            }
        }
    }
    job.mass_out[i] = m;
}

// Step 3: one wave per NU (b, h) units of one chunk, from m_start (the maps
// after step 2, or the initial mass when there is one chunk). AUX = 0: the
// gain records; AUX = 1: the per-event quantities of `aux` instead (the
// forward replay of the segment backward); AUX = 2: both (a forward that
// saves them for its backward). NU > 1 (at most 32 / NU
// events per token): unit u takes lanes [u * 64 / NU, (u + 1) * 64 / NU),
// so every lane of a record load or gain store serves an event; the units
// past the last (b, h) repeat it (same records, same values stored).
// FL: also the read-after-write flags of the paired scan (job.flags): per
// token, whether one of its write slots is a read slot of the token before.
// Each token's reads post the token under their slots in an LDS tag table;
// the next token's writes look their slots up. The first token of a chunk
// (whose predecessor another chunk replays) is flagged.
template<bool MA, int MP, int AUX = 0, int NU = 1, bool FL = false>
__global__ __launch_bounds__(kWave) void segment_mass_kernel(const SegmentJob job, int t_pad, int chunk_len,
                                                            const float2 *starts, const MassAux aux) {
    static_assert(NU == 1 || (MP == 1 && !AUX), "several units per wave: one pass of events, no AUX");
    static_assert(!(FL && AUX), "flags: the forward pre-pass only");
    constexpr int HALF = kWave / NU / 2;
    using L = MassLanes<MP, HALF>;
    // half the fetch of the records: fewer registers, more resident waves
    constexpr int CH = L::CH / 2;
    extern __shared__ __align__(16) float lds[];
    const int n_bh = job.B * job.H;
    const int ck = blockIdx.y, nck = gridDim.y;
    const int lane = static_cast<int>(threadIdx.x);
    const int unit = lane / (2 * HALF);
    const int bh = min(static_cast<int>(blockIdx.x) * NU + unit, n_bh - 1);
    const int hl = lane % HALF;
    const bool wlane = (lane / HALF) % 2 == 0;
    const int A = job.A, Kw = job.Kw, Kr = job.Kr;
    const float eps = job.eps;
    // unit v's masses at lds + v * (A + 2) + 2; [-2], [-1]: the no-op slots of padding records
    float *ms = lds + unit * (A + 2) + 2;
#pragma unroll
    for (int v = 0; v < NU; ++v) {
        const int bv = min(static_cast<int>(blockIdx.x) * NU + v, n_bh - 1);
        float *mv = lds + v * (A + 2) + 2;
        if (starts) {
            const float2 *src = starts + (static_cast<int64_t>(bv) * nck + ck) * A;
            for (int a = lane; a < A; a += kWave)
                mv[a] = src[a].x;
        } else {
            const float *src = job.init_mass + static_cast<int64_t>(bv) * A;
            for (int a = lane; a < A; a += kWave)
                mv[a] = src[a];
        }
        if (lane < 2)
            mv[lane - 2] = 1.f;
    }
    // AUX: per slot of unit v, the token whose read last posted there and its
    // weight (tables of A after the NU units' masses)
    int *rtag = reinterpret_cast<int *>(lds + NU * (A + 2)) + unit * A;
    float *rval = lds + NU * (A + 2) + NU * A + unit * A;
    if constexpr (AUX) {
        int *rtags = reinterpret_cast<int *>(lds + NU * (A + 2));
        for (int a = lane; a < NU * A; a += kWave)
            rtags[a] = -1;
    }
    // FL: unit v's tags at ftag + v * (A + 3) + 3: [-2] where no-op writes
    // look (never posted), [-1] where no-op reads post ([-3] unused)
    int *ftag = reinterpret_cast<int *>(lds + NU * (A + 2));
    int *tg = ftag + unit * (A + 3) + 3;
    if constexpr (FL) {
        for (int a = lane; a < NU * (A + 3); a += kWave)
            ftag[a] = INT_MIN;
    }
    __syncthreads();

    const L ln(lane, Kw, Kr);
    const WriteRec *gw = job.wrec + static_cast<int64_t>(bh) * Kw * t_pad;
    const ReadRec *gr = job.rrec + static_cast<int64_t>(bh) * Kr * t_pad;
    // gain records of this head (not written in the record-keeping mode)
    const int ek = max(Kw, Kr);
    GainRec *gg = AUX == 1 ? nullptr : job.gain + static_cast<int64_t>(bh) * ek * t_pad;
    const int t_begin = ck * chunk_len, t_end = min(job.T, t_begin + chunk_len);
    int *gfl = FL ? job.flags + static_cast<int64_t>(bh) * t_pad : nullptr;
    auto run = [&](int t0, const MassRecs<MP, CH> &c) {
        // FL: per token of the chunk, the tag each pass's write slot holds
        // (compared once the chunk is done, off the mass chain)
        int tgv[CH][MP];
        auto wev = [&](int p, int j, int &a, float &w, float &al) {
            const bool act = wlane & ln.act[p] & (t0 + j < t_end);  // bitwise: no exec-mask region
            a = act ? c.w[p][j].x : -2;
            w = act ? __int_as_float(c.w[p][j].y) : 0.f;
            al = act ? __int_as_float(c.w[p][j].z) : 1.f;
        };
        auto finish = [&](int j, const int (&a)[MP], const float (&w)[MP], const float (&al)[MP], float (&m)[MP]) {
            const int t = t0 + j;
            const bool live = t < t_end;
            int rb[MP];
#pragma unroll
            for (int p = 0; p < MP; ++p) {
                const bool act = !wlane & ln.act[p] & live;
                rb[p] = act ? c.r[p][j].x : -1;
            }
            if constexpr (FL) {
                // the tags this token's write slots hold, before its own
                // reads post theirs (read lanes look at a slot never posted).
                // The tags are posted by other lanes (the read lanes of the
                // token before, and of this token): the barriers keep the
                // compiler from moving these loads above the one's stores or
                // below the other's.
                __builtin_amdgcn_wave_barrier();
#pragma unroll
                for (int p = 0; p < MP; ++p)
                    tgv[j][p] = tg[wlane ? a[p] : -2];
                __builtin_amdgcn_wave_barrier();
            }
            float gn[MP];
#pragma unroll
            for (int p = 0; p < MP; ++p) {
                const float m2 = fmaf(al[p], m[p], w[p]);
                if constexpr (FL) {
                    // one store: the write lanes' masses, the read lanes' tags
                    float *dst = wlane ? &ms[a[p]] : reinterpret_cast<float *>(&tg[rb[p]]);
                    *dst = wlane ? m2 : __int_as_float(t);
                } else {
                    ms[a[p]] = m2;
                }
                gn[p] = scan_gain(w[p], m2 + eps);
            }
            // (FL: the read lanes stored their tags, not into the masses,
            // above; the barrier keeps their post-write mass loads below
            // the write lanes' mass stores)
            if constexpr (FL && MA)
                __builtin_amdgcn_wave_barrier();
            {
                float rr[MP], mm[MP];
                float sr = 0.f, srm = 0.f;
#pragma unroll
                for (int p = 0; p < MP; ++p) {
                    const bool act = !wlane & ln.act[p] & live;
                    rr[p] = act ? __int_as_float(c.r[p][j].y) : 0.f;
                    mm[p] = 0.f;
                    if constexpr (MA || AUX) {
                        mm[p] = ms[rb[p]];  // post-write mass
                        const float rs = ln.on[p] ? rr[p] : 0.f;  // stand-ins add nothing
                        sr += rs;
                        srm += rs * mm[p];
                    }
                }
                float scale = 1.f;
                if constexpr (MA) {
                    sr = event_sum<HALF>(sr);
                    srm = event_sum<HALF>(srm);
                    scale = sr / (srm + eps);
                }
                float re[MP];
#pragma unroll
                for (int p = 0; p < MP; ++p) {
                    re[p] = MA ? rr[p] * mm[p] * scale : rr[p];
                    if constexpr (AUX != 1) {
                        // every event below max(Kw, Kr) gets a record (past Kw
                        // the no-op write: slot -2, gain 0; past Kr the no-op
                        // read: slot -1, weight 0); write lanes store its first
                        // half, read lanes its second. Tokens past the end
                        // store no-op records into the padding rows.
                        int2 *dst = reinterpret_cast<int2 *>(&gg[static_cast<int64_t>(t) * ek + ln.es[p]]) + (wlane ? 0 : 1);
                        *dst = wlane ? make_int2(a[p], __float_as_int(gn[p])) : make_int2(rb[p], __float_as_int(re[p]));
                    }
                }
                if constexpr (AUX) {
                    // each write's record carries the effective weight of the read of
                    // the same slot in this token (0 if none): the reads post
                    // (token, weight) under their slots, then the writes look up theirs.
                    // Other lanes post what a lane looks up: the barriers keep the
                    // compiler from moving the lookups above the posts (or this
                    // token's posts above the previous token's lookups).
                    __builtin_amdgcn_wave_barrier();
#pragma unroll
                    for (int p = 0; p < MP; ++p) {
                        if (!wlane & (rb[p] >= 0)) {
                            rtag[rb[p]] = t;
                            rval[rb[p]] = re[p];
                        }
                    }
                    __builtin_amdgcn_wave_barrier();
                    float rmatch[MP];
#pragma unroll
                    for (int p = 0; p < MP; ++p) {
                        // (bitwise, both tables read on every lane: a
                        // short-circuit LDS read would be an exec-mask region
                        // waiting on its own load)
                        const int sl = a[p] < 0 ? 0 : a[p];
                        const bool hit = wlane & (a[p] >= 0) & (rtag[sl] == t);
                        const float rv = rval[sl];
                        rmatch[p] = hit ? rv : 0.f;
                    }
                    // one store per event for both halves: the write lanes' record
                    // into wev, the read lanes' into rev
#pragma unroll
                    for (int p = 0; p < MP; ++p) {
                        const int64_t tb = static_cast<int64_t>(bh) * job.T + t;
                        int4 *dst = wlane ? aux.wev + tb * Kw + ln.ev[p] : aux.rev + tb * Kr + ln.ev[p];
                        const int4 rec = wlane ? make_int4(a[p], __float_as_int(gn[p]), __float_as_int(rmatch[p]),
                                                           __float_as_int(m[p]))
                                               : make_int4(rb[p], __float_as_int(re[p]), __float_as_int(mm[p]), 0);
                        if (ln.on[p] & live)
                            *dst = rec;
                    }
                }
            }
        };
#pragma unroll
        for (int j0 = 0; j0 < CH; j0 += 2) {
            const int j1 = j0 + 1;
            // token j1 shares a slot with token j0 (in any unit: event 0's record carries the flag)
            int ov;
            if constexpr (NU == 1)
                ov = __builtin_amdgcn_readfirstlane(c.w[0][j1].w) & 1;
            else
                ov = __ballot(lane % (2 * HALF) == 0 && (c.w[0][j1].w & 1) != 0) != 0;
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
        if constexpr (FL) {
            // per token: a hit in any write lane of this lane's unit; lane hl
            // stores token t0 + hl's flag (lanes past the chunk's tokens
            // repeat the last one's store)
            const int ubase = unit * 2 * HALF;
            uint32_t rwm = 0;
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                bool hit = false;
#pragma unroll
                for (int p = 0; p < MP; ++p)
                    hit |= wlane & ln.on[p] & (tgv[j][p] == t0 + j - 1);
                const uint64_t hb = __ballot(hit);
                const bool unit_hit = ((hb >> ubase) & ((1ull << HALF) - 1)) != 0;
                const bool first = t0 + j == t_begin && t_begin > 0;
                rwm |= unit_hit || first ? 1u << j : 0u;
            }
            const int jj = min(hl, min(CH, t_end - t0) - 1);
            gfl[t0 + jj] = static_cast<int>((rwm >> jj) & 1u);
        }
    };
    const int nc = (t_end - t_begin + CH - 1) / CH;
    // the loads stay two fetches ahead of the mass chain: a ring of three
    // buffers rotating in an unrolled loop (no copy of pending loads);
    // fetches past the last repeat it
    auto at = [&](int i) { return t_begin + max(min(i, nc - 1), 0) * CH; };
    MassRecs<MP, CH> ca, cb, cc;
    mass_fetch<false>(ln, gw, gr, t_pad, at(0), ca);
    mass_fetch<false>(ln, gw, gr, t_pad, at(1), cb);
    for (int ci = 0; ci < nc; ci += 3) {
        mass_fetch<false>(ln, gw, gr, t_pad, at(ci + 2), cc);
        __builtin_amdgcn_sched_barrier(0);
        run(t_begin + ci * CH, ca);
        __builtin_amdgcn_sched_barrier(0);
        if (ci + 1 >= nc)
            break;
        mass_fetch<false>(ln, gw, gr, t_pad, at(ci + 3), ca);
        __builtin_amdgcn_sched_barrier(0);
        run(t_begin + (ci + 1) * CH, cb);
        __builtin_amdgcn_sched_barrier(0);
        if (ci + 2 >= nc)
            break;
        mass_fetch<false>(ln, gw, gr, t_pad, at(ci + 4), cb);
        __builtin_amdgcn_sched_barrier(0);
        run(t_begin + (ci + 2) * CH, cc);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (!starts) {
        __syncthreads();
#pragma unroll
        for (int v = 0; v < NU; ++v) {
            const int bv = min(static_cast<int>(blockIdx.x) * NU + v, n_bh - 1);
            const float *mv = lds + v * (A + 2) + 2;
            float *mdst = job.mass_out + static_cast<int64_t>(bv) * A;
            for (int a = lane; a < A; a += kWave)
                mdst[a] = mv[a];
        }
    }
}

// Time chunks of the mass passes: about kMassChunkTokens tokens each, or
// shorter (down to 64 tokens) until the (b, h, chunk) waves put one wave on
// every SIMD. Measured on MI355X, mass pre-pass + scan: config 2 (128
// heads, T = 4096) 0.81 ms at chunks of 128 tokens, 0.79 at 256, 0.81 at
// 512; config 4 (32 heads, T = 8192) 1.44 at 64 and 128, 1.42 at 256. The
// training step's backward replay is also fastest at 256.
constexpr int kReplayChunkFactor = 1;
constexpr int kMassChunkTokens = 256;

// Chunks of the mass pre-pass: as above, chunks a multiple of 16 tokens,
// and maps that fit the scratch buffer.
int mass_chunks(const SegmentJob &job, size_t scratch_bytes, int n_cu, int *chunk_len) {
    const int64_t bh = static_cast<int64_t>(job.B) * job.H;
    const int fill = static_cast<int>(std::min<int64_t>((4 * n_cu + bh - 1) / bh, std::max(1, job.T / 64)));
    int nck = std::max((job.T + kMassChunkTokens - 1) / kMassChunkTokens, std::max(1, fill));
    while (nck > 1 && static_cast<size_t>(bh) * nck * job.A * sizeof(float2) > scratch_bytes)
        nck /= 2;
    if (static_cast<int64_t>(job.A + 2) * 8 > kLdsPerCu)
        nck = 1;  // a chunk's maps do not fit in LDS (A > 20478): one serial replay
    const int len = ((job.T + nck - 1) / nck + 15) / 16 * 16;
    *chunk_len = std::max(16, len);
    return (job.T + *chunk_len - 1) / *chunk_len;
}

// LDS of the replay kernel: the masses of its NU units (and with AUX the
// read tag table, with FL the flag tag tables).
size_t mass_lds_bytes(int A, bool aux, int nu = 1, bool fl = false) {
    return static_cast<size_t>(A + 2) * 4 * nu + (aux ? static_cast<size_t>(A) * 8 * nu : 0) +
           (fl ? static_cast<size_t>(A + 3) * 4 * nu : 0);
}

// The replay kernel with NU units per wave: (b, h) units of a chunk in
// groups of NU.
template<bool MA, int MP, int AUX, int NU>
void launch_replay_units(const SegmentJob &job, int t_pad, int len, int nck, const float2 *starts, const MassAux &aux,
                         hipStream_t stream) {
    const unsigned groups = static_cast<unsigned>((job.B * job.H + NU - 1) / NU);
    const bool fl = !AUX && job.flags;
    const dim3 grid(groups, static_cast<unsigned>(nck));
    if constexpr (!AUX) {
        if (fl) {
            hipLaunchKernelGGL((segment_mass_kernel<MA, MP, AUX, NU, true>), grid, dim3(kWave),
                               mass_lds_bytes(job.A, false, NU, true), stream, job, t_pad, len, starts, aux);
            return;
        }
    }
    hipLaunchKernelGGL((segment_mass_kernel<MA, MP, AUX, NU>), grid, dim3(kWave), mass_lds_bytes(job.A, AUX != 0, NU),
                       stream, job, t_pad, len, starts, aux);
}

// Units per replay wave: four when a token has at most 8 events and the
// four units' masses take at most 64 KB of LDS, else one (the record-keeping
// modes, bound by their record stores, measured no faster with four). Measured on
// MI355X: config 2 (K = 8) segment stage 0.762 -> 0.755 ms with four units;
// config 4 (K = 16) 1.420 -> 1.433 ms with two (so one there), and both
// slower with the time chunks halved to keep the wave count.
template<bool MA, int MP, int AUX>
void launch_mass_replay_nu(const SegmentJob &job, int t_pad, int len, int nck, const float2 *starts,
                           const MassAux &aux, hipStream_t stream) {
    if constexpr (MP == 1 && !AUX) {
        if (std::max(job.Kw, job.Kr) <= 8 && mass_lds_bytes(job.A, false, 4, job.flags != nullptr) <= 64 * 1024)
            return launch_replay_units<MA, MP, AUX, 4>(job, t_pad, len, nck, starts, aux, stream);
    }
    launch_replay_units<MA, MP, AUX, 1>(job, t_pad, len, nck, starts, aux, stream);
}

// `maps` is scratch for the chunk maps (maps_bytes of it); the final masses
// go to job.mass_out.
template<bool MA, int MP, int AUX>
hipError_t launch_mass_pass_mp(const SegmentJob &job, int t_pad, int n_cu, void *maps_buf, size_t maps_bytes,
                               const MassAux &aux, hipStream_t stream) {
    int len = 0;
    const int nck = mass_chunks(job, maps_bytes, n_cu, &len);
    const unsigned bh = static_cast<unsigned>(job.B * job.H);
    if (nck <= 1) {
        launch_mass_replay_nu<MA, MP, AUX>(job, t_pad, job.T, 1, nullptr, aux, stream);
        return hipGetLastError();
    }
    auto *maps = static_cast<float2 *>(maps_buf);
    if (MP == 1 && std::max(job.Kw, job.Kr) <= 8 && static_cast<size_t>(job.A + 2) * 8 * 4 <= 64 * 1024)
        hipLaunchKernelGGL((mass_chunk_map_kernel<1, 4>), dim3((bh + 3) / 4, nck), dim3(kWave),
                           static_cast<size_t>(job.A + 2) * 8 * 4, stream, job, maps, t_pad, len);
    else
        hipLaunchKernelGGL((mass_chunk_map_kernel<MP>), dim3(bh, nck), dim3(kWave),
                           static_cast<size_t>(job.A + 2) * 8, stream, job, maps, t_pad, len);
    const int64_t n = static_cast<int64_t>(bh) * job.A;
    hipLaunchKernelGGL(mass_chunk_scan_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, stream, job,
                       maps, nck);
    launch_mass_replay_nu<MA, MP, AUX>(job, t_pad, len, nck, maps, aux, stream);
    return hipGetLastError();
}

// Wide slot spaces: the mass pre-pass of one slot range [r0, r0 + AL) of
// every (b, h), one wave per (b, h) over the whole sequence (no time
// chunks), launched once per range in range order. The range's masses live
// in LDS; events on other slots act on the no-op slots. Every range sees
// every event, and each event's output is written by one range: the write
// half by the range holding the write slot, the read half by the range
// holding the read slot, and the halves of no-op events (slot < 0: masked,
// inactive, or past top-k) by range 0. Mass-aware reads store r m (m: the
// post-write mass of their slot); mass_read_scale_kernel turns them into
// effective weights once every range has run. Lanes as in
// segment_mass_kernel: write events on lanes 0..31, read events on 32..63.
// The forward (AUX false) writes gain records and runs beyond
// kMaxPrePassSlots; the record-keeping mode of the segment backward (AUX
// true: the per-event quantities of MassAux, with the tag table that matches
// each write to the same token's read of its slot) runs beyond
// kMaxAuxSlots.
template<bool MA, int MP, bool AUX>
__global__ __launch_bounds__(kWave) void segment_mass_range_kernel(const SegmentJob job, int t_pad, int r0, int AL,
                                                                  const MassAux aux) {
    using L = MassLanes<MP>;
    constexpr int CH = L::CH;
    extern __shared__ __align__(16) float lds[];
    const int bh = static_cast<int>(blockIdx.x);
    const int lane = static_cast<int>(threadIdx.x);
    const int hl = lane % 32;
    const int A = job.A, Kw = job.Kw, Kr = job.Kr, T = job.T;
    const float eps = job.eps;
    float *ms = lds + 2;  // ms[-2], ms[-1]: the no-op slots
    // AUX: per slot, the token whose read last posted there and its weight
    // ([-1]: where lanes without a read post)
    int *rtag = reinterpret_cast<int *>(lds + AL + 2) + 1;
    float *rval = lds + 2 * AL + 4;
    {
        const float *src = job.init_mass + static_cast<int64_t>(bh) * A + r0;
        for (int a = lane; a < AL; a += kWave)
            ms[a] = src[a];
        if (lane < 2)
            lds[lane] = 1.f;
        if constexpr (AUX) {
            for (int a = lane - 1; a < AL; a += kWave)
                rtag[a] = -1;
        }
    }
    __syncthreads();
    const L ln(lane, Kw, Kr);
    const WriteRec *gw = job.wrec + static_cast<int64_t>(bh) * Kw * t_pad;
    const ReadRec *gr = job.rrec + static_cast<int64_t>(bh) * Kr * t_pad;
    const int ek = max(Kw, Kr);
    GainRec *gg = AUX ? nullptr : job.gain + static_cast<int64_t>(bh) * ek * t_pad;
    const bool first = r0 == 0;
    for (int t0 = 0; t0 < T; t0 += CH) {
        MassRecs<MP, CH> c;
        mass_fetch<false>(ln, gw, gr, t_pad, t0, c);
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            const int t = t0 + j;
            if (t >= T)
                break;
            // writes of token t on the range's slots
            int wa[MP], wl[MP];
            bool win[MP];
            float gn[MP], mb[MP];
#pragma unroll
            for (int p = 0; p < MP; ++p) {
                wa[p] = ln.wl && ln.on[p] ? c.w[p][j].x : -2;
                const int loc = wa[p] - r0;
                win[p] = wa[p] >= 0 && static_cast<unsigned>(loc) < static_cast<unsigned>(AL);
                wl[p] = win[p] ? loc : -2;
                const float w = win[p] ? __int_as_float(c.w[p][j].y) : 0.f;
                const float al = win[p] ? __int_as_float(c.w[p][j].z) : 1.f;
                mb[p] = ms[wl[p]];
                const float m2 = fmaf(al, mb[p], w);
                ms[wl[p]] = m2;
                gn[p] = scan_gain(w, m2 + eps);
            }
            // then its reads (LDS keeps the wave's accesses in order: the
            // masses read are the post-write ones)
            int rb[MP], rl[MP];
            bool rin[MP];
            float re[MP], mr[MP];
#pragma unroll
            for (int p = 0; p < MP; ++p) {
                rb[p] = !ln.wl && ln.on[p] ? c.r[p][j].x : -1;
                const int loc = rb[p] - r0;
                rin[p] = rb[p] >= 0 && static_cast<unsigned>(loc) < static_cast<unsigned>(AL);
                rl[p] = rin[p] ? loc : -1;
                const float r = rin[p] ? __int_as_float(c.r[p][j].y) : 0.f;
                mr[p] = MA || AUX ? ms[rl[p]] : 1.f;
                re[p] = MA ? r * mr[p] : r;
                if constexpr (AUX) {
                    rtag[rl[p]] = t;
                    rval[rl[p]] = re[p];
                }
            }
#pragma unroll
            for (int p = 0; p < MP; ++p) {
                const int e = p * 32 + hl;
                if constexpr (AUX) {
                    // the weight of this token's read of the write's slot, if any
                    const int sl = win[p] ? wl[p] : -1;
                    const float rmatch = win[p] && rtag[sl] == t ? rval[sl] : 0.f;
                    const int64_t tb = static_cast<int64_t>(bh) * T + t;
                    if (ln.wl) {
                        if (e < Kw && (wa[p] >= 0 ? win[p] : first))
                            aux.wev[tb * Kw + e] = make_int4(wa[p] >= 0 ? wa[p] : -2, __float_as_int(gn[p]),
                                                             __float_as_int(rmatch), __float_as_int(mb[p]));
                    } else if (e < Kr && (rb[p] >= 0 ? rin[p] : first)) {
                        aux.rev[tb * Kr + e] = make_int4(rb[p] >= 0 ? rb[p] : -1, __float_as_int(re[p]),
                                                         __float_as_int(mr[p]), 0);
                    }
                } else if (e < ek) {
                    int2 *dst = reinterpret_cast<int2 *>(&gg[static_cast<int64_t>(t) * ek + e]) + (ln.wl ? 0 : 1);
                    if (ln.wl) {
                        if (wa[p] >= 0 ? win[p] : first)
                            *dst = make_int2(wa[p] >= 0 ? wa[p] : -2, __float_as_int(wa[p] >= 0 ? gn[p] : 0.f));
                    } else if (rb[p] >= 0 ? rin[p] : first) {
                        *dst = make_int2(rb[p] >= 0 ? rb[p] : -1, __float_as_int(rb[p] >= 0 ? re[p] : 0.f));
                    }
                }
            }
        }
    }
    __syncthreads();
    float *mdst = job.mass_out + static_cast<int64_t>(bh) * A + r0;
    for (int a = lane; a < AL; a += kWave)
        mdst[a] = ms[a];
}

// Mass-aware reads after the ranged pre-pass: per (b, h, token), with S_r the
// sum of the token's read weights and S_m the sum of the stored r m, each
// read's effective weight is r m S_r / (S_m + eps), as the chunked pre-pass
// computes it. AUX: the same for the backward's per-event records (the read
// weights and each write's matched read weight).
template<bool AUX>
__global__ __launch_bounds__(256) void mass_read_scale_kernel(const SegmentJob job, int t_pad, const MassAux aux) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<int64_t>(job.B) * job.H * job.T)
        return;
    const int64_t bh = i / job.T;
    const int t = static_cast<int>(i - bh * job.T);
    const int Kw = job.Kw, Kr = job.Kr, ek = max(Kw, Kr);
    const ReadRec *rr = job.rrec + bh * Kr * t_pad + t;
    float sr = 0.f, sm = 0.f;
    if constexpr (AUX) {
        int4 *rv = aux.rev + i * Kr;
        for (int k = 0; k < Kr; ++k) {
            sr += rr[static_cast<int64_t>(k) * t_pad].r;
            sm += __int_as_float(rv[k].y);
        }
        const float scale = sr / (sm + job.eps);
        for (int k = 0; k < Kr; ++k)
            rv[k].y = __float_as_int(__int_as_float(rv[k].y) * scale);
        int4 *wv = aux.wev + i * Kw;
        for (int k = 0; k < Kw; ++k)
            wv[k].z = __float_as_int(__int_as_float(wv[k].z) * scale);
    } else {
        GainRec *g = job.gain + (bh * t_pad + t) * ek;
        for (int k = 0; k < Kr; ++k) {
            sr += rr[static_cast<int64_t>(k) * t_pad].r;
            sm += g[k].r;
        }
        const float scale = sr / (sm + job.eps);
        for (int k = 0; k < Kr; ++k)
            g[k].r *= scale;
    }
}

// The pre-pass in slot ranges of at most `max_al` slots, in order, then the
// mass-aware read weights.
template<bool AUX>
hipError_t launch_mass_ranges(const SegmentJob &job, int t_pad, int64_t max_al, const MassAux &aux,
                              hipStream_t stream) {
    const int nr = static_cast<int>((job.A + max_al - 1) / max_al);
    const int al = (job.A + nr - 1) / nr;
    const int kmax = std::max(job.Kw, job.Kr);
    const dim3 grid(static_cast<unsigned>(job.B * job.H));
    for (int r = 0; r < nr; ++r) {
        const int r0 = r * al, n = std::min(al, job.A - r0);
        const size_t lds = static_cast<size_t>(n + 2) * 4 + (AUX ? static_cast<size_t>(n + 1) * 8 : 0);
#define RAMNET_MASS_RANGE(MA, MP) \
    hipLaunchKernelGGL((segment_mass_range_kernel<MA, MP, AUX>), grid, dim3(kWave), lds, stream, job, t_pad, r0, n, aux)
        if (job.mass_aware) {
            if (kmax <= 32) RAMNET_MASS_RANGE(true, 1);
            else if (kmax <= 64) RAMNET_MASS_RANGE(true, 2);
            else RAMNET_MASS_RANGE(true, 4);
        } else {
            if (kmax <= 32) RAMNET_MASS_RANGE(false, 1);
            else if (kmax <= 64) RAMNET_MASS_RANGE(false, 2);
            else RAMNET_MASS_RANGE(false, 4);
        }
#undef RAMNET_MASS_RANGE
    }
    if (job.mass_aware) {
        const int64_t n = static_cast<int64_t>(job.B) * job.H * job.T;
        hipLaunchKernelGGL((mass_read_scale_kernel<AUX>), dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                           stream, job, t_pad, aux);
    }
    return hipGetLastError();
}

template<bool MA, int AUX>
hipError_t launch_mass_pass(const SegmentJob &job, int t_pad, int n_cu, void *maps, size_t maps_bytes,
                            const MassAux &aux, hipStream_t stream) {
    const int kmax = std::max(job.Kw, job.Kr);
    if (kmax <= 32)
        return launch_mass_pass_mp<MA, 1, AUX>(job, t_pad, n_cu, maps, maps_bytes, aux, stream);
    if (kmax <= 64)
        return launch_mass_pass_mp<MA, 2, AUX>(job, t_pad, n_cu, maps, maps_bytes, aux, stream);
    return launch_mass_pass_mp<MA, 4, AUX>(job, t_pad, n_cu, maps, maps_bytes, aux, stream);
}

}  // namespace

int64_t mass_replay_scratch_bytes(int B, int H, int T, int A) {
    SegmentJob job{};
    job.B = B;
    job.H = H;
    job.T = T;
    job.A = A;
    int len = 0;
    const int nck = mass_chunks(job, static_cast<size_t>(1) << 62, kReplayChunkFactor * cu_count(), &len);
    return nck <= 1 ? 0 : static_cast<int64_t>(B) * H * nck * A * static_cast<int64_t>(sizeof(float2));
}

int mass_replay_chunks(const SegmentJob &job, size_t maps_bytes, int *chunk_len) {
    return mass_chunks(job, maps_bytes, kReplayChunkFactor * cu_count(), chunk_len);
}

hipError_t launch_mass_replay(const SegmentJob &job, const MassAux &aux, void *maps, size_t maps_bytes,
                              hipStream_t stream) {
    if (static_cast<int64_t>(job.B) * job.H * job.T == 0)
        return hipSuccess;
    const int t_pad = scan_t_pad(job.T);
    if (job.A > kMaxAuxSlots)
        return launch_mass_ranges<true>(job, t_pad, kMaxAuxSlots, aux, stream);
    const int n = kReplayChunkFactor * cu_count();
    return job.mass_aware ? launch_mass_pass<true, 1>(job, t_pad, n, maps, maps_bytes, aux, stream)
                          : launch_mass_pass<false, 1>(job, t_pad, n, maps, maps_bytes, aux, stream);
}

bool segment_saved_aux(int A) { return A <= kMaxAuxSlots; }

template<typename Scalar>
hipError_t launch_pack(const PackJob &job, unsigned blocks, int t_pad, hipStream_t stream) {
    const int ke = std::max(job.Kw, job.Kr);
    if (ke <= 16) {
        const int64_t n = static_cast<int64_t>(job.B) * job.H * t_pad;
        const dim3 grid(static_cast<unsigned>((n + 255) / 256));
        if (ke <= 8)
            hipLaunchKernelGGL((pack_token_records_kernel<Scalar, 8>), grid, dim3(256), 0, stream, job, t_pad);
        else
            hipLaunchKernelGGL((pack_token_records_kernel<Scalar, 16>), grid, dim3(256), 0, stream, job, t_pad);
    } else if (job.Kw <= 8) {
        hipLaunchKernelGGL((pack_records_kernel<Scalar, 8>), dim3(blocks), dim3(256), 0, stream, job, t_pad);
    } else {
        hipLaunchKernelGGL((pack_records_kernel<Scalar, 16>), dim3(blocks), dim3(256), 0, stream, job, t_pad);
    }
    return hipGetLastError();
}

hipError_t launch_pack_records(const PackJob &job, hipStream_t stream, const char **why) {
    const int t_pad = scan_t_pad(job.T);
    const int64_t n = static_cast<int64_t>(job.B) * job.H * (job.Kw + job.Kr) * t_pad;
    if (n == 0)
        return hipSuccess;
    const unsigned blocks = static_cast<unsigned>((n + 255) / 256);
    switch (job.dtype) {
        case kF32: return launch_pack<float>(job, blocks, t_pad, stream);
        case kF16: return launch_pack<_Float16>(job, blocks, t_pad, stream);
        case kBF16: return launch_pack<bf16_t>(job, blocks, t_pad, stream);
        default: *why = "record packing: unsupported dtype"; return hipErrorInvalidValue;
    }
}

namespace {
// dst = src over n floats: the state copy of a call without tokens.
__global__ __launch_bounds__(256) void state_copy_kernel(float *dst, const float *src, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n)
        dst[i] = src[i];
}
}  // namespace

// RAMNET_SCAN_LAYOUT="vec,epp,np,nw[,pre[,tp]]" replaces the planner's
// choice (tests sweep every compiled layout with it; also a tuning knob).
// tp = 2 names a paired layout (pre = 1, np = 1; epp events per half wave).
// The layout must be compiled, cover max(Kw, Kr) events and fit in LDS.
static int layout_override(const SegmentJob &job, Plan *p, const char **why) {
    const char *env = std::getenv("RAMNET_SCAN_LAYOUT");
    if (!env || !*env)
        return 0;
    int vec = 0, epp = 0, np = 0, nw = 0, pre = 0, tp = 1;
    const int n = std::sscanf(env, "%d,%d,%d,%d,%d,%d", &vec, &epp, &np, &nw, &pre, &tp);
    const bool pair = n == 6 && tp == 2;
    const bool named = pair ? pre == 1 && np == 1 && scan_pair_layout_compiled(vec, epp, nw)
                            : (n >= 4 && n <= 6) && (pre == 0 || pre == 1) && tp == 1 &&
                                  scan_layout_compiled(vec, epp, np, nw, pre != 0);
    if (!named) {
        *why = "RAMNET_SCAN_LAYOUT names no compiled layout (vec,epp,np,nw[,pre[,tp]])";
        return -1;
    }
    const size_t lds = pair ? scan_pair_lds_bytes(job.A, vec, epp, nw, dtype_bytes(job.dtype))
                            : scan_lds_bytes(job.A, vec, epp, np, nw, dtype_bytes(job.dtype), pre != 0);
    if (epp * np < std::max(job.Kw, job.Kr) || static_cast<int64_t>(lds) > kLdsPerCu ||
        (pre && job.A > kMaxPrePassSlots) ||
        (pair && (job.A > kMaxPairSlots || !pair_records_fit(std::max(job.Kw, job.Kr), job.T)))) {
        *why = "RAMNET_SCAN_LAYOUT does not cover top_k or does not fit in LDS";
        return -1;
    }
    *p = {vec, epp, np, nw, nw * (kWave / (pair ? 2 : 1) / epp) * vec, lds, pre != 0};
    p->tp = pair ? 2 : 1;
    return 1;
}

// The layout a launch of this job uses: the override, else the planner's
// choice for the job's B, H, dtype and this device's CU count. A job that
// saves rows takes the override only where it can save them.
static bool pick_plan(const SegmentJob &job, Plan *p, const char **why) {
    if (job.save.w) {
        const SavedRows &sv = job.save;
        const int forced = layout_override(job, p, why);
        if (forced > 0 && p->pre && p->tp == 1 && job.A <= kMaxPrePassSlots && save_fits(sv, job.T) &&
            save_layout_ok(&sv, p->vec, p->epp, p->np, p->cs, job.C))
            return true;
        if (!make_plan(job.B, job.H, job.A, job.C, job.Kw, job.Kr, dtype_bytes(job.dtype), cu_count(), job.T, p, &sv)) {
            *why = "segment forward: no layout saves the backward's rows for this shape (see "
                   "ramnet_segment_saved_bytes)";
            return false;
        }
        return true;
    }
    const int forced = layout_override(job, p, why);
    if (forced < 0)
        return false;
    if (!forced && !make_plan(job.B, job.H, job.A, job.C, job.Kw, job.Kr, dtype_bytes(job.dtype), cu_count(), job.T, p)) {
        *why = "segment forward: shape outside the LDS-resident scan (top_k <= 128; slot spaces wider than one "
               "resident slice are scanned in at most 4096 slot ranges)";
        return false;
    }
    return true;
}

int segment_plan(int B, int H, int T, int A, int C, int Kw, int Kr, int dtype, int *cs, int *lds_bytes, int *pre,
                 int *ranges) {
    SegmentJob job{};
    job.B = B;
    job.H = H;
    job.T = T;
    job.A = A;
    job.C = C;
    job.Kw = Kw;
    job.Kr = Kr;
    job.dtype = dtype;
    Plan p{};
    const char *why = nullptr;
    if (!pick_plan(job, &p, &why))
        return 0;
    if (cs)
        *cs = p.cs;
    if (lds_bytes)
        *lds_bytes = static_cast<int>(p.lds);
    if (pre)
        *pre = p.pre ? 1 : 0;
    if (ranges)
        *ranges = p.nr;
    return 1;
}

bool segment_forward_can_save(int B, int H, int T, int A, int C, int Kw, int Kr, int dtype, const SavedRows &geo) {
    Plan p{};
    return make_plan(B, H, A, C, Kw, Kr, dtype_bytes(dtype), cu_count(), T, &p, &geo);
}

hipError_t launch_segment_forward(const SegmentJob &job, hipStream_t stream, const char **why) {
    if (static_cast<int64_t>(job.B) * job.H == 0)
        return hipSuccess;
    Plan p{};
    if (!pick_plan(job, &p, why))
        return hipErrorInvalidValue;
    if (job.T == 0) {
        // no events: the final state is the initial state (a kernel, not a
        // copy, so that callers may capture the call in a graph)
        const int64_t ns = static_cast<int64_t>(job.B) * job.H * job.A;
        if (job.slot_out != job.init_slot)
            hipLaunchKernelGGL(state_copy_kernel, dim3(static_cast<unsigned>((ns * job.C + 255) / 256)), dim3(256), 0,
                               stream, job.slot_out, job.init_slot, ns * job.C);
        hipLaunchKernelGGL(state_copy_kernel, dim3(static_cast<unsigned>((ns + 255) / 256)), dim3(256), 0, stream,
                           job.mass_out, job.init_mass, ns);
        return hipGetLastError();
    }
    if (p.pre && !job.gain) {
        *why = "segment forward: the precomputed-gain layout needs the gain records of the scan workspace";
        return hipErrorInvalidValue;
    }
    if (p.tp == 2 && !job.flags) {
        *why = "segment forward: the paired layout needs the flags of the scan workspace";
        return hipErrorInvalidValue;
    }
    // the pre-pass writes the paired scan's flags only when it runs
    SegmentJob pj = job;
    if (p.tp != 2)
        pj.flags = nullptr;
    ScanGeom geo{};
    geo.n_slices = (job.C + p.cs - 1) / p.cs;
    geo.n_units = job.B * job.H * geo.n_slices;
    geo.t_pad = scan_t_pad(job.T);
    geo.n_chunks = (job.T + kChunk - 1) / kChunk;
    geo.r0 = 0;
    geo.n_local = job.A;
    if (job.dtype != kF32 && job.dtype != kF16 && job.dtype != kBF16) {
        *why = "segment forward: unsupported dtype";
        return hipErrorInvalidValue;
    }
    if (p.nr > 1 && !job.yacc) {
        *why = "segment forward: a scan in slot ranges needs fp32 read sums (y for fp32 y, else workspace)";
        return hipErrorInvalidValue;
    }
    if (p.pre) {
        hipError_t err;
        if (job.A > kMaxPrePassSlots) {
            err = launch_mass_ranges<false>(job, geo.t_pad, kMaxPrePassSlots, MassAux{}, stream);
        } else {
            // the chunk maps use y as scratch: the scan overwrites it afterwards
            const size_t y_bytes = static_cast<size_t>(job.B) * job.H * job.T * job.C * dtype_bytes(job.dtype);
            const MassAux none{};
            const int n = kReplayChunkFactor * cu_count();
            if (job.save.w && job.save.aux.wev) {
                // a saving forward also keeps the backward's per-event records
                err = job.mass_aware ? launch_mass_pass<true, 2>(pj, geo.t_pad, n, job.y, y_bytes, job.save.aux, stream)
                                     : launch_mass_pass<false, 2>(pj, geo.t_pad, n, job.y, y_bytes, job.save.aux, stream);
            } else {
                err = job.mass_aware ? launch_mass_pass<true, 0>(pj, geo.t_pad, n, job.y, y_bytes, none, stream)
                                     : launch_mass_pass<false, 0>(pj, geo.t_pad, n, job.y, y_bytes, none, stream);
            }
        }
        if (err != hipSuccess)
            return err;
    }
    if (p.tp == 2) {
        switch (job.dtype) {
            case kF32: return launch_scan_pair_f32(pj, geo, p.vec, p.epp, p.nw, stream);
            case kF16: return launch_scan_pair_f16(pj, geo, p.vec, p.epp, p.nw, stream);
            default: return launch_scan_pair_bf16(pj, geo, p.vec, p.epp, p.nw, stream);
        }
    }
    // slot ranges in order: each adds its read sums to the fp32 sums of the
    // ranges before it, and the last stores y
    const int al = (job.A + p.nr - 1) / p.nr;
    for (int r = 0; r < p.nr; ++r) {
        geo.r0 = r * al;
        geo.n_local = std::min(al, job.A - geo.r0);
        geo.last = r == p.nr - 1 ? 1 : 0;
        hipError_t err;
        switch (job.dtype) {
            case kF32: err = launch_scan_f32(job, geo, p.vec, p.epp, p.np, p.nw, p.pre, stream); break;
            case kF16: err = launch_scan_f16(job, geo, p.vec, p.epp, p.np, p.nw, p.pre, stream); break;
            default: err = launch_scan_bf16(job, geo, p.vec, p.epp, p.np, p.nw, p.pre, stream); break;
        }
        if (err != hipSuccess)
            return err;
    }
    return hipSuccess;
}

}  // namespace ramnet
