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
// share a CU's LDS, then dispatches to the per-dtype kernels.
#include "ramnet_device.hpp"
#include "ramnet_kernels.hpp"
#include "segment_scan.hpp"

#include <algorithm>
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

int cu_count() {
    static int cached = 0;
    if (cached == 0) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
            cached = n;
        else
            cached = 256;
    }
    return cached;
}

int dtype_bytes(int dtype) { return dtype == kF32 ? 4 : 2; }

struct Plan {
    int vec, epp, np, nw, cs;
    size_t lds;
};

// Cost model of one layout, in cycles per token of one round of resident
// workgroups: a wave's token loop is bound by its dependency chain (LDS
// read -> update -> LDS write, ~kChainCycles) or by the issue of its VALU
// work (~10 + 6 * VEC * NP instructions, 4 cycles each, shared by the waves
// on one SIMD), whichever is longer. Total = rounds * per-token cycles.
constexpr int64_t kChainCycles = 160;

bool make_plan(int B, int H, int A, int C, int Kw, int Kr, int elem, int n_cu, Plan *out) {
    const int kmax = std::max(Kw, Kr);
    if (kmax > 2 * kWave)
        return false;
    const int epp0 = std::min(kWave, std::max(4, pow2_ceil(kmax)));
    bool found = false;
    int64_t best = 0;
    for (int epp = 4; epp <= kWave; epp <<= 1) {
        const int np = (kmax + epp - 1) / epp;
        if (np > 2 || (np == 2 && epp * 2 < epp0))
            continue;
        for (int nw = 4; nw >= 1; nw >>= 1) {
            for (int vec = 4; vec >= 1; vec >>= 1) {
                if (!scan_layout_compiled(vec, epp, np, nw))
                    continue;
                const int cs = nw * (kWave / epp) * vec;
                const size_t lds = scan_lds_bytes(A, vec, epp, np, nw, elem);
                const int64_t gran = (static_cast<int64_t>(lds) + kLdsGranule - 1) / kLdsGranule * kLdsGranule;
                if (gran > kLdsPerCu)
                    continue;
                const int64_t units = static_cast<int64_t>(B) * H * ((C + cs - 1) / cs);
                const int64_t per_cu = std::min<int64_t>(kLdsPerCu / gran, std::max(1, 8 / nw));
                const int64_t rounds = (units + per_cu * n_cu - 1) / (per_cu * n_cu);
                const int64_t resident = std::min<int64_t>(per_cu, (units + n_cu - 1) / n_cu);
                const int64_t waves_per_simd = (resident * nw + 3) / 4;
                const int64_t issue = 4 * (10 + 6 * vec * np) * waves_per_simd;
                int64_t cost = rounds * std::max(kChainCycles, issue);
                if (C % cs != 0)
                    cost = cost * 3 / 2;  // partial slices take the guarded path
                const bool better = !found || cost < best ||
                                    (cost == best && (nw > out->nw || (nw == out->nw && cs > out->cs)));
                if (better) {
                    *out = {vec, epp, np, nw, cs, lds};
                    best = cost;
                    found = true;
                }
            }
        }
    }
    return found;
}

// Scan records from decoder outputs: one thread per (b*H + h, event, t) with
// t < T_pad. Writes keep positive weights; reads were stored negated.
template<typename Scalar>
__global__ __launch_bounds__(256) void pack_records_kernel(const PackJob job, int t_pad) {
    const int Kt = job.Kw + job.Kr;
    const int64_t n = static_cast<int64_t>(job.B) * job.H * Kt * t_pad;
    const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    write_noop_chunk(job.noop_w, job.noop_r, gid);
    if (gid >= n)
        return;
    const int t = static_cast<int>(gid % t_pad);
    const int64_t rest = gid / t_pad;
    const int k = static_cast<int>(rest % Kt);
    const int bh = static_cast<int>(rest / Kt);
    const int b = bh / job.H;
    const int T = job.T, A = job.A;
    const int tl = t < T ? t : T - 1;
    const int64_t src = (static_cast<int64_t>(bh) * Kt + k) * T + tl;
    const int a = job.addr_idx[src] - bh * A;
    const float v = job.addr_val[src];
    const float g = load_f32(static_cast<const Scalar *>(job.gamma) + static_cast<int64_t>(bh) * T + tl);
    const uint8_t *mp = job.mask ? job.mask + static_cast<int64_t>(b) * T + tl : &kScanAllValid;
    const bool live = t < T && *mp != 0 && static_cast<unsigned>(a) < static_cast<unsigned>(A);
    if (k < job.Kw) {
        const bool act = live && v != 0.f;
        // overlap with token t - 1 is not computed here: assumed (the scan
        // then orders the two tokens' row accesses strictly)
        const float overlap = __int_as_float(1);
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

}  // namespace

hipError_t launch_pack_records(const PackJob &job, hipStream_t stream, const char **why) {
    const int t_pad = scan_t_pad(job.T);
    const int64_t n = static_cast<int64_t>(job.B) * job.H * (job.Kw + job.Kr) * t_pad;
    if (n == 0)
        return hipSuccess;
    const unsigned blocks = static_cast<unsigned>((n + 255) / 256);
    switch (job.dtype) {
        case kF32: hipLaunchKernelGGL(pack_records_kernel<float>, dim3(blocks), dim3(256), 0, stream, job, t_pad); break;
        case kF16: hipLaunchKernelGGL(pack_records_kernel<_Float16>, dim3(blocks), dim3(256), 0, stream, job, t_pad); break;
        case kBF16: hipLaunchKernelGGL(pack_records_kernel<bf16_t>, dim3(blocks), dim3(256), 0, stream, job, t_pad); break;
        default: *why = "record packing: unsupported dtype"; return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

int segment_plan(int A, int C, int Kw, int Kr, int *cs, int *lds_bytes) {
    Plan p{};
    if (!make_plan(8, 16, A, C, Kw, Kr, 2, 256, &p))
        return 0;
    if (cs)
        *cs = p.cs;
    if (lds_bytes)
        *lds_bytes = static_cast<int>(p.lds);
    return 1;
}

// RAMNET_SCAN_LAYOUT="vec,epp,np,nw" replaces the planner's choice (tests
// sweep every compiled layout with it; also a tuning knob). The layout must
// be compiled, cover max(Kw, Kr) events and fit in LDS.
static int layout_override(const SegmentJob &job, Plan *p, const char **why) {
    const char *env = std::getenv("RAMNET_SCAN_LAYOUT");
    if (!env || !*env)
        return 0;
    int vec = 0, epp = 0, np = 0, nw = 0;
    if (std::sscanf(env, "%d,%d,%d,%d", &vec, &epp, &np, &nw) != 4 || !scan_layout_compiled(vec, epp, np, nw)) {
        *why = "RAMNET_SCAN_LAYOUT names no compiled layout (vec,epp,np,nw)";
        return -1;
    }
    const size_t lds = scan_lds_bytes(job.A, vec, epp, np, nw, dtype_bytes(job.dtype));
    if (epp * np < std::max(job.Kw, job.Kr) || static_cast<int64_t>(lds) > kLdsPerCu) {
        *why = "RAMNET_SCAN_LAYOUT does not cover top_k or does not fit in LDS";
        return -1;
    }
    *p = {vec, epp, np, nw, nw * (kWave / epp) * vec, lds};
    return 1;
}

hipError_t launch_segment_forward(const SegmentJob &job, hipStream_t stream, const char **why) {
    if (static_cast<int64_t>(job.B) * job.H == 0)
        return hipSuccess;
    Plan p{};
    const int forced = layout_override(job, &p, why);
    if (forced < 0)
        return hipErrorInvalidValue;
    if (!forced && !make_plan(job.B, job.H, job.A, job.C, job.Kw, job.Kr, dtype_bytes(job.dtype), cu_count(), &p)) {
        *why = "segment forward: shape outside the LDS-resident scan (needs (A*CS + A)*4 bytes <= 160 KiB for some "
               "slice width and top_k <= 128)";
        return hipErrorInvalidValue;
    }
    ScanGeom geo{};
    geo.n_slices = (job.C + p.cs - 1) / p.cs;
    geo.n_units = job.B * job.H * geo.n_slices;
    geo.t_pad = scan_t_pad(job.T);
    geo.n_chunks = (job.T + kChunk - 1) / kChunk;
    switch (job.dtype) {
        case kF32: return launch_scan_f32(job, geo, p.vec, p.epp, p.np, p.nw, stream);
        case kF16: return launch_scan_f16(job, geo, p.vec, p.epp, p.np, p.nw, stream);
        case kBF16: return launch_scan_bf16(job, geo, p.vec, p.epp, p.np, p.nw, stream);
        default: *why = "segment forward: unsupported dtype"; return hipErrorInvalidValue;
    }
}

}  // namespace ramnet
