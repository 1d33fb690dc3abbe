// Fused single-token decode step against a persistent slot state.
//
// Semantics follow the reference decode step
// (csrc/ram_attn_topk_autoregressive.cu:37-191 and the torch path
// torch_impl.py:217-288 at T = 1): decode the write and read addresses,
// apply the K gated-sparse-update writes (row + mass read-modify-write),
// then read y = sum_k r_k s_{a_k} from the post-write state. A masked batch
// row leaves the state untouched and gets y = 0.
//
// MI355X mapping: one 64-lane wave per (b, h).
//  * Fast path (P <= 64, K <= 16, C <= 256): the two addresses are decoded
//    cooperatively (one per half-wave when they fit, lane-parallel bitonic
//    sorts), then every write row, every read row that is not also written,
//    and their masses are requested in one batch so the step costs a single
//    HBM round trip; reads of a just-written slot take the updated row from
//    LDS instead of re-reading memory.
//  * General path: exact LDS search for each address, then sequential row
//    updates and reads.
#include "ramnet_device.hpp"
#include "ramnet_kernels.hpp"
#include "ramnet_search.hpp"

#include <algorithm>

namespace ramnet {

namespace {

constexpr int kEv = 16;     // fast path: up to 16 write and 16 read slots
constexpr int kMaxCpl = 4;  // fast path: up to 4 channels per lane (C <= 256)
// The fast path issues its row loads unconditionally from clamped in-bounds
// addresses: a guarded load would wait for its data inside the branch and
// serialise the HBM round trips.

__device__ __forceinline__ float gsu_gain(float w, float d) {
    float r = __builtin_amdgcn_rcpf(d);
    r = fmaf(r, fmaf(-d, r, 1.f), r);
    return w * r;
}

// 32-bit buffer accesses of fp32 data (the builtins move raw bits).
__device__ __forceinline__ float buf_load_f32(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
__device__ __forceinline__ void buf_store_f32(float v, __amdgpu_buffer_rsrc_t r, int voff, int soff) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, voff, soff, 0);
}

// One event per lane from a group's sorted top list: (slot after CAPE,
// weight), or (0, 0) on lanes past K.
__device__ __forceinline__ void lane_event(float v, int c, bool inactive, int K, float re_norm, int li, int g0,
                                           int shift, int A, int &slot, float &val) {
    float lse = 0.f;
    const float v0 = __shfl(v, g0);
    if (re_norm != 0.f && !inactive && v0 > kNegInfF) {
        const float e = expf(v - v0);
        float sum = 0.f;
        for (int k = K - 1; k >= 0; --k)
            sum += __shfl(e, g0 + k);
        lse = v0 + log_sum(sum);
    }
    const int content = inactive ? li : c;
    int o = content - shift;
    o = o < 0 ? o + A : o;
    slot = li < K ? o : 0;
    val = li < K && !inactive ? expf(v - re_norm * lse) : 0.f;
}

// Value of `v` on lane L (L uniform; a constant after unrolling), as a
// wave-uniform scalar.
__device__ __forceinline__ float lane_f(float v, int L) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), L));
}
__device__ __forceinline__ int lane_i(int v, int L) { return __builtin_amdgcn_readlane(v, L); }

// FULLC: C == 64 * kCpl, so every lane owns kCpl real channels.
// Events live one per lane: write event k on lane k, read event k on lane
// RB + k (RB = 32 when the two addresses share the wave as half-waves, else
// 0 with separate registers). The event math (mass, alpha, gain) runs lane
// parallel; each row's scalars are then broadcast with v_readlane. Rows and
// masses of one (b, h) are addressed through buffer resources (32-bit
// offsets; the launcher keeps A * C * 4 below 2^31).
template<typename T, int GW, int KE, int kCpl, bool FULLC>
__global__ __launch_bounds__(64) void autoregressive_fast_kernel(const DecodeJob job) {
    constexpr int RB = GW == 32 ? 32 : 0;
    __shared__ int s_ws[KE], s_rs[KE];
    __shared__ float s_wv[KE];
    __shared__ float s_row[KE][kWave * kCpl];

    // grid (B, H): the (b, h) pair without a division
    const int b = blockIdx.x, h = blockIdx.y;
    const int lane = threadIdx.x;
    const int H = job.H, A = job.A, C = job.C, U = job.U, P = job.P, Kw = job.Kw, Kr = job.Kr;
    const int bh = b * H + h;
    T *yrow = static_cast<T *>(job.y) + static_cast<int64_t>(bh) * C;

    // ---- every input of the step in one batch of loads
    const T *wp = static_cast<const T *>(job.w_addr) + static_cast<int64_t>(bh) * U * P;
    const T *rp = static_cast<const T *>(job.r_addr) + static_cast<int64_t>(bh) * U * P;
    GroupLogits<T> lw, lr;
    if constexpr (GW == 32) {
        lw.load((lane >> 5) ? rp : wp, U, P, lane & 31);
    } else {
        lw.load(wp, U, P, lane);
        lr.load(rp, U, P, lane);
    }
    int coff[kCpl];  // byte offset of each owned channel (clamped into the row)
#pragma unroll
    for (int j = 0; j < kCpl; ++j) {
        const int c = lane + j * kWave;
        coff[j] = (FULLC || c < C ? c : C - 1) * 4;
    }
    const T *xp = static_cast<const T *>(job.x) + static_cast<int64_t>(bh) * C;
    float xv[kCpl];
#pragma unroll
    for (int j = 0; j < kCpl; ++j)
        xv[j] = load_f32(xp + coff[j] / 4);
    const float gamma = load_f32(static_cast<const T *>(job.gamma) + bh);
    const int pos = job.position_ids[b];
    const uint8_t valid = job.mask ? job.mask[b] : 1;
    if (!valid) {
        for (int c = lane; c < C; c += kWave)
            store_f32(yrow + c, 0.f);
        return;
    }
    const int shift = h < job.embed_num ? pos_mod(pos, A) : 0;
    const auto srs = __builtin_amdgcn_make_buffer_rsrc(job.slot + static_cast<int64_t>(bh) * A * C, 0, A * C * 4,
                                                       kBufWord3);
    const auto mrs = __builtin_amdgcn_make_buffer_rsrc(job.mass + static_cast<int64_t>(bh) * A, 0, A * 4, kBufWord3);

    // ---- address decode: per-lane events, their masses, the slot tables
    int ow, orr;      // write / read event slot of this lane
    float vw, vr;     // their weights
    float emw, emr;   // their pre-step masses
    if constexpr (GW == 32) {
        const int half = lane >> 5, li = lane & 31;
        const int K = half ? Kr : Kw;
        float v;
        int c;
        const bool inactive = group_search<T, 32>(lw, U, P, K, li, v, c);
        lane_event(v, c, inactive, K, half ? job.r_re_norm : job.w_re_norm, li, half * 32, shift, A, ow, vw);
        orr = ow;
        vr = vw;
        emw = buf_load_f32(mrs, ow * 4, 0);
        emr = emw;
        if (li < KE) {
            (half ? s_rs : s_ws)[li] = ow;
            if (!half)
                s_wv[li] = vw;
        }
    } else {
        float v;
        int c;
        bool inactive = group_search<T, 64>(lw, U, P, Kw, lane, v, c);
        lane_event(v, c, inactive, Kw, job.w_re_norm, lane, 0, shift, A, ow, vw);
        emw = buf_load_f32(mrs, ow * 4, 0);
        inactive = group_search<T, 64>(lr, U, P, Kr, lane, v, c);
        lane_event(v, c, inactive, Kr, job.r_re_norm, lane, 0, shift, A, orr, vr);
        emr = buf_load_f32(mrs, orr * 4, 0);
        if (lane < KE) {
            s_ws[lane] = ow;
            s_wv[lane] = vw;
            s_rs[lane] = orr;
        }
    }

    // ---- one batch of row requests (row k's offset is a scalar)
    const int rowb = C * 4;
    float wrow[KE][kCpl], rrow[KE][kCpl];
#pragma unroll
    for (int k = 0; k < KE; ++k) {
        const int so = lane_i(ow, k) * rowb;
#pragma unroll
        for (int j = 0; j < kCpl; ++j)
            wrow[k][j] = buf_load_f32(srs, coff[j], so);
    }
#pragma unroll
    for (int k = 0; k < KE; ++k) {
        const int so = lane_i(orr, RB + k) * rowb;
#pragma unroll
        for (int j = 0; j < kCpl; ++j)
            rrow[k][j] = buf_load_f32(srs, coff[j], so);
    }
    // (one wave per workgroup: its LDS accesses complete in order, so the
    // slot tables written above are visible to the reads below)
    __builtin_amdgcn_wave_barrier();
    // Forwarding: fwd[k] = the write event (nonzero weight) on read k's slot,
    // or -1. One lane per (read, write) pair compares the slots; a ballot per
    // 64 pairs collects the matches (top-K slots are distinct, so at most one
    // write matches a read). The event tables are read unconditionally (both
    // indices are below KE) and the conditions combined bitwise, so the
    // comparison has no divergent branch.
    static_assert((KE * KE) % kWave == 0, "forwarding rounds cover whole waves");
    int fwd[KE];
#pragma unroll
    for (int base = 0; base < KE * KE; base += kWave) {
        const int l = base + lane;
        const int k = (l / KE) % KE, j2 = l % KE;
        const int ws = s_ws[j2], rs = s_rs[k];
        const float wvj = s_wv[j2];
        const bool match = (j2 < Kw) & (k < Kr) & (wvj != 0.f) & (ws == rs);
        const uint64_t hits = __ballot(match);
#pragma unroll
        for (int k2 = 0; k2 < KE; ++k2) {
            if (k2 * KE >= base && k2 * KE < base + kWave) {
                const uint32_t bits =
                    static_cast<uint32_t>(hits >> (k2 * KE - base)) & ((KE >= 32 ? 0u : (1u << KE)) - 1u);
                // highest set bit, -1 when none, without a zero test:
                // clz(2b + 1) = clz(b) - 1 for b != 0 and 31 for b = 0. (hipcc
                // 7.2 turned `bits ? 31 - clz(bits) : -1` on the top field of
                // the ballot into a 64-bit VALU compare and left the select
                // reading a stale SCC, dropping those forwards.)
                static_assert(KE <= 16, "2 * bits + 1 must fit 32 bits");
                fwd[k2] = 30 - __builtin_clz(2u * bits + 1u);
            }
        }
    }
    // ---- write math, one write event per lane. e^-|gamma| is shared by the
    // events: alpha = num / den with the stable form of gsu_alpha, divided
    // with one Newton-refined reciprocal.
    const bool gpos = gamma >= 0.f;
    const float eg = expf(gpos ? -gamma : gamma);
    const float cw = 1.f - vw;
    const float den = gpos ? fmaf(eg, cw, vw) : fmaf(eg, vw, cw);
    const float alpha = gsu_gain(gpos ? cw * eg : cw, den);
    const float m2 = fmaf(alpha, emw, vw);
    const float gain = gsu_gain(vw, m2 + job.eps);
    const bool wlane = GW == 32 ? lane < 32 : true;
    if (wlane && lane < Kw && vw != 0.f)
        buf_store_f32(m2, mrs, ow * 4, 0);
    // every row load is in flight before the first update (the fence stops
    // the scheduler from sinking loads into the update branches, where each
    // would wait for its own data)
    __builtin_amdgcn_sched_barrier(0);
    // ---- row updates
#pragma unroll
    for (int k = 0; k < KE; ++k) {
        if (lane_f(vw, k) != 0.f) {
            const float g = lane_f(gain, k);
            const int so = lane_i(ow, k) * rowb;
#pragma unroll
            for (int j = 0; j < kCpl; ++j) {
                const int c = lane + j * kWave;
                const float sv = fmaf(g, xv[j] - wrow[k][j], wrow[k][j]);
                s_row[k][c] = sv;  // each lane re-reads only what it wrote
                if (FULLC || c < C)
                    buf_store_f32(sv, srs, coff[j], so);
            }
        }
    }

    // ---- reads of the post-write state. The forwarded rows of every read
    // are fetched from LDS in one batch (index clamped, value selected), so
    // the reads cost one LDS round trip; events past top-K have r = 0.
    float sval[KE][kCpl];
#pragma unroll
    for (int k = 0; k < KE; ++k) {
        const int f = fwd[k];
        const int fc = f < 0 ? 0 : f;
#pragma unroll
        for (int j = 0; j < kCpl; ++j) {
            const float lv = s_row[fc][lane + j * kWave];
            sval[k][j] = f >= 0 ? lv : rrow[k][j];
        }
    }
    float rv[KE], rw[KE];  // read weights (mass-aware: r * post-write mass)
#pragma unroll
    for (int k = 0; k < KE; ++k) {
        rv[k] = lane_f(vr, RB + k);
        rw[k] = rv[k];
    }
    if (job.mass_aware) {
        float wm[KE];
#pragma unroll
        for (int k = 0; k < KE; ++k)
            wm[k] = lane_f(m2, k);
#pragma unroll
        for (int k = 0; k < KE; ++k) {
            float m = lane_f(emr, RB + k);
#pragma unroll
            for (int j2 = 0; j2 < KE; ++j2)
                m = fwd[k] == j2 ? wm[j2] : m;
            rw[k] = rv[k] * m;
        }
    }
    float acc[kCpl];
#pragma unroll
    for (int j = 0; j < kCpl; ++j)
        acc[j] = 0.f;
    float sr = 0.f, srm = 0.f;
#pragma unroll
    for (int k = 0; k < KE; ++k) {
        sr += rv[k];
        srm += rw[k];
#pragma unroll
        for (int j = 0; j < kCpl; ++j)
            acc[j] = fmaf(rw[k], sval[k][j], acc[j]);
    }
    const float scale = job.mass_aware ? sr / (srm + job.eps) : 1.f;
#pragma unroll
    for (int j = 0; j < kCpl; ++j) {
        const int c = lane + j * kWave;
        if (FULLC || c < C)
            store_f32(yrow + c, acc[j] * scale);
    }
}

// General shapes: exact LDS search, then sequential row updates.
template<typename T>
__global__ __launch_bounds__(64) void autoregressive_general_kernel(const DecodeJob job, int NA, int NPD) {
    extern __shared__ float smem[];
    __shared__ int s_flag;
    // grid (B, H): the (b, h) pair without a division
    const int b = blockIdx.x, h = blockIdx.y;
    const int lane = threadIdx.x;
    const int H = job.H, A = job.A, C = job.C, U = job.U, P = job.P, Kw = job.Kw, Kr = job.Kr;
    const int bh = b * H + h;
    T *yrow = static_cast<T *>(job.y) + static_cast<int64_t>(bh) * C;
    if (job.mask && !job.mask[b]) {
        for (int c = lane; c < C; c += kWave)
            store_f32(yrow + c, 0.f);
        return;
    }
    float *lg = smem;
    float *ex = lg + U * P;
    float *sv = ex + U * NPD;
    int *si = reinterpret_cast<int *>(sv + NA);
    int *ev_slot = si + NA;            // Kw + Kr
    float *ev_val = reinterpret_cast<float *>(ev_slot + Kw + Kr);  // Kw + Kr
    const int shift = h < job.embed_num ? pos_mod(job.position_ids[b], A) : 0;

    for (int which = 0; which < 2; ++which) {
        const T *ptr = static_cast<const T *>(which ? job.r_addr : job.w_addr) + static_cast<int64_t>(bh) * U * P;
        const int K = which ? Kr : Kw;
        const float re = which ? job.r_re_norm : job.w_re_norm;
        const bool inactive = block_search_exact(ptr, 1, U, P, A, NA, NPD, lg, ex, sv, si, &s_flag);
        const float lse = (re != 0.f && !inactive) ? topk_lse_serial(sv, K) : 0.f;
        for (int k = lane; k < K; k += kWave) {
            const int content = inactive ? k : si[k];
            int o = content - shift;
            o = o < 0 ? o + A : o;
            ev_slot[which * Kw + k] = o;
            ev_val[which * Kw + k] = inactive ? 0.f : expf(sv[k] - re * lse);
        }
        __syncthreads();
    }

    float *slot = job.slot + static_cast<int64_t>(bh) * A * C;
    float *mass = job.mass + static_cast<int64_t>(bh) * A;
    const T *xp = static_cast<const T *>(job.x) + static_cast<int64_t>(bh) * C;
    const float gamma = load_f32(static_cast<const T *>(job.gamma) + bh);
    for (int k = 0; k < Kw; ++k) {
        const float w = ev_val[k];
        if (w == 0.f)
            continue;
        const int a = ev_slot[k];
        const float alpha = gsu_alpha(w, gamma);
        const float m2 = fmaf(alpha, mass[a], w);
        const float g = gsu_gain(w, m2 + job.eps);
        float *row = slot + static_cast<int64_t>(a) * C;
        for (int c = lane; c < C; c += kWave) {
            const float s = row[c];
            row[c] = fmaf(g, load_f32(xp + c) - s, s);
        }
        __syncthreads();
        if (lane == 0)
            mass[a] = m2;
        __syncthreads();
    }
    __threadfence_block();
    __syncthreads();
    float sr = 0.f, srm = 0.f;
    for (int k = 0; k < Kr; ++k) {
        const float r = ev_val[Kw + k];
        sr += r;
        srm += job.mass_aware ? r * mass[ev_slot[Kw + k]] : r;
    }
    const float scale = job.mass_aware ? sr / (srm + job.eps) : 1.f;
    for (int c = lane; c < C; c += kWave) {
        float acc = 0.f;
        for (int k = 0; k < Kr; ++k) {
            const float r = ev_val[Kw + k];
            if (r == 0.f)
                continue;
            const int a = ev_slot[Kw + k];
            const float wgt = job.mass_aware ? r * mass[a] : r;
            acc = fmaf(wgt, slot[static_cast<int64_t>(a) * C + c], acc);
        }
        store_f32(yrow + c, acc * scale);
    }
}

int pow2_ceil(int x) {
    int p = 1;
    while (p < x)
        p <<= 1;
    return p;
}

template<typename T>
hipError_t launch_typed(const DecodeJob &job, hipStream_t stream, const char **why) {
    const int kmax = std::max(job.Kw, job.Kr);
    const int stair = staircase_count(kmax);
    const bool fast_ok = job.P <= 64 && kmax <= kEv && job.C <= kWave * kMaxCpl && stair <= 64 &&
                         static_cast<int64_t>(job.A) * job.C * 4 <= INT32_MAX;
    if (job.H > 65535) {
        *why = "decode step: at most 65535 heads (grid y dimension)";
        return hipErrorInvalidValue;
    }
    const dim3 grid(static_cast<unsigned>(job.B), static_cast<unsigned>(job.H));
    if (fast_ok) {
        const bool half = job.P <= 32 && stair <= 32;
        const bool narrow = job.C <= 2 * kWave;
        const bool few = kmax <= 8;
        const dim3 g(grid), blk(kWave);  // one wave per (b, h)
#define RAMNET_AR_LAUNCH(GW, KE, CPL)                                                                          \
    do {                                                                                                        \
        if (job.C == (CPL) * kWave)                                                                             \
            hipLaunchKernelGGL((autoregressive_fast_kernel<T, GW, KE, CPL, true>), g, blk, 0, stream, job);    \
        else                                                                                                    \
            hipLaunchKernelGGL((autoregressive_fast_kernel<T, GW, KE, CPL, false>), g, blk, 0, stream, job);   \
    } while (0)
        if (half) {
            if (few) { if (narrow) RAMNET_AR_LAUNCH(32, 8, 2); else RAMNET_AR_LAUNCH(32, 8, 4); }
            else { if (narrow) RAMNET_AR_LAUNCH(32, 16, 2); else RAMNET_AR_LAUNCH(32, 16, 4); }
        } else {
            if (few) { if (narrow) RAMNET_AR_LAUNCH(64, 8, 2); else RAMNET_AR_LAUNCH(64, 8, 4); }
            else { if (narrow) RAMNET_AR_LAUNCH(64, 16, 2); else RAMNET_AR_LAUNCH(64, 16, 4); }
        }
#undef RAMNET_AR_LAUNCH
        return hipGetLastError();
    }
    const int NA = pow2_ceil(job.A), NPD = pow2_ceil(job.P);
    const size_t lds = static_cast<size_t>(job.U) * job.P * 4 + static_cast<size_t>(job.U) * NPD * 4 +
                       static_cast<size_t>(NA) * 8 + static_cast<size_t>(job.Kw + job.Kr) * 8;
    if (lds > 96 * 1024) {
        *why = "decode step: shape needs P <= 64, top_k <= 16, C <= 256 and A*C*4 < 2^31, or P**U small enough for the exact LDS search (A <= 8192)";
        return hipErrorInvalidValue;
    }
    hipLaunchKernelGGL(autoregressive_general_kernel<T>, grid, dim3(kWave), lds, stream, job, NA, NPD);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_autoregressive(const DecodeJob &job, hipStream_t stream, const char **why) {
    if (job.B * job.H == 0)
        return hipSuccess;
    switch (job.dtype) {
        case kF32: return launch_typed<float>(job, stream, why);
        case kF16: return launch_typed<_Float16>(job, stream, why);
        case kBF16: return launch_typed<bf16_t>(job, stream, why);
        default: *why = "decode step: unsupported dtype"; return hipErrorInvalidValue;
    }
}

}  // namespace ramnet
