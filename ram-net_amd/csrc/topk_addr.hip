// Product-Softmax top-K address decoder for gfx950.
//
// Semantics follow the reference decoder
// (packages/ramnet-ops/src/ramnet_ops/impl/torch_impl.py:152-214 and
// csrc/ram_attn_topk_addr.cu:51-117):
//   L_u = log_softmax(x_u) per digit (fp32),
//   score(c) = ((L_0[d_0] + L_1[d_1]) + L_2[d_2]) ..., c = sum_u d_u P^u,
//   top-K of score under (score desc, content index asc),
//   val = exp(score - r * logsumexp_K(score)),
//   CAPE: out = (c - pos) mod A for heads h < embed_num,
//   an address with any all -inf digit is inactive: val = 0.
//
// Two kernels:
//  * topk_addr_lane_kernel: one lane per (b, h, t) address (lane_search.hpp):
//    per digit the top-K logits are selected on packed (value, index) sort
//    keys, and the running top-K prefix list is combined with each digit
//    over the staircase of candidates that can reach the top K, so the
//    search never materialises the A = P^U scores. Used for P <= 64, K <= 16.
//  * topk_addr_bruteforce_kernel: one workgroup per address materialises all
//    A scores in LDS and bitonic-sorts them; exact for every K <= A.
//    Used for the shapes the lane kernel does not cover (A <= 8192).
#include "ramnet_device.hpp"
#include "ramnet_kernels.hpp"
#include "ramnet_search.hpp"
#include "lane_search.hpp"

#include <math.h>

namespace ramnet {

namespace {

constexpr float kNegInf = -__builtin_huge_valf();

// Whether token tl of batch row b is unmasked. Without a mask the load reads
// a byte of this row's position ids instead (always in bounds) and is
// ignored: a load that is always made needs no branch.
__device__ __forceinline__ bool addr_unmasked(const AddrJob &job, int b, int tl) {
    const bool has = job.mask != nullptr;
    const uint8_t *row = has ? job.mask + static_cast<int64_t>(b) * job.T
                             : reinterpret_cast<const uint8_t *>(job.position_ids + static_cast<int64_t>(b) * job.T);
    return !has | (row[tl] != 0);
}

// Record mode output of one address (source 0 = writes, 1 = reads). `get(k,
// c, v)` yields the k-th selected content slot and its weight. Events of
// masked or padding tokens, inactive addresses and zero weights become
// no-ops pointing at the scan's dummy rows (slot -2 for writes, -1 for reads).
// KM > 0 unrolls over a register list of that size; KM == 0 loops at run
// time (list in LDS).
template<typename Scalar, int KM, typename Get>
__device__ __forceinline__ void write_records(const AddrJob &job, int which, int64_t bh, int b, int t, int tl,
                                              bool inactive, Get get, int K, int shift, int overlap) {
    const int T = job.T, A = job.A;
    const int Tp = scan_t_pad(T);
    // (conditions are bitwise: a short-circuit test of a lane value becomes
    // an exec-mask region, scalar instructions and a scheduling boundary)
    const bool live = (t < T) & addr_unmasked(job, b, tl) & !inactive;
    const float g = which == 0 ? load_f32(static_cast<const Scalar *>(job.gamma) + bh * T + tl) : 0.f;
    // this lane's record of event 0; event k is k * Tp records further (a
    // uniform 32-bit step, not a 64-bit index product per event)
    WriteRec *wr0 = job.wrec + bh * K * Tp + t;
    ReadRec *rr0 = job.rrec + bh * K * Tp + t;
    auto one = [&](int k) {
        int c;
        float v;
        get(k, c, v);
        int o = c - shift;
        o = o < 0 ? o + A : o;
        const bool act = live & (v != 0.f);
        if (which == 0) {
            // alpha on every lane, kept through an opaque bit mask (a select
            // of the quotient would be turned back into a branch around the
            // division)
            const uint32_t m = opaque(act ? ~0u : 0u);
            const float al = __uint_as_float((__float_as_uint(gsu_alpha(v, g)) & m) | (__float_as_uint(1.f) & ~m));
            wr0[static_cast<uint32_t>(k * Tp)] = WriteRec{act ? o : -2, act ? v : 0.f, al, __int_as_float(overlap)};
        } else {
            rr0[static_cast<uint32_t>(k * Tp)] = act ? ReadRec{o, v} : ReadRec{-1, 0.f};
        }
    };
    if constexpr (KM > 0) {
#pragma unroll
        for (int k = 0; k < KM; ++k)
            if (k < K)
                one(k);
    } else {
        for (int k = 0; k < K; ++k)
            one(k);
    }
}

// FAST: P == NP and the logits are read through a buffer resource with
// 32-bit lane offsets (the host checks that every offset fits); otherwise
// any P <= NP, through 64-bit pointers.
template<typename Scalar, int NP, int KM, bool FAST>
// Occupancy: the per-lane search holds its digit in registers (about 210
// VGPRs unconstrained, two waves per SIMD). Capping it at 168 (three waves)
// hides more of the sort chains' latency at the cost of a few spills at
// K = 16. With the staircase merge, config 2 (K = 8) fits 168 without
// spilling, and measures faster there than capped at 128 with a few spills
// (four waves per SIMD): 0.086 -> 0.081 ms.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void topk_addr_lane_kernel(
    const AddrJob job) {
    const AddrSource &src = job.src[blockIdx.y];
    const int T = job.T, H = job.H, U = job.U, P = job.P, A = job.A;
    const bool rec_mode = job.wrec != nullptr;
    const int Tg = rec_mode ? scan_t_pad(T) : T;  // record mode also writes the padding tokens
    const int64_t n = static_cast<int64_t>(job.B) * job.H * Tg;
    const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (gid >= n)
        return;
    const int t = static_cast<int>(gid % Tg);
    const int tl = t < T ? t : T - 1;
    const int64_t bh = gid / Tg;
    const int h = static_cast<int>(bh % H);
    const int b = static_cast<int>(bh / H);
    const Scalar *base = static_cast<const Scalar *>(src.addr) + bh * static_cast<int64_t>(U * P) * T + tl;

    float mv[KM];  // sorted top-KM scores
    int mi[KM];    // their content indices
    uint32_t ok[KM];
    bool found;
    if constexpr (FAST) {
        // resource based at the first active lane's logits: later lanes sit at
        // equal or higher addresses (same or later (b, h, t)), within
        // 2 * U * P * T elements of it
        // (readfirstlane returns a signed int: widen each half through
        // uint32_t, or a low half with bit 31 set would sign-extend over the
        // high half)
        const uint64_t mine = reinterpret_cast<uint64_t>(base);
        const uint32_t first_hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(mine >> 32)));
        const uint32_t first_lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(mine)));
        const uint64_t first = (static_cast<uint64_t>(first_hi) << 32) | first_lo;
        const uint64_t end = reinterpret_cast<uint64_t>(static_cast<const Scalar *>(src.addr) +
                                                        static_cast<int64_t>(job.B) * H * U * P * T);
        const uint64_t span = end - first;
        const int records = span < 0x7fffffffull ? static_cast<int>(span) : 0x7fffffff;
        const BufferLogits<Scalar> load{
            __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void *>(first), 0, records, kBufWord3),
            static_cast<int>(mine - first), T * static_cast<int>(sizeof(Scalar)), P};
        found = lane_search<Scalar, NP, KM, true>(load, U, P, mv, mi, ok);
    } else {
        const GlobalLogits<Scalar> load{base, T, P};
        found = lane_search<Scalar, NP, KM, false>(load, U, P, mv, mi, ok);
    }
    const bool inactive = !found;

    const int K = src.top_k;
    // log-sum-exp of the selected scores, computed on every lane and kept
    // where it applies (no divergent branch)
    // (exponentials as exp2 of a prescaled argument, one transcendental
    // instruction each, as the digits' log-sum-exps take them)
    constexpr float kLog2e = 1.4426950408889634f;
    float sum = 0.f;
#pragma unroll
    for (int k = KM - 1; k >= 0; --k)
        if (k < K)
            sum += __builtin_amdgcn_exp2f((mv[k] - mv[0]) * kLog2e);
    const bool norm = (src.re_norm != 0.f) & !inactive & (mv[0] > kNegInf);
    const float lse = norm ? mv[0] + log_sum(sum) : 0.f;
    const int shift = h < job.embed_num ? pos_mod(job.position_ids[static_cast<int64_t>(b) * T + tl], A) : 0;
    if (rec_mode) {
        // Overlap flags of the write address, bit d - 1 for d = 1, 2, 3:
        // whether a written slot of this token is also written by token
        // t - d (decoded d lanes back; in another wave for the first d
        // lanes, so assumed). The scan loads the rows of up to four tokens
        // before their writes and loads a token's rows again only when they
        // may have been written within its group.
        int overlap = 0;
        if (blockIdx.y == 0) {
            const bool live = (t < T) & addr_unmasked(job, b, tl) & !inactive;
            // this token's write slots (-1: none); the tokens before post
            // theirs with -2 for none, which never matches
            int mine[KM], post[KM];
#pragma unroll
            for (int k = 0; k < KM; ++k) {
                int o = mi[k] - shift;
                o = o < 0 ? o + A : o;
                const bool on = live & (k < K);
                mine[k] = on ? o : -1;
                post[k] = on ? o : -2;
            }
            const int wl = static_cast<int>(threadIdx.x & (kWave - 1));
#pragma unroll
            for (int d = 1; d <= 3; ++d) {
                int prev[KM];
#pragma unroll
                for (int k = 0; k < KM; ++k)
                    prev[k] = __shfl_up(post[k], d);
                bool hit = false;
#pragma unroll
                for (int k = 0; k < KM; ++k)
#pragma unroll
                    for (int k2 = 0; k2 < KM; ++k2)
                        hit |= mine[k] == prev[k2];
                overlap |= ((t >= d) & (hit | (wl < d))) ? 1 << (d - 1) : 0;
            }
        }
        write_records<Scalar, KM>(job, blockIdx.y, bh, b, t, tl, inactive, [&](int k, int &c, float &v) {
            c = mi[k];
            v = __builtin_amdgcn_exp2f((mv[k] - src.re_norm * lse) * kLog2e);
        }, K, shift, overlap);
        return;
    }
    const int idx_base = (job.encode_batch_idx ? static_cast<int>(bh) : h) * A;
    const int64_t row0 = (bh * job.k_total + src.k_off) * static_cast<int64_t>(T) + t;
    int *ip = job.idx_out + row0;  // event k at k * T (a uniform 32-bit step)
    float *vp = job.val_out + row0;
#pragma unroll
    for (int k = 0; k < KM; ++k) {
        if (k < K) {
            const int c = inactive ? k : mi[k];
            const float val = inactive ? 0.f : __builtin_amdgcn_exp2f((mv[k] - src.re_norm * lse) * kLog2e);
            int o = c - shift;
            o = o < 0 ? o + A : o;
            ip[static_cast<uint32_t>(k * T)] = idx_base + o;
            vp[static_cast<uint32_t>(k * T)] = src.sign * val;
        }
    }
}

// Workgroup-per-address search: exact (STAIR false: all A scores in LDS,
// NA = pow2 >= A) or the staircase search for slot spaces of any size (STAIR
// true: NA is the candidate buffer NC).
template<typename Scalar, bool STAIR>
__global__ __launch_bounds__(256) void topk_addr_bruteforce_kernel(const AddrJob job, int NA, int NPD) {
    extern __shared__ float smem[];
    const AddrSource &src = job.src[blockIdx.y];
    const int T = job.T, H = job.H, U = job.U, P = job.P, A = job.A;
    const bool rec_mode = job.wrec != nullptr;
    const int Tg = rec_mode ? scan_t_pad(T) : T;
    const int64_t gid = blockIdx.x;  // (b, h, t)
    const int t = static_cast<int>(gid % Tg);
    const int tl = t < T ? t : T - 1;
    const int64_t bh = gid / Tg;
    const int h = static_cast<int>(bh % H);
    const int b = static_cast<int>(bh / H);
    const Scalar *base = static_cast<const Scalar *>(src.addr) + bh * static_cast<int64_t>(U * P) * T + tl;

    const int K = src.top_k;
    float *lg = smem;
    float *ex = lg + U * P;
    int *di = reinterpret_cast<int *>(ex + U * NPD);  // staircase only
    float *sv = STAIR ? reinterpret_cast<float *>(di + U * NPD) : ex + U * NPD;
    int *si = reinterpret_cast<int *>(sv + NA);
    float *pv = reinterpret_cast<float *>(si + NA);    // staircase only: K each, then K + 1
    int *pi = reinterpret_cast<int *>(pv + K);
    int *off = pi + K;
    __shared__ int s_flag;
    __shared__ float s_lse;
    bool inactive;
    if constexpr (STAIR)
        inactive = block_search_stair(base, static_cast<int64_t>(T), U, P, K, NPD, NA, lg, ex, di, sv, si, pv, pi, off,
                                      &s_flag);
    else
        inactive = block_search_exact(base, static_cast<int64_t>(T), U, P, A, NA, NPD, lg, ex, sv, si, &s_flag);
    const int tid = threadIdx.x;
    if (tid == 0)
        s_lse = (src.re_norm != 0.f && !inactive) ? topk_lse_serial(sv, K) : 0.f;
    __syncthreads();
    const int shift = h < job.embed_num ? pos_mod(job.position_ids[static_cast<int64_t>(b) * T + tl], A) : 0;
    if (rec_mode) {
        if (tid == 0)
            write_records<Scalar, 0>(job, blockIdx.y, bh, b, t, tl, inactive, [&](int k, int &c, float &v) {
                c = si[k];
                v = expf(sv[k] - src.re_norm * s_lse);
            }, K, shift, 7);  // overlaps with tokens t - 1 .. t - 3 not computed: assumed
        return;
    }
    const int idx_base = (job.encode_batch_idx ? static_cast<int>(bh) : h) * A;
    const int64_t row0 = (bh * job.k_total + src.k_off) * static_cast<int64_t>(T) + t;
    for (int k = tid; k < K; k += blockDim.x) {
        const int c = inactive ? k : si[k];
        const float val = inactive ? 0.f : expf(sv[k] - src.re_norm * s_lse);
        int o = c - shift;
        o = o < 0 ? o + A : o;
        job.idx_out[row0 + static_cast<int64_t>(k) * T] = idx_base + o;
        job.val_out[row0 + static_cast<int64_t>(k) * T] = src.sign * val;
    }
}

int pow2_at_least(int x) {
    int p = 1;
    while (p < x)
        p <<= 1;
    return p;
}

int grid_t(const AddrJob &job) { return job.wrec ? scan_t_pad(job.T) : job.T; }

}  // namespace

// Candidate buffer of the staircase search: a power of two holding every
// candidate of one step (the prefix list is at most top_k long) and the
// initial digit list.
int stair_buffer(int P, int K, int NPD) {
    const int c = stair_count(K, P, K);
    return pow2_at_least(c > NPD ? c : NPD);
}

namespace {

template<typename T, int NP, int KM>
hipError_t launch_lane(const AddrJob &job, hipStream_t stream) {
    const int64_t n = static_cast<int64_t>(job.B) * job.H * grid_t(job);
    const dim3 grid(static_cast<unsigned>((n + 255) / 256), job.n_src);
    // a wave spans at most two (b, h) rows: lane offsets stay below
    // 2 * U * P * T elements from the wave's first lane
    const int64_t span = 2 * static_cast<int64_t>(job.U) * job.P * job.T * static_cast<int64_t>(sizeof(T)) + 256;
    if (span <= 0x7fffffff && job.P == NP)
        hipLaunchKernelGGL((topk_addr_lane_kernel<T, NP, KM, true>), grid, dim3(256), 0, stream, job);
    else
        hipLaunchKernelGGL((topk_addr_lane_kernel<T, NP, KM, false>), grid, dim3(256), 0, stream, job);
    return hipGetLastError();
}

template<typename T, int NP>
hipError_t launch_lane_k(const AddrJob &job, int km, hipStream_t stream) {
    switch (km) {
        case 4: return launch_lane<T, NP, 4>(job, stream);
        case 8: return launch_lane<T, NP, 8>(job, stream);
        default: return launch_lane<T, NP, 16>(job, stream);
    }
}

template<typename T>
hipError_t launch_typed(const AddrJob &job, hipStream_t stream, const char **why) {
    int kmax = 0;
    for (int s = 0; s < job.n_src; ++s)
        kmax = job.src[s].top_k > kmax ? job.src[s].top_k : kmax;
    const int np = pow2_at_least(job.P < 4 ? 4 : job.P);
    const int km = pow2_at_least(kmax < 4 ? 4 : kmax);
    const bool lane_ok = np <= 64 && km <= 16;
    if (lane_ok) {
        switch (np) {
            case 4: return launch_lane_k<T, 4>(job, km, stream);
            case 8: return launch_lane_k<T, 8>(job, km, stream);
            case 16: return launch_lane_k<T, 16>(job, km, stream);
            case 32: return launch_lane_k<T, 32>(job, km, stream);
            default: return launch_lane_k<T, 64>(job, km, stream);
        }
    }
    const int NA = pow2_at_least(job.A);
    const int NPD = pow2_at_least(job.P);
    const size_t lds = static_cast<size_t>(job.U) * job.P * 4 + static_cast<size_t>(job.U) * NPD * 4 + static_cast<size_t>(NA) * 8;
    const int64_t n = static_cast<int64_t>(job.B) * job.H * grid_t(job);
    if (n > 0x7fffffff) {
        *why = "address decoder: B*H*T too large for the workgroup search grid";
        return hipErrorInvalidValue;
    }
    const dim3 grid(static_cast<unsigned>(n), job.n_src);
    if (lds <= 96 * 1024) {
        hipLaunchKernelGGL((topk_addr_bruteforce_kernel<T, false>), grid, dim3(256), lds, stream, job, NA, NPD);
        return hipGetLastError();
    }
    // wider slot spaces: the staircase search, any A, top_k <= 128
    if (kmax > 128 || NPD > 1024) {
        *why = "address decoder: slot spaces beyond the exact LDS search (A > 8192) take top_k <= 128 and P <= 1024";
        return hipErrorInvalidValue;
    }
    const int NC = stair_buffer(job.P, kmax, NPD);
    const size_t lds_s = static_cast<size_t>(job.U) * job.P * 4 + static_cast<size_t>(job.U) * NPD * 8 +
                         static_cast<size_t>(NC) * 8 + static_cast<size_t>(kmax) * 8 + static_cast<size_t>(kmax + 1) * 4;
    if (lds_s > 96 * 1024) {
        *why = "address decoder: staircase search scratch exceeds LDS (U * P too large)";
        return hipErrorInvalidValue;
    }
    hipLaunchKernelGGL((topk_addr_bruteforce_kernel<T, true>), grid, dim3(256), lds_s, stream, job, NC, NPD);
    return hipGetLastError();
}

// ---- backward (reference: csrc/ram_attn_topk_addr.cu:119-226)
//
// With v_k the selected weights, D_k = dL/dv_k * v_k is the gradient of the
// score s_k = sum_u L_u[d_u(k)] when re_norm = 0; re-normalisation
// v_k = exp(s_k - r LSE) subtracts r p_k sum_j D_j with p_k = v_k / sum v.
// Through the per-digit log-softmax L_u = x_u - logsumexp(x_u):
//     dL/dx_u[q] = sum_{k: d_u(k) = q} D_k - softmax(x_u)[q] (1 - r) sum_k D_k,
// since the p_k sum to one. The selection itself carries no gradient, and an
// inactive address (all weights 0) gets none. One lane per (b, h, t); the
// logits of a digit are read coalesced across the lanes' consecutive t,
// once into registers when P <= PR, else in three passes (max, sum,
// gradient). KM > 0 keeps the K terms in registers; KM = 0 streams them for
// any K. BUF (P == PR, and every lane's offsets from the wave's first lane
// fit in 31 bits): the logits and their gradients go through buffer
// resources based at the wave's first lane, with 32-bit lane offsets, so the
// 2 * U * P per-lane addresses are not kept in (spilled) scalar registers.
template<typename Scalar, int KM, int PR, bool BUF = false>
__global__ __launch_bounds__(256) void topk_addr_backward_kernel(const AddrBwdJob job) {
    static_assert(!BUF || PR > 0, "buffer resources: the logits held in registers");
    const int T = job.T, H = job.H, A = job.A, P = job.P, U = job.U, K = job.K;
    const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (gid >= static_cast<int64_t>(job.B) * H * T)
        return;
    const int t = static_cast<int>(gid % T);
    const int64_t bh = gid / T;
    const int b = static_cast<int>(bh / H), h = static_cast<int>(bh % H);
    const int64_t row0 = (bh * job.k_total + job.k_off) * T + t;  // event k at row0 + k * T
    const float re = job.re_norm;
    const int shift = h < job.embed_num ? pos_mod(job.position_ids[static_cast<int64_t>(b) * T + t], A) : 0;
    auto weight = [&](int k) { return job.sign * job.val[row0 + static_cast<int64_t>(k) * T]; };
    auto dscore = [&](int k) { return job.grad_val[row0 + static_cast<int64_t>(k) * T] * weight(k); };
    auto content = [&](int k) {
        const int o = job.idx[row0 + static_cast<int64_t>(k) * T] % A;  // drops a (b*H + h)*A encoding
        const int c = o + shift;
        return c >= A ? c - A : c;
    };
    float dsum = 0.f, vsum = 0.f;
    float D[KM > 0 ? KM : 1];
    float wk[KM > 0 ? KM : 1];
    int c[KM > 0 ? KM : 1];
    if constexpr (KM > 0) {
        // every lane loads all KM events (clamped to the last one), so the
        // loads issue together instead of one branch and wait each
#pragma unroll
        for (int k = 0; k < KM; ++k) {
            const bool on = k < K;
            const int kc = on ? k : K - 1;
            const float w = weight(kc);
            const float d = job.grad_val[row0 + static_cast<int64_t>(kc) * T] * w;
            const int ck = content(kc);
            wk[k] = on ? w : 0.f;
            D[k] = on ? d : 0.f;
            c[k] = on ? ck : -1;
            dsum += D[k];
            vsum += wk[k];
        }
    } else {
        for (int k = 0; k < K; ++k) {
            dsum += dscore(k);
            vsum += weight(k);
        }
    }
    // (conditions bitwise and corrections selected, not branched on: a
    // lane-dependent branch is an exec-mask region)
    const bool renorm = (re != 0.f) & (vsum > 0.f);
    auto dk = [&](int k) {  // the re-normalised D_k (streaming form)
        const float d = dscore(k);
        return renorm ? d - re * (weight(k) / vsum) * dsum : d;
    };
    if constexpr (KM > 0) {
#pragma unroll
        for (int k = 0; k < KM; ++k) {
            // (a bit select through an opaque mask: a select of the quotient
            // would be turned back into a branch around the division)
            const float dr = D[k] - re * (wk[k] / vsum) * dsum;
            const uint32_t m = opaque((renorm & (k < K)) ? ~0u : 0u);
            D[k] = __uint_as_float((__float_as_uint(dr) & m) | (__float_as_uint(D[k]) & ~m));
        }
    }
    const float dsoft = (1.f - re) * dsum;
    const Scalar *xp = static_cast<const Scalar *>(job.addr) + bh * U * P * static_cast<int64_t>(T) + t;
    Scalar *gp = static_cast<Scalar *>(job.grad_addr) + bh * U * P * static_cast<int64_t>(T) + t;
    // BUF: resources based at the first active lane's logit and gradient
    // (later lanes are at equal or higher addresses, within 2 * U * P * T
    // elements: a wave spans at most two (b, h) rows). readfirstlane returns
    // a signed int: each half is widened through uint32_t.
    auto first_of = [](uint64_t mine) {
        const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(mine >> 32)));
        const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(mine)));
        return (static_cast<uint64_t>(hi) << 32) | lo;
    };
    const uint64_t xmine = reinterpret_cast<uint64_t>(xp), gmine = reinterpret_cast<uint64_t>(gp);
    const uint64_t xfirst = BUF ? first_of(xmine) : xmine, gfirst = BUF ? first_of(gmine) : gmine;
    [[maybe_unused]] const auto xrs =
        __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void *>(xfirst), 0, 0x7fffffff, kBufWord3);
    [[maybe_unused]] const auto grs =
        __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void *>(gfirst), 0, 0x7fffffff, kBufWord3);
    [[maybe_unused]] const int xoff = static_cast<int>(xmine - xfirst), goff = static_cast<int>(gmine - gfirst);
    [[maybe_unused]] const int step = T * static_cast<int>(sizeof(Scalar));
    int stride = 1;
    for (int u = 0; u < U; ++u, stride *= P) {
        const Scalar *xu = xp + static_cast<int64_t>(u) * P * T;
        Scalar *gu = gp + static_cast<int64_t>(u) * P * T;
        float xr[PR > 0 ? PR : 1];  // the digit's logits, then their exponentials
        float mx = -__builtin_huge_valf();
        if constexpr (BUF) {
#pragma unroll
            for (int q = 0; q < PR; ++q) {
                const int o = xoff + (u * PR + q) * step;
                uint32_t bits;
                if constexpr (sizeof(Scalar) == 2)
                    bits = __builtin_amdgcn_raw_buffer_load_b16(xrs, o, 0, 0);
                else
                    bits = __builtin_amdgcn_raw_buffer_load_b32(xrs, o, 0, 0);
                xr[q] = bits_f32<Scalar>(bits);
                mx = fmaxf(mx, xr[q]);
            }
        } else if constexpr (PR > 0) {
#pragma unroll
            for (int q = 0; q < PR; ++q) {
                xr[q] = load_f32(xu + static_cast<int64_t>(q < P ? q : P - 1) * T);
                mx = q < P ? fmaxf(mx, xr[q]) : mx;
            }
        } else {
            for (int q = 0; q < P; ++q)
                mx = fmaxf(mx, load_f32(xu + static_cast<int64_t>(q) * T));
        }
        const bool live = mx > -__builtin_huge_valf();
        float se = 0.f;
        if constexpr (PR > 0) {
#pragma unroll
            for (int q = 0; q < PR; ++q) {
                // exp2 of a prescaled argument (one transcendental
                // instruction), as the forward's log-sum-exp takes it
                const float e = __builtin_amdgcn_exp2f((xr[q] - mx) * 1.4426950408889634f);
                xr[q] = (live & (q < P)) ? e : 0.f;
                se += xr[q];
            }
        } else {
            for (int q = 0; q < P; ++q)
                se += live ? expf(load_f32(xu + static_cast<int64_t>(q) * T) - mx) : 0.f;
        }
        const float scale = live ? dsoft / se : 0.f;
        int du[KM > 0 ? KM : 1];
        if constexpr (KM > 0) {
            // digit u of each content index: shifts when P is a power of two
            // (a uniform branch), else integer division
            if ((P & (P - 1)) == 0) {
                const int sh = u * __builtin_ctz(static_cast<unsigned>(P));
#pragma unroll
                for (int k = 0; k < KM; ++k)
                    du[k] = c[k] < 0 ? -1 : (c[k] >> sh) & (P - 1);
            } else {
#pragma unroll
                for (int k = 0; k < KM; ++k)
                    du[k] = c[k] < 0 ? -1 : (c[k] / stride) % P;
            }
        }
        auto grad_of = [&](int q) {
            float g = 0.f;
            if constexpr (KM > 0) {
#pragma unroll
                for (int k = 0; k < KM; ++k)
                    g += du[k] == q ? D[k] : 0.f;
            } else {
                for (int k = 0; k < K; ++k)
                    g += (content(k) / stride) % P == q ? dk(k) : 0.f;
            }
            return g;
        };
        if constexpr (BUF) {
#pragma unroll
            for (int q = 0; q < PR; ++q) {
                const int o = goff + (u * PR + q) * step;
                const float v = grad_of(q) - xr[q] * scale;
                if constexpr (sizeof(Scalar) == 4)
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), grs, o, 0, 0);
                else if constexpr (__is_same(Scalar, bf16_t))
                    __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16_bits(v), grs, o, 0, 0);
                else
                    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, static_cast<_Float16>(v)), grs, o,
                                                          0, 0);
            }
        } else if constexpr (PR > 0) {
            if (P == PR) {  // the common case: stores without a branch each
#pragma unroll
                for (int q = 0; q < PR; ++q)
                    store_f32(gu + static_cast<int64_t>(q) * T, grad_of(q) - xr[q] * scale);
            } else {
#pragma unroll
                for (int q = 0; q < PR; ++q)
                    if (q < P)
                        store_f32(gu + static_cast<int64_t>(q) * T, grad_of(q) - xr[q] * scale);
            }
        } else {
            for (int q = 0; q < P; ++q) {
                const float sm = live ? expf(load_f32(xu + static_cast<int64_t>(q) * T) - mx) : 0.f;
                store_f32(gu + static_cast<int64_t>(q) * T, grad_of(q) - sm * scale);
            }
        }
    }
}

template<typename T>
hipError_t launch_backward_typed(const AddrBwdJob &job, hipStream_t stream) {
    const int64_t n = static_cast<int64_t>(job.B) * job.H * job.T;
    const dim3 grid(static_cast<unsigned>((n + 255) / 256)), blk(256);
    // a digit's logits fit in registers up to P = 32; P = 16 has its own
    // instance, whose stores need no per-logit branch
    // offsets from a wave's first lane stay below 2 * U * P * T elements
    const bool buf = 2 * static_cast<int64_t>(job.U) * job.P * job.T * static_cast<int64_t>(sizeof(T)) + 256 <=
                     0x7fffffff;
#define RAMNET_ADDR_BWD(KM)                                                                          \
    do {                                                                                             \
        if (job.P == 16 && buf)                                                                      \
            hipLaunchKernelGGL((topk_addr_backward_kernel<T, KM, 16, true>), grid, blk, 0, stream, job); \
        else if (job.P == 32 && buf)                                                                 \
            hipLaunchKernelGGL((topk_addr_backward_kernel<T, KM, 32, true>), grid, blk, 0, stream, job); \
        else if (job.P == 16)                                                                        \
            hipLaunchKernelGGL((topk_addr_backward_kernel<T, KM, 16>), grid, blk, 0, stream, job);   \
        else if (job.P <= 32)                                                                        \
            hipLaunchKernelGGL((topk_addr_backward_kernel<T, KM, 32>), grid, blk, 0, stream, job);   \
        else                                                                                         \
            hipLaunchKernelGGL((topk_addr_backward_kernel<T, KM, 0>), grid, blk, 0, stream, job);    \
    } while (0)
    if (job.K <= 8)
        RAMNET_ADDR_BWD(8);
    else if (job.K <= 16)
        RAMNET_ADDR_BWD(16);
    else if (job.K <= 32)
        RAMNET_ADDR_BWD(32);
    else
        RAMNET_ADDR_BWD(0);
#undef RAMNET_ADDR_BWD
    return hipGetLastError();
}

}  // namespace

hipError_t launch_topk_addr_backward(const AddrBwdJob &job, hipStream_t stream, const char **why) {
    if (static_cast<int64_t>(job.B) * job.H * job.T == 0)
        return hipSuccess;
    switch (job.dtype) {
        case kF32: return launch_backward_typed<float>(job, stream);
        case kF16: return launch_backward_typed<_Float16>(job, stream);
        case kBF16: return launch_backward_typed<bf16_t>(job, stream);
        default: *why = "address decoder backward: unsupported dtype"; return hipErrorInvalidValue;
    }
}

hipError_t launch_topk_addr(const AddrJob &job, hipStream_t stream, const char **why) {
    if (static_cast<int64_t>(job.B) * job.H * job.T == 0)
        return hipSuccess;
    switch (job.dtype) {
        case kF32: return launch_typed<float>(job, stream, why);
        case kF16: return launch_typed<_Float16>(job, stream, why);
        case kBF16: return launch_typed<bf16_t>(job, stream, why);
        default: *why = "address decoder: unsupported dtype"; return hipErrorInvalidValue;
    }
}

}  // namespace ramnet
