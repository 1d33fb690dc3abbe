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
    // Hide from the optimiser that slot and weight are 0 on lanes past K.
    // Later stages read event 0 with v_readlane on exactly those lanes
    // (`lane < Kw ? own slot : event 0's slot`); hipcc 7.2 turned that select
    // into a branch over the lanes past Kw, rebuilt the slot there as the
    // constant 0 and read lane 0 of it, so those lanes stored event 0's mass
    // into slot 0. The barrier is volatile so that it stays here, where every
    // lane executes it.
    asm volatile("" : "+v"(slot), "+v"(val));
}

// Value of `v` on lane L (L uniform; a constant after unrolling), as a
// wave-uniform scalar.
__device__ __forceinline__ float lane_f(float v, int L) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), L));
}
__device__ __forceinline__ int lane_i(int v, int L) { return __builtin_amdgcn_readlane(v, L); }

// Channels of one lane. FULLC (C == 64 * kCpl, pointers aligned to the
// vector width): the kCpl consecutive channels lane * kCpl ..., moved with
// one vector access per row. Otherwise channels lane + 64 j, clamped into
// the row, one dword each. coff[j] is channel j's byte offset in a row (for
// FULLC only coff[0] is used).
template<int kCpl, bool FULLC>
__device__ __forceinline__ void lane_channels(int lane, int C, int *coff) {
#pragma unroll
    for (int j = 0; j < kCpl; ++j) {
        const int c = FULLC ? lane * kCpl + j : lane + j * kWave;
        coff[j] = (FULLC || c < C ? c : C - 1) * 4;
    }
}
template<int kCpl, bool FULLC>
__device__ __forceinline__ bool owns(int lane, int j, int C) {
    return FULLC || lane + j * kWave < C;
}

template<int kCpl, bool FULLC>
__device__ __forceinline__ void row_load(__amdgpu_buffer_rsrc_t r, const int *coff, int so, float *v) {
    if constexpr (FULLC && kCpl == 2) {
        const auto q = __builtin_amdgcn_raw_buffer_load_b64(r, coff[0], so, 0);
        v[0] = __uint_as_float(q[0]);
        v[1] = __uint_as_float(q[1]);
    } else if constexpr (FULLC && kCpl == 4) {
        const auto q = __builtin_amdgcn_raw_buffer_load_b128(r, coff[0], so, 0);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            v[j] = __uint_as_float(q[j]);
    } else {
#pragma unroll
        for (int j = 0; j < kCpl; ++j)
            v[j] = buf_load_f32(r, coff[j], so);
    }
}
template<int kCpl, bool FULLC>
__device__ __forceinline__ void row_store(const float *v, __amdgpu_buffer_rsrc_t r, const int *coff, int so, int lane,
                                          int C) {
    if constexpr (FULLC && kCpl == 2) {
        using u2 = __attribute__((ext_vector_type(2))) unsigned int;
        const u2 q = {__float_as_uint(v[0]), __float_as_uint(v[1])};
        __builtin_amdgcn_raw_buffer_store_b64(q, r, coff[0], so, 0);
    } else if constexpr (FULLC && kCpl == 4) {
        using u4 = __attribute__((ext_vector_type(4))) unsigned int;
        const u4 q = {__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])};
        __builtin_amdgcn_raw_buffer_store_b128(q, r, coff[0], so, 0);
    } else {
#pragma unroll
        for (int j = 0; j < kCpl; ++j)
            if (owns<kCpl, FULLC>(lane, j, C))
                buf_store_f32(v[j], r, coff[j], so);
    }
}

// Storage bits of one lane's kCpl values of x, converted when read (a
// prefetch waits for nothing until the values are used).
template<typename T, int kCpl, bool FULLC>
struct XRaw {
    static constexpr int kWords = FULLC ? (kCpl * static_cast<int>(sizeof(T)) + 3) / 4 : kCpl;
    uint32_t w[kWords];

    __device__ __forceinline__ void load(const T *row, const int *coff, int lane) {
        if constexpr (FULLC) {
            const uint32_t *p = reinterpret_cast<const uint32_t *>(row + lane * kCpl);
            if constexpr (kWords == 1) {
                w[0] = *p;
            } else if constexpr (kWords == 2) {
                const uint2 q = *reinterpret_cast<const uint2 *>(p);
                w[0] = q.x;
                w[1] = q.y;
            } else {
                const uint4 q = *reinterpret_cast<const uint4 *>(p);
                w[0] = q.x;
                w[1] = q.y;
                w[2] = q.z;
                w[3] = q.w;
            }
        } else {
#pragma unroll
            for (int j = 0; j < kCpl; ++j)
                w[j] = load_bits(row + coff[j] / 4);
        }
    }
    __device__ __forceinline__ float get(int j) const {
        if constexpr (FULLC && sizeof(T) == 2)
            return bits_f32<T>((j & 1) ? w[j / 2] >> 16 : w[j / 2] & 0xffffu);
        else
            return bits_f32<T>(w[j]);
    }
};

template<typename T>
__device__ __forceinline__ uint32_t f32_storage_bits(float v) {
    if constexpr (sizeof(T) == 4)
        return __float_as_uint(v);
    else if constexpr (__is_same(T, bf16_t))
        return f32_to_bf16_bits(v);
    else
        return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
}

// y of one lane's channels, in T.
template<typename T, int kCpl, bool FULLC>
__device__ __forceinline__ void store_y(T *row, const float *v, int lane, int C) {
    if constexpr (FULLC) {
        uint32_t *p = reinterpret_cast<uint32_t *>(row + lane * kCpl);
        if constexpr (sizeof(T) == 4) {
            if constexpr (kCpl == 2)
                *reinterpret_cast<uint2 *>(p) = make_uint2(__float_as_uint(v[0]), __float_as_uint(v[1]));
            else
                *reinterpret_cast<uint4 *>(p) = make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]),
                                                           __float_as_uint(v[2]), __float_as_uint(v[3]));
        } else {
            uint32_t q[kCpl / 2];
#pragma unroll
            for (int i = 0; i < kCpl / 2; ++i)
                q[i] = f32_storage_bits<T>(v[2 * i]) | (f32_storage_bits<T>(v[2 * i + 1]) << 16);
            if constexpr (kCpl == 2)
                *p = q[0];
            else
                *reinterpret_cast<uint2 *>(p) = make_uint2(q[0], q[1]);
        }
    } else {
#pragma unroll
        for (int j = 0; j < kCpl; ++j)
            if (owns<kCpl, FULLC>(lane, j, C))
                store_f32(row + lane + j * kWave, v[j]);
    }
}

// The fast path in four stages, shared by the single-step kernel and the
// multi-step kernel. Events live one per lane: write event k on lane k, read
// event k on lane RB + k (RB = 32 when the two addresses share the wave as
// half-waves, else 0 with separate registers). The event math (mass, alpha,
// gain) runs lane parallel; each row's scalars are then broadcast with
// v_readlane. Rows and masses of one (b, h) are addressed through buffer
// resources (32-bit offsets; the launcher keeps A * C * 4 below 2^31).
template<int KE, int kCpl>
struct StepState {
    int ow, orr;             // write / read event slot of this lane
    float vw, vr;            // their weights
    float emw, emr;          // their pre-step masses
    int fwd[KE];             // write event on read k's slot, or -1
    bool any_fwd;            // some read takes a row this step writes
    float wrow[KE][kCpl];    // pre-step rows of the write events
    float rrow[KE][kCpl];    // pre-step rows of the read events
};

// Stage 1: decode both addresses into per-lane events and the LDS slot
// tables (s_ws/s_rs/s_wv) that stage 3 reads.
template<typename T, int GW, int KE, int kCpl>
__device__ __forceinline__ void decode_events(const DecodeJob &job, const GroupLogits<T> &lw,
                                              const GroupLogits<T> &lr, int shift, int lane, int *s_ws, int *s_rs,
                                              float *s_wv, StepState<KE, kCpl> &st) {
    const int A = job.A, U = job.U, P = job.P, Kw = job.Kw, Kr = job.Kr;
    float v;
    int c;
    if constexpr (GW == 32) {
        const int half = lane >> 5, li = lane & 31;
        const int K = half ? Kr : Kw;
        const bool inactive = group_search<T, 32>(lw, U, P, K, li, v, c);
        lane_event(v, c, inactive, K, half ? job.r_re_norm : job.w_re_norm, li, half * 32, shift, A, st.ow, st.vw);
        st.orr = st.ow;
        st.vr = st.vw;
        if (li < KE) {
            (half ? s_rs : s_ws)[li] = st.ow;
            if (!half)
                s_wv[li] = st.vw;
        }
    } else {
        bool inactive = group_search<T, 64>(lw, U, P, Kw, lane, v, c);
        lane_event(v, c, inactive, Kw, job.w_re_norm, lane, 0, shift, A, st.ow, st.vw);
        inactive = group_search<T, 64>(lr, U, P, Kr, lane, v, c);
        lane_event(v, c, inactive, Kr, job.r_re_norm, lane, 0, shift, A, st.orr, st.vr);
        if (lane < KE) {
            s_ws[lane] = st.ow;
            s_wv[lane] = st.vw;
            s_rs[lane] = st.orr;
        }
    }
}

// Stage 2: one batch of requests for the events' masses and rows (row k's
// offset is a scalar). Loads come from clamped in-bounds slots, unguarded.
// Write event k of the row stages: k itself, or, past a top-k below KE, the
// last real event (so that its row update repeats that event's store).
template<int KE, bool FULLK>
__device__ __forceinline__ int write_event(int k, int Kw) {
    return FULLK || k < Kw ? k : Kw - 1;
}

template<int GW, int KE, int kCpl, bool FULLC, bool FULLK>
__device__ __forceinline__ void issue_rows(__amdgpu_buffer_rsrc_t srs, __amdgpu_buffer_rsrc_t mrs, const int *coff,
                                           int rowb, int Kw, StepState<KE, kCpl> &st) {
    constexpr int RB = GW == 32 ? 32 : 0;
    st.emw = buf_load_f32(mrs, st.ow * 4, 0);
    st.emr = GW == 32 ? st.emw : buf_load_f32(mrs, st.orr * 4, 0);
#pragma unroll
    for (int k = 0; k < KE; ++k)
        row_load<kCpl, FULLC>(srs, coff, lane_i(st.ow, write_event<KE, FULLK>(k, Kw)) * rowb, st.wrow[k]);
#pragma unroll
    for (int k = 0; k < KE; ++k)
        row_load<kCpl, FULLC>(srs, coff, lane_i(st.orr, RB + k) * rowb, st.rrow[k]);
}

// Stage 3: forwarding, fwd[k] = the write event (nonzero weight) on read k's
// slot, or -1. One lane per (read, write) pair compares the slots; a ballot
// per 64 pairs collects the matches (top-K slots are distinct, so at most one
// write matches a read). The event tables are read unconditionally (both
// indices are below KE) and the conditions combined bitwise, so the
// comparison has no divergent branch. (One wave per workgroup: its LDS
// accesses complete in order, so the tables written in stage 1 are visible.)
template<int KE, int kCpl>
__device__ __forceinline__ void forward_map(const DecodeJob &job, int lane, const int *s_ws, const int *s_rs,
                                            const float *s_wv, StepState<KE, kCpl> &st) {
    __builtin_amdgcn_wave_barrier();
    static_assert((KE * KE) % kWave == 0, "forwarding rounds cover whole waves");
    uint64_t any = 0;
#pragma unroll
    for (int base = 0; base < KE * KE; base += kWave) {
        const int l = base + lane;
        const int k = (l / KE) % KE, j2 = l % KE;
        const int ws = s_ws[j2], rs = s_rs[k];
        const float wvj = s_wv[j2];
        const bool match = (j2 < job.Kw) & (k < job.Kr) & (wvj != 0.f) & (ws == rs);
        const uint64_t hits = __ballot(match);
        any |= hits;
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
                st.fwd[k2] = 30 - __builtin_clz(2u * bits + 1u);
            }
        }
    }
    st.any_fwd = any != 0;
}

// Stage 4: the K writes (masses, then rows), then the reads of the
// post-write state into y (`yrow`, C values). A step with valid == false (a
// masked batch row) has all its weights taken as 0, so its state is stored
// back unchanged and y is 0. A write event of weight 0 stores its row and
// mass back unchanged (gain 0); top-K slots are distinct, so no such store
// meets another write. Every memory instruction here executes on every path
// (lanes and events past top-k repeat a real event's store of the same
// value): the compiler's memory-counter waits then see the same number of
// requests on every path, which lets the multi-step kernel's waits skip
// this stage's stores.
template<typename T, int GW, int KE, int kCpl, bool FULLC, bool FULLK>
__device__ __forceinline__ void apply_step(const DecodeJob &job, const StepState<KE, kCpl> &st,
                                           const XRaw<T, kCpl, FULLC> &xr, float gamma, bool valid,
                                           __amdgpu_buffer_rsrc_t srs, __amdgpu_buffer_rsrc_t mrs, const int *coff,
                                           int rowb, int lane, float (*s_row)[kWave * kCpl], T *yrow) {
    constexpr int RB = GW == 32 ? 32 : 0;
    const int C = job.C, Kw = FULLK ? KE : job.Kw;
    float xv[kCpl];
#pragma unroll
    for (int j = 0; j < kCpl; ++j)
        xv[j] = xr.get(j);
    // write math, one write event per lane. e^-|gamma| is shared by the
    // events: alpha = num / den with the stable form of gsu_alpha, divided
    // with one Newton-refined reciprocal.
    const float vw = valid ? st.vw : 0.f;
    const bool gpos = gamma >= 0.f;
    const float eg = expf(gpos ? -gamma : gamma);
    const float cw = 1.f - vw;
    const float den = gpos ? fmaf(eg, cw, vw) : fmaf(eg, vw, cw);
    const float alpha = gsu_gain(gpos ? cw * eg : cw, den);
    const float m2 = vw != 0.f ? fmaf(alpha, st.emw, vw) : st.emw;
    const float gain = gsu_gain(vw, m2 + job.eps);
    const bool wlane = (GW == 32 ? lane < 32 : true) && lane < Kw;
    // lanes that are not write events store write event 0's mass again
    const int mso = wlane ? st.ow * 4 : lane_i(st.ow, 0) * 4;
    buf_store_f32(wlane ? m2 : lane_f(m2, 0), mrs, mso, 0);
    // every row load is in flight before the first update (the fence stops
    // the scheduler from sinking loads into the update branches, where each
    // would wait for its own data)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < KE; ++k) {
        const int e = write_event<KE, FULLK>(k, Kw);
        const float g = lane_f(gain, e);
        float upd[kCpl];
#pragma unroll
        for (int j = 0; j < kCpl; ++j)
            upd[j] = fmaf(g, xv[j] - st.wrow[k][j], st.wrow[k][j]);
        row_store<kCpl, FULLC>(upd, srs, coff, lane_i(st.ow, e) * rowb, lane, C);
    }

    // reads of the post-write state, summed in event order
    const float vr = valid ? st.vr : 0.f;
    float rv[KE];
#pragma unroll
    for (int k = 0; k < KE; ++k)
        rv[k] = lane_f(vr, RB + k);
    float acc[kCpl];
#pragma unroll
    for (int j = 0; j < kCpl; ++j)
        acc[j] = 0.f;
    float sr = 0.f, srm = 0.f;
    if (!(valid && st.any_fwd)) {
        // no read meets a row written this step (the common case)
#pragma unroll
        for (int k = 0; k < KE; ++k) {
            const float rw = job.mass_aware ? rv[k] * lane_f(st.emr, RB + k) : rv[k];
            sr += rv[k];
            srm += rw;
#pragma unroll
            for (int j = 0; j < kCpl; ++j)
                acc[j] = fmaf(rw, st.rrow[k][j], acc[j]);
        }
    } else {
        // forwarded rows: the written rows (recomputed from the same
        // operands) go through LDS, each lane re-reading only what it wrote
#pragma unroll
        for (int k = 0; k < KE; ++k) {
            if (FULLK || k < Kw) {
                const float g = lane_f(gain, k);
#pragma unroll
                for (int j = 0; j < kCpl; ++j)
                    s_row[k][lane * kCpl + j] = fmaf(g, xv[j] - st.wrow[k][j], st.wrow[k][j]);
            }
        }
        __builtin_amdgcn_wave_barrier();
        float wm[KE];
#pragma unroll
        for (int k = 0; k < KE; ++k)
            wm[k] = lane_f(m2, k);
#pragma unroll
        for (int k = 0; k < KE; ++k) {
            const int f = st.fwd[k];
            const int fc = f < 0 ? 0 : f;
            float m = lane_f(st.emr, RB + k);
#pragma unroll
            for (int j2 = 0; j2 < KE; ++j2)
                m = f == j2 ? wm[j2] : m;
            const float rw = job.mass_aware ? rv[k] * m : rv[k];
            sr += rv[k];
            srm += rw;
#pragma unroll
            for (int j = 0; j < kCpl; ++j) {
                const float lv = s_row[fc][lane * kCpl + j];
                acc[j] = fmaf(rw, f >= 0 ? lv : st.rrow[k][j], acc[j]);
            }
        }
    }
    const float scale = job.mass_aware ? sr / (srm + job.eps) : 1.f;
    float yv[kCpl];
#pragma unroll
    for (int j = 0; j < kCpl; ++j)
        yv[j] = acc[j] * scale;
    store_y<T, kCpl, FULLC>(yrow, yv, lane, C);
}

// One decode step, one wave per (b, h).
template<typename T, int GW, int KE, int kCpl, bool FULLC, bool FULLK>
__global__ __launch_bounds__(64) void autoregressive_fast_kernel(const DecodeJob job) {
    __shared__ int s_ws[KE], s_rs[KE];
    __shared__ float s_wv[KE];
    __shared__ float s_row[KE][kWave * kCpl];

    // grid (B, H): the (b, h) pair without a division
    const int b = blockIdx.x, h = blockIdx.y;
    const int lane = threadIdx.x;
    const int H = job.H, A = job.A, C = job.C, U = job.U, P = job.P;
    const int bh = b * H + h;
    T *yrow = static_cast<T *>(job.y) + static_cast<int64_t>(bh) * C;

    // every input of the step in one batch of loads
    const T *wp = static_cast<const T *>(job.w_addr) + static_cast<int64_t>(bh) * U * P;
    const T *rp = static_cast<const T *>(job.r_addr) + static_cast<int64_t>(bh) * U * P;
    GroupLogits<T> lw, lr;
    if constexpr (GW == 32) {
        lw.load((lane >> 5) ? rp : wp, U, P, lane & 31);
    } else {
        lw.load(wp, U, P, lane);
        lr.load(rp, U, P, lane);
    }
    int coff[kCpl];
    lane_channels<kCpl, FULLC>(lane, C, coff);
    XRaw<T, kCpl, FULLC> xr;
    xr.load(static_cast<const T *>(job.x) + static_cast<int64_t>(bh) * C, coff, lane);
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
    const int rowb = C * 4;

    StepState<KE, kCpl> st;
    decode_events<T, GW, KE, kCpl>(job, lw, lr, shift, lane, s_ws, s_rs, s_wv, st);
    issue_rows<GW, KE, kCpl, FULLC, FULLK>(srs, mrs, coff, rowb, job.Kw, st);
    forward_map<KE, kCpl>(job, lane, s_ws, s_rs, s_wv, st);
    apply_step<T, GW, KE, kCpl, FULLC, FULLK>(job, st, xr, gamma, true, srs, mrs, coff, rowb, lane, s_row, yrow);
}

// The mask byte read by steps without a mask. It lives in global memory
// (not constant memory) so that the mask pointer stays a global pointer: a
// pointer that may be either would be read with flat loads, which count on
// both memory counters and make every wait on them a full wait.
__device__ uint8_t kValidStep = 1;

// S consecutive decode steps in one launch (the multi-step form of
// ramnet_topk_autoregressive_steps_). Inputs and y carry a leading step
// dimension; position_ids and mask are (S, B).
//
// One workgroup of two waves per (b, h). A single wave would issue every
// instruction of a step in one dependent chain at one wave per SIMD, so the
// work is split: wave 0 (the decoder) decodes the addresses of step s + 2
// while wave 1 (the updater) applies step s and requests step s + 1's rows.
// They hand the events over through a two-slot LDS ring and meet at one
// workgroup barrier per step (each role's code passes the same S + 2
// barriers, in its own loop). The decoder fills ring slot s % 2 with step
// s + 2's events during iteration s; the updater took that slot's previous
// contents (step s's events) before the barrier ending iteration s - 1.
//
// The updater's memory requests are issued in program order: step s + 1's
// rows after step s's stores, and every row channel is accessed by the lane
// that owns it, so step s + 1 reads step s's stores in program order; the
// masses are read back by other lanes of the same wave, whose memory
// instructions are processed in issue order. Values are prefetched as raw
// bits and converted where they are used, and every memory instruction of a
// loop iteration executes on every path (steps past the last repeat it,
// clamped), so the compiler's memory-counter waits cover only what each
// stage needs.
template<int KE>
struct StepRing {
    int2 ev[2][kWave];  // per lane: (event slot, weight bits)
    int fwd[2][KE];     // forwarding map of the step
    int any[2];
};

template<typename T, int KE, int kCpl, bool FULLC, bool FULLK>
__global__ __launch_bounds__(2 * kWave) void autoregressive_steps_kernel(const DecodeJob job, const int S) {
    constexpr int GW = 32;
    __shared__ int s_ws[KE], s_rs[KE];
    __shared__ float s_wv[KE];
    __shared__ float s_row[KE][kWave * kCpl];
    __shared__ StepRing<KE> ring;

    const int b = blockIdx.x, h = blockIdx.y;
    const int lane = threadIdx.x & (kWave - 1);
    // the role is uniform per wave; readfirstlane tells the compiler so, and
    // the role branches become scalar branches
    const bool decoder = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x)) < kWave;
    const int B = job.B, H = job.H, A = job.A, C = job.C, U = job.U, P = job.P;
    const int bh = b * H + h;
    const int64_t BH = static_cast<int64_t>(B) * H;
    const int64_t step_addr = BH * U * P, step_x = BH * C;
    const int last = S - 1;

    // decoder state: step logits and position (prefetched a step ahead)
    const T *ap = static_cast<const T *>((lane >> 5) ? job.r_addr : job.w_addr) + static_cast<int64_t>(bh) * U * P;
    // The position is read per lane (through an index the compiler cannot
    // see is uniform), so it stays a vector value: a scalar load would share
    // its completion counter with the LDS accesses, and a uniform vector load
    // would be moved to a scalar register right after it issues.
    const int32_t *pp = job.position_ids + b + static_cast<int>(opaque(0u));
    const bool cape = h < job.embed_num;
    GroupLogits<T> lg;
    int pos = 0;
    // Decode step `t` (clamped) into ring slot `slot`, then prefetch the
    // logits and position of step `next` (clamped).
    auto produce = [&](int t, int slot, int next) {
        StepState<KE, kCpl> ev;
        decode_events<T, GW, KE, kCpl>(job, lg, lg, cape ? pos_mod(pos, A) : 0, lane, s_ws, s_rs, s_wv, ev);
        const int64_t n = next < last ? next : last;
        lg.load(ap + n * step_addr, U, P, lane & 31);
        pos = pp[n * B];
        forward_map<KE, kCpl>(job, lane, s_ws, s_rs, s_wv, ev);
        ring.ev[slot][lane] = make_int2(ev.ow, __float_as_int(ev.vw));
        if (lane == 0) {
#pragma unroll
            for (int k = 0; k < KE; ++k)
                ring.fwd[slot][k] = ev.fwd[k];
            ring.any[slot] = ev.any_fwd ? 1 : 0;
        }
        (void)t;
    };

    // updater state
    const T *xp = static_cast<const T *>(job.x) + static_cast<int64_t>(bh) * C;
    const T *gp = static_cast<const T *>(job.gamma) + bh;
    T *yp = static_cast<T *>(job.y) + static_cast<int64_t>(bh) * C;
    // without a mask every step reads a constant 1 (stride 0), so the mask
    // load is unconditional like every other request of the loop
    const uint8_t *mp = job.mask ? job.mask + b + static_cast<int>(opaque(0u)) : &kValidStep;
    const int64_t mstride = job.mask ? B : 0;
    int coff[kCpl];
    lane_channels<kCpl, FULLC>(lane, C, coff);
    const auto srs = __builtin_amdgcn_make_buffer_rsrc(job.slot + static_cast<int64_t>(bh) * A * C, 0, A * C * 4,
                                                       kBufWord3);
    const auto mrs = __builtin_amdgcn_make_buffer_rsrc(job.mass + static_cast<int64_t>(bh) * A, 0, A * 4, kBufWord3);
    const int rowb = C * 4;
    StepState<KE, kCpl> st;
    XRaw<T, kCpl, FULLC> xr;
    uint32_t gr = 0;
    int valid = 1;
    // Take step `t`'s events from ring slot `slot`, prefetch its apply
    // inputs, request its rows (t clamped).
    auto take = [&](int t, int slot) {
        const int2 e = ring.ev[slot][lane];
        st.ow = e.x;
        st.vw = __int_as_float(e.y);
        st.orr = st.ow;
        st.vr = st.vw;
#pragma unroll
        for (int k = 0; k < KE; ++k)
            st.fwd[k] = ring.fwd[slot][k];
        st.any_fwd = ring.any[slot] != 0;
        const int64_t c = t < last ? t : last;
        xr.load(xp + c * step_x, coff, lane);
        gr = load_bits(gp + c * BH);
        valid = mp[c * mstride];
        // the fence keeps the row requests after the prefetch and after the
        // previous step's stores
        __builtin_amdgcn_sched_barrier(0);
        issue_rows<GW, KE, kCpl, FULLC, FULLK>(srs, mrs, coff, rowb, job.Kw, st);
    };

    // Each role runs its own loop (so that the compiler's memory-counter
    // analysis sees one wave's requests per loop); both pass S + 2 barriers.
    if (decoder) {
        lg.load(ap, U, P, lane & 31);
        pos = pp[0];
        produce(0, 0, 1);
        __syncthreads();
        produce(1, 1, 2);
        __syncthreads();
        for (int s = 0; s < S; ++s) {
            produce(s + 2, s & 1, s + 3);
            __syncthreads();
        }
    } else {
        __syncthreads();
        take(0, 0);
        __syncthreads();
        for (int s = 0; s < S; ++s) {
            apply_step<T, GW, KE, kCpl, FULLC, FULLK>(job, st, xr, bits_f32<T>(gr), valid != 0, srs, mrs, coff,
                                                      rowb, lane, s_row, yp + s * step_x);
            take(s + 1, (s + 1) & 1);
            __syncthreads();
        }
    }
}

// General shapes: exact LDS search (STAIR false, NA = pow2 >= A) or the
// staircase search for wider slot spaces (STAIR true, NA = candidate buffer),
// then sequential row updates.
template<typename T, bool STAIR>
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
    const int KM = Kw > Kr ? Kw : Kr;
    float *lg = smem;
    float *ex = lg + U * P;
    int *di = reinterpret_cast<int *>(ex + U * NPD);  // staircase only
    float *sv = STAIR ? reinterpret_cast<float *>(di + U * NPD) : ex + U * NPD;
    int *si = reinterpret_cast<int *>(sv + NA);
    float *pv = reinterpret_cast<float *>(si + NA);    // staircase only: KM, KM, KM + 1
    int *pi = reinterpret_cast<int *>(pv + (STAIR ? KM : 0));
    int *off = pi + (STAIR ? KM : 0);
    int *ev_slot = off + (STAIR ? KM + 1 : 0);  // Kw + Kr
    float *ev_val = reinterpret_cast<float *>(ev_slot + Kw + Kr);  // Kw + Kr
    const int shift = h < job.embed_num ? pos_mod(job.position_ids[b], A) : 0;

    for (int which = 0; which < 2; ++which) {
        const T *ptr = static_cast<const T *>(which ? job.r_addr : job.w_addr) + static_cast<int64_t>(bh) * U * P;
        const int K = which ? Kr : Kw;
        const float re = which ? job.r_re_norm : job.w_re_norm;
        bool inactive;
        if constexpr (STAIR)
            inactive = block_search_stair(ptr, 1, U, P, K, NPD, NA, lg, ex, di, sv, si, pv, pi, off, &s_flag);
        else
            inactive = block_search_exact(ptr, 1, U, P, A, NA, NPD, lg, ex, sv, si, &s_flag);
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

// Whether x, y and the slot state allow the kernels' vector accesses of cpl
// channels (the FULLC forms; each row then starts on a multiple of the
// vector width, since C == 64 * cpl).
template<typename T>
bool vector_aligned(const DecodeJob &job, int cpl) {
    const uintptr_t xa = reinterpret_cast<uintptr_t>(job.x), ya = reinterpret_cast<uintptr_t>(job.y);
    const uintptr_t sa = reinterpret_cast<uintptr_t>(job.slot);
    const uintptr_t xw = static_cast<uintptr_t>(cpl) * sizeof(T), sw = static_cast<uintptr_t>(cpl) * 4;
    return xa % xw == 0 && ya % xw == 0 && sa % sw == 0;
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
#define RAMNET_AR_LAUNCH_K(GW, KE, CPL, FK)                                                                    \
    do {                                                                                                        \
        if (job.C == (CPL) * kWave && vector_aligned<T>(job, CPL))                                              \
            hipLaunchKernelGGL((autoregressive_fast_kernel<T, GW, KE, CPL, true, FK>), g, blk, 0, stream, job); \
        else                                                                                                    \
            hipLaunchKernelGGL((autoregressive_fast_kernel<T, GW, KE, CPL, false, FK>), g, blk, 0, stream, job);\
    } while (0)
#define RAMNET_AR_LAUNCH(GW, KE, CPL)                                                                          \
    do {                                                                                                        \
        if (job.Kw == (KE) && job.Kr == (KE))                                                                   \
            RAMNET_AR_LAUNCH_K(GW, KE, CPL, true);                                                              \
        else                                                                                                    \
            RAMNET_AR_LAUNCH_K(GW, KE, CPL, false);                                                             \
    } while (0)
        if (half) {
            if (few) { if (narrow) RAMNET_AR_LAUNCH(32, 8, 2); else RAMNET_AR_LAUNCH(32, 8, 4); }
            else { if (narrow) RAMNET_AR_LAUNCH(32, 16, 2); else RAMNET_AR_LAUNCH(32, 16, 4); }
        } else {
            if (few) { if (narrow) RAMNET_AR_LAUNCH(64, 8, 2); else RAMNET_AR_LAUNCH(64, 8, 4); }
            else { if (narrow) RAMNET_AR_LAUNCH(64, 16, 2); else RAMNET_AR_LAUNCH(64, 16, 4); }
        }
#undef RAMNET_AR_LAUNCH_K
#undef RAMNET_AR_LAUNCH
        return hipGetLastError();
    }
    const int NA = pow2_ceil(job.A), NPD = pow2_ceil(job.P);
    const size_t lds = static_cast<size_t>(job.U) * job.P * 4 + static_cast<size_t>(job.U) * NPD * 4 +
                       static_cast<size_t>(NA) * 8 + static_cast<size_t>(job.Kw + job.Kr) * 8;
    if (lds <= 96 * 1024) {
        hipLaunchKernelGGL((autoregressive_general_kernel<T, false>), grid, dim3(kWave), lds, stream, job, NA, NPD);
        return hipGetLastError();
    }
    // wider slot spaces: the staircase search, any A
    const int km = std::max(job.Kw, job.Kr);
    if (km > 128 || NPD > 1024) {
        *why = "decode step: slot spaces beyond the exact LDS search (A > 8192) take top_k <= 128 and P <= 1024";
        return hipErrorInvalidValue;
    }
    const int NC = stair_buffer(job.P, km, NPD);
    const size_t lds_s = static_cast<size_t>(job.U) * job.P * 4 + static_cast<size_t>(job.U) * NPD * 8 +
                         static_cast<size_t>(NC) * 8 + static_cast<size_t>(km) * 8 + static_cast<size_t>(km + 1) * 4 +
                         static_cast<size_t>(job.Kw + job.Kr) * 8;
    if (lds_s > 96 * 1024) {
        *why = "decode step: staircase search scratch exceeds LDS (U * P too large)";
        return hipErrorInvalidValue;
    }
    hipLaunchKernelGGL((autoregressive_general_kernel<T, true>), grid, dim3(kWave), lds_s, stream, job, NC, NPD);
    return hipGetLastError();
}

// S steps: one launch of the multi-step kernel when the shape takes the
// half-wave fast path, else S launches of the single-step kernels on the
// step's slices of the inputs.
template<typename T>
hipError_t launch_typed_steps(const DecodeJob &job, int S, hipStream_t stream, const char **why) {
    const int kmax = std::max(job.Kw, job.Kr);
    const int stair = staircase_count(kmax);
    const bool persistent = job.P <= 32 && kmax <= kEv && stair <= 32 && job.C <= kWave * kMaxCpl &&
                            static_cast<int64_t>(job.A) * job.C * 4 <= INT32_MAX && job.H <= 65535;
    if (persistent) {
        const dim3 g(static_cast<unsigned>(job.B), static_cast<unsigned>(job.H)), blk(2 * kWave);
        const bool narrow = job.C <= 2 * kWave;
        const bool few = kmax <= 8;
#define RAMNET_AR_STEPS_K(KE, CPL, FK)                                                                          \
    do {                                                                                                        \
        if (job.C == (CPL) * kWave && vector_aligned<T>(job, CPL))                                              \
            hipLaunchKernelGGL((autoregressive_steps_kernel<T, KE, CPL, true, FK>), g, blk, 0, stream, job, S);  \
        else                                                                                                    \
            hipLaunchKernelGGL((autoregressive_steps_kernel<T, KE, CPL, false, FK>), g, blk, 0, stream, job, S); \
    } while (0)
#define RAMNET_AR_STEPS(KE, CPL)                                                                                \
    do {                                                                                                        \
        if (job.Kw == (KE) && job.Kr == (KE))                                                                   \
            RAMNET_AR_STEPS_K(KE, CPL, true);                                                                   \
        else                                                                                                    \
            RAMNET_AR_STEPS_K(KE, CPL, false);                                                                  \
    } while (0)
        if (few) { if (narrow) RAMNET_AR_STEPS(8, 2); else RAMNET_AR_STEPS(8, 4); }
        else { if (narrow) RAMNET_AR_STEPS(16, 2); else RAMNET_AR_STEPS(16, 4); }
#undef RAMNET_AR_STEPS_K
#undef RAMNET_AR_STEPS
        return hipGetLastError();
    }
    const int64_t BH = static_cast<int64_t>(job.B) * job.H;
    for (int s = 0; s < S; ++s) {
        DecodeJob one = job;
        one.w_addr = static_cast<const T *>(job.w_addr) + s * BH * job.U * job.P;
        one.r_addr = static_cast<const T *>(job.r_addr) + s * BH * job.U * job.P;
        one.x = static_cast<const T *>(job.x) + s * BH * job.C;
        one.gamma = static_cast<const T *>(job.gamma) + s * BH;
        one.y = static_cast<T *>(job.y) + s * BH * job.C;
        one.position_ids = job.position_ids + static_cast<int64_t>(s) * job.B;
        one.mask = job.mask ? job.mask + static_cast<int64_t>(s) * job.B : nullptr;
        const hipError_t err = launch_typed<T>(one, stream, why);
        if (err != hipSuccess)
            return err;
    }
    return hipSuccess;
}

}  // namespace

hipError_t launch_autoregressive_steps(const DecodeJob &job, int S, hipStream_t stream, const char **why) {
    if (job.B * job.H == 0 || S == 0)
        return hipSuccess;
    switch (job.dtype) {
        case kF32: return launch_typed_steps<float>(job, S, stream, why);
        case kF16: return launch_typed_steps<_Float16>(job, S, stream, why);
        case kBF16: return launch_typed_steps<bf16_t>(job, S, stream, why);
        default: *why = "decode steps: unsupported dtype"; return hipErrorInvalidValue;
    }
}

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
