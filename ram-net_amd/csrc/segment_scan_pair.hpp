// Paired form of the precomputed-gain segment scan: two tokens per wave step.
//
// The one-token form (segment_scan.hpp) spreads a token's events over all 64
// lanes of a wave, so a slice of CS channels keeps one token chain per wave,
// and the LDS that a slice of A x CS fp32 slots takes caps the waves a CU
// holds: at 4 per CU (config 2: A = 1024, CS = 32) each SIMD runs a single
// chain and idles through every LDS round trip of it; at 2 per CU (config
// 4: A = 4096, CS = 8) half the SIMDs get none.
//
// Here lanes 0..31 carry the even token of a pair and lanes 32..63 the odd
// one; within each half, EPP events x LPE = 32 / EPP channel groups,
// event-fastest (the event sums are DPP exchanges within a row). One LDS
// instruction serves both tokens, and a wave owns half the channels it owns
// in the one-token form: the same slice is split over twice the waves, so
// the LDS that held 4 chains per CU now holds 8, and each instruction still
// carries 64 lanes of work.
//
// A pair (a, b) = (2s, 2s + 1) runs as: the rows both tokens write, loaded;
// both tokens' writes in one instruction; both tokens' reads in one
// instruction. That equals the in-order execution (writes of a, reads of a,
// writes of b, reads of b) unless b writes a slot that a also writes (bit 0
// of b's flags, from the decoder's overlap test) or a slot that a reads
// (bit 3, from the mass pre-pass). Such a pair runs in order, one half at a
// time, with the other half's lanes pointed at the dummy rows. Pairs go in
// groups of two (four tokens, whose write rows are all loaded before the
// first pair's writes); the second pair's rows are loaded again when one of
// its tokens may write a slot that the first pair wrote (bits 0-1 of its
// even token, 1-2 of its odd token: overlap with the token d = 1, 2, 3
// back, bit d - 1).
//
// Records: each lane loads the gain records of its own (token, event) from
// global memory straight into registers, one chunk ahead (no LDS stage);
// x goes through a small private LDS stage per wave, laid out by channel and
// token parity so that each lane reads its half's tokens contiguously.
#pragma once

#include "segment_scan.hpp"

namespace ramnet {

// Tokens per chunk of the paired scan: 2 * EPP, so that a chunk's pairs
// fill one reduce-scatter over the event lanes; at most 32 (the record
// padding).
constexpr int scan_pair_chunk_len(int epp) { return 2 * epp < 32 ? 2 * epp : 32; }

// Staged x of the workgroup: per wave a row per channel and token parity.
__host__ __device__ constexpr size_t scan_pair_stage_bytes(int vec, int epp, int nw, int elem) {
    return static_cast<size_t>(nw) * (kWave / 2 / epp) * vec * 2 * ((scan_pair_chunk_len(epp) / 2) * elem + 16);
}
// LDS of one workgroup: the slot slice with its two dummy rows, then the
// staged x.
inline size_t scan_pair_lds_bytes(int A, int vec, int epp, int nw, int elem) {
    const int cs = nw * (kWave / 2 / epp) * vec;
    return scan_stage_offset(A, scan_row_stride(vec, cs), true) + scan_pair_stage_bytes(vec, epp, nw, elem);
}

template<typename Scalar, int VEC, int EPP, int NW, bool FAST>
__global__ __launch_bounds__(kWave * NW) void segment_scan_pair_kernel(const SegmentJob job, const ScanGeom geo) {
    constexpr int HW = kWave / 2;  // lanes per token of a pair
    static_assert(EPP >= 2 && EPP <= HW && (EPP & (EPP - 1)) == 0, "paired scan: EPP a power of two in [2, 32]");
    constexpr int LPE = HW / EPP;      // lanes per event
    constexpr int CSW = LPE * VEC;     // channels per wave
    constexpr int CS = NW * CSW;       // channels per slice
    constexpr int CH = scan_pair_chunk_len(EPP);  // tokens per chunk
    constexpr int NPS = CH / 2;                  // pairs per chunk
    constexpr int ES = static_cast<int>(sizeof(Scalar));
    constexpr int XRB = NPS * ES + 16;  // staged x row: one channel, one parity, + 16 bytes against bank conflicts
    constexpr int XIW = (CSW * CH + kWave - 1) / kWave;  // staged x elements per lane
    constexpr int LOGE = __builtin_ctz(EPP);
    constexpr int LOGR = __builtin_ctz(NPS);
    static_assert(LOGR >= 1 && LOGR <= LOGE, "a chunk holds between 2 and EPP pairs");
    constexpr int SH = LOGE - LOGR;  // low event bits summed after the reduce-scatter
    static_assert(NPS % 2 == 0, "chunks hold whole groups of two pairs");
    using Bits = std::conditional_t<ES == 4, uint32_t, uint16_t>;

    extern __shared__ __align__(16) float lds[];
    // slices of one (b, h) on one XCD (workgroups are dealt round-robin to the 8 XCDs)
    const int per_xcd = (geo.n_units + 7) / 8;
    const int unit = static_cast<int>(blockIdx.x % 8) * per_xcd + static_cast<int>(blockIdx.x / 8);
    if (unit >= geo.n_units)
        return;
    const int tid = static_cast<int>(threadIdx.x);
    const int wave = tid / kWave;
    const int lane = tid % kWave;
    const int bh = unit / geo.n_slices;
    const int c0 = (unit - bh * geo.n_slices) * CS;
    const int T = job.T, A = job.A, C = job.C, Tp = geo.t_pad;
    const int EK = job.Kw > job.Kr ? job.Kw : job.Kr;
    constexpr int RS = scan_row_stride(VEC, CS);

    float *st = lds + 2 * RS;  // slot 0 of the slice; rows -2 (dummy write) and -1 (zero read) in front
    char *stage0 = reinterpret_cast<char *>(lds) + scan_stage_offset(A, RS, true);

    // ---- state slice -> LDS
    {
        const float *src = job.init_slot + static_cast<int64_t>(bh) * A * C;
        for (int i = tid; i < A * CS; i += kWave * NW) {
            const int a = i / CS, c = i - a * CS;
            const bool ok = c0 + c < C;
            const float v = src[static_cast<int64_t>(a) * C + (ok ? c0 + c : 0)];
            st[a * RS + c] = ok ? v : 0.f;
        }
        for (int i = tid; i < 2 * RS; i += kWave * NW)
            lds[i] = 0.f;
    }

    // ---- lanes: tp = token of the pair, ev = event, cg = channel group
    const int tp = lane / HW;
    const int hl = lane % HW;
    const int ev = hl % EPP;
    const int cg = hl / EPP;
    const int cl = wave * CSW + cg * VEC;  // first channel of this lane within the slice
    uint32_t hi[6];
    hi[0] = bit_mask<1>(lane);
    hi[1] = bit_mask<2>(lane);
    hi[2] = bit_mask<4>(lane);
    hi[3] = bit_mask<8>(lane);
    hi[4] = bit_mask<16>(lane);
    hi[5] = bit_mask<32>(lane);
    // Row addresses: slot * amul + base. Lanes past the head's events load
    // the last event's records and act on the dummy rows.
    const bool dead = ev >= EK;
    const int amul = dead ? 0 : RS * 4;
    const int lrow = static_cast<int>(lds_addr(st) + static_cast<uint32_t>(cl) * 4);
    const int awb = dead ? static_cast<int>(lds_addr(lds) + static_cast<uint32_t>(cl) * 4) : lrow;       // row -2
    const int arb = dead ? static_cast<int>(lds_addr(lds + RS) + static_cast<uint32_t>(cl) * 4) : lrow;  // row -1
    const int evc = ev < EK ? ev : EK - 1;

    const GainRec *gp = job.gain + static_cast<int64_t>(bh) * EK * Tp;
    const WriteRec *gw = job.wrec + static_cast<int64_t>(bh) * job.Kw * Tp;
    const int *gf = job.flags + static_cast<int64_t>(bh) * Tp;
    const Scalar *gx = static_cast<const Scalar *>(job.x) + static_cast<int64_t>(bh) * T * C;
    Scalar *gy = static_cast<Scalar *>(job.y) + static_cast<int64_t>(bh) * T * C;
    // this wave's x stage: row (channel c of the wave, parity q) at (2 c + q) * XRB
    char *px = stage0 + wave * (CSW * 2 * XRB);

    struct Fetch {
        int4 rec[NPS];  // {write slot, gain, read slot, read weight} of token 2 s + tp, event ev
        Bits x[XIW];
        int ov;  // overlap bits of token t0 + lane (decoder, write event 0), lanes < CH
        int rw;  // 1 if token t0 + lane writes a slot that token t0 + lane - 1 reads (mass pre-pass)
    };
    // the head's gain records through a buffer resource: a lane offset fixed
    // for the whole sequence plus a wave-uniform offset per pair (no 64-bit
    // address arithmetic per load; the host keeps a head's records below
    // 2^31 bytes)
    const auto grs = __builtin_amdgcn_make_buffer_rsrc(const_cast<GainRec *>(gp), 0, EK * Tp * 16, kBufWord3);
    const int gvo = (tp * EK + evc) * 16;
    auto fetch = [&](int t0, Fetch &f) {
#pragma unroll
        for (int s = 0; s < NPS; ++s) {
            const auto q = __builtin_amdgcn_raw_buffer_load_b128(grs, gvo, (t0 + 2 * s) * EK * 16, 0);
            f.rec[s] = make_int4(static_cast<int>(q[0]), static_cast<int>(q[1]), static_cast<int>(q[2]),
                                 static_cast<int>(q[3]));
        }
#pragma unroll
        for (int k = 0; k < XIW; ++k) {
            const int it = min(lane + k * kWave, CSW * CH - 1);
            const int j = it / CSW, c = wave * CSW + it % CSW;
            const int t = t0 + j < T ? t0 + j : T - 1;
            const int ch = c0 + c < C ? c0 + c : C - 1;
            f.x[k] = *reinterpret_cast<const Bits *>(gx + static_cast<int64_t>(t) * C + ch);
        }
        // (loads without a branch: a conditional one would be waited for at once)
        const int tf = t0 + min(lane, CH - 1);
        f.ov = *(job.Kw > 0 ? reinterpret_cast<const int *>(&gw[tf].overlap) : &kNoFlag);
        f.rw = gf[tf];
    };
    auto x_deposit = [&](const Fetch &f) {
#pragma unroll
        for (int k = 0; k < XIW; ++k) {
            const int it = min(lane + k * kWave, CSW * CH - 1);
            const int j = it / CSW, c = it % CSW;
            *reinterpret_cast<Bits *>(px + (2 * c + (j & 1)) * XRB + (j >> 1) * ES) = f.x[k];
        }
    };

    // One chunk: NPS pairs from registers f (consumed: the slots become row
    // addresses). TAIL guards tokens past T.
    auto chunk = [&](int t0, auto tail_tag, Fetch &f) {
        constexpr bool TAIL = decltype(tail_tag)::value;
        // hazard masks, bit j = token t0 + j (see the file comment)
        uint64_t m_ser, m_ww, m_rel;
        {
            const int fv = lane < CH && t0 + lane < T ? (f.ov & 7) | (f.rw << 3) : 0;
            const bool odd = (lane & 1) != 0;
            m_ser = __ballot(odd && (fv & 9) != 0);
            m_ww = __ballot(odd && (fv & 1) != 0);
            m_rel = __ballot((lane & 2) != 0 && (fv & (odd ? 6 : 3)) != 0);
        }
        // this lane's x: its channel rows of its parity
        constexpr int XW = (NPS * ES + 15) / 16;
        uint4 xr[VEC][XW];
#pragma unroll
        for (int v = 0; v < VEC; ++v)
#pragma unroll
            for (int q = 0; q < XW; ++q)
                xr[v][q] = *reinterpret_cast<const uint4 *>(px + (2 * (cg * VEC + v) + tp) * XRB + q * 16);
        auto x_at = [&](int v, int s) -> float {
            const uint4 q4 = xr[v][(s * ES) / 16];
            const int wi = ((s * ES) % 16) / 4;
            const uint32_t wd = wi == 0 ? q4.x : wi == 1 ? q4.y : wi == 2 ? q4.z : q4.w;
            if constexpr (ES == 4)
                return __uint_as_float(wd);
            else
                return half_bits_to_f<Scalar>((wd >> (16 * (s % 2))) & 0xffffu);
        };
        auto &rec = f.rec;
        // row addresses of pair s; the first group's before the pair loop,
        // each later group's during the group before it, where they fill the
        // wait for that group's rows
        auto addresses = [&](int s) {
            int wa = rec[s].x, ra = rec[s].z;
            if constexpr (TAIL) {
                const bool live = t0 + 2 * s + tp < T;
                wa = live ? wa : -2;
                ra = live ? ra : -1;
                rec[s].w = live ? rec[s].w : 0;
            }
            rec[s].x = mad24(wa, amul, awb);
            rec[s].z = mad24(ra, amul, arb);
        };
        auto row = [&](int a) { return lds_at(static_cast<uint32_t>(a)); };
        auto write = [&](int s, const FVec<VEC> &sv, int addr) {
            const float g = __int_as_float(rec[s].y);
            FVec<VEC> o;
#pragma unroll
            for (int v = 0; v < VEC; ++v)
                o.v[v] = fmaf(g, x_at(v, s) - sv.v[v], sv.v[v]);
            lds_store<VEC>(row(addr), o);
        };
        // one pair: writes then reads, both halves at once, or in order
        // (SER) with the idle half on the dummy rows; WW: the odd token's
        // rows are loaded again after the even token's writes
        auto pair = [&](int s, const FVec<VEC> &sv, FVec<VEC> &rv) {
            const bool ser = ((m_ser >> (2 * s + 1)) & 1u) != 0;
            if (__builtin_expect(!ser, 1)) {
                write(s, sv, rec[s].x);
                rv = lds_load<VEC>(row(rec[s].z));
            } else {
                // the even token with the odd half's lanes masked off, then
                // the odd token (its rows loaded again if the even token
                // wrote one of them)
                FVec<VEC> sb = sv;
                if (tp == 0) {
                    write(s, sv, rec[s].x);
                    rv = lds_load<VEC>(row(rec[s].z));
                }
                // The odd half's lanes stored nothing above: without this
                // the compiler would take their row load for unchanged since
                // the group's first loads and reuse those values, though
                // other lanes of the wave have just written the rows.
                __builtin_amdgcn_wave_barrier();
                if (((m_ww >> (2 * s + 1)) & 1u) != 0) {
                    if (tp != 0)
                        sb = lds_load<VEC>(row(rec[s].x));
                    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
                }
                if (tp != 0) {
                    write(s, sb, rec[s].x);
                    rv = lds_load<VEC>(row(rec[s].z));
                }
            }
        };
        // read sums: each lane's partial per pair, then one reduce-scatter
        // over the event lanes per chunk
        float part[VEC][NPS];
        auto reduce = [&](int s, const FVec<VEC> &rv) {
            const float wgt = __int_as_float(rec[s].w);
            // (opaque: the first exchange's DPP add would otherwise be
            // contracted with the product into a DPP move and an fma)
#pragma unroll
            for (int v = 0; v < VEC; ++v)
                part[v][s] = __uint_as_float(opaque(__float_as_uint(wgt * rv.v[v])));
        };
        FVec<VEC> rp[2];
        addresses(0);
        addresses(1);
#pragma unroll
        for (int s0 = 0; s0 < NPS; s0 += 2) {
            FVec<VEC> sv0, sv1;
            sv0 = lds_load<VEC>(row(rec[s0].x));
            sv1 = lds_load<VEC>(row(rec[s0 + 1].x));
            if (s0 > 0) {
                reduce(s0 - 2, rp[0]);
                reduce(s0 - 1, rp[1]);
            }
            if (s0 + 2 < NPS) {
                addresses(s0 + 2);
                addresses(s0 + 3);
            }
            pair(s0, sv0, rp[0]);
            if (__builtin_expect(((m_rel >> (2 * s0 + 2)) & 3u) != 0, 0)) {
                __builtin_amdgcn_wave_barrier();  // rows written by other lanes
                sv1 = lds_load<VEC>(row(rec[s0 + 1].x));
                __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
            }
            pair(s0 + 1, sv1, rp[1]);
        }
        reduce(NPS - 2, rp[0]);
        reduce(NPS - 1, rp[1]);
        FVec<VEC> y;
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
            event_scatter<LOGR - 1, SH, NPS>(part[v], hi);
            y.v[v] = event_sum<(1 << SH)>(part[v][0]);
        }
        // lane (tp, ev, cg) holds pair ev >> SH: token t0 + 2 (ev >> SH) + tp
        const int t = t0 + 2 * (ev >> SH) + tp;
        if ((ev & ((1 << SH) - 1)) == 0 && (!TAIL || t < T)) {
            Scalar *yp = gy + static_cast<int64_t>(t) * C + c0 + cl;
            if constexpr (FAST) {
                store_act_vec<Scalar, VEC>(yp, y);
            } else {
#pragma unroll
                for (int v = 0; v < VEC; ++v)
                    if (c0 + cl + v < C)
                        store_out(yp + v, y.v[v]);
            }
        }
    };

    // ---- pipeline: chunk ci runs from registers while chunk ci + 1 loads;
    // two chunks per iteration with swapped buffers (no copy of registers
    // with loads pending). Chunks wholly inside T run unguarded.
    using Full = std::false_type;
    using Tail = std::true_type;
    const int nc = (T + CH - 1) / CH;
    const int n_full = T / CH;
    auto clampc = [&](int c) { return (c < nc ? c : nc - 1) * CH; };
    auto run = [&](int ci, Fetch &f) {
        x_deposit(f);
        if (ci < n_full)
            chunk(ci * CH, Full{}, f);
        else
            chunk(ci * CH, Tail{}, f);
    };
    __syncthreads();  // state slice loaded
    if (nc > 0) {
        Fetch fa, fb;
        fetch(0, fa);
        for (int ci = 0; ci < nc; ci += 2) {
            fetch(clampc(ci + 1), fb);
            __builtin_amdgcn_sched_barrier(0);
            run(ci, fa);
            __builtin_amdgcn_sched_barrier(0);
            if (ci + 1 >= nc)
                break;
            fetch(clampc(ci + 2), fa);
            __builtin_amdgcn_sched_barrier(0);
            run(ci + 1, fb);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    __syncthreads();

    // ---- LDS -> post state
    {
        float *dst = job.slot_out + static_cast<int64_t>(bh) * A * C;
        for (int i = tid; i < A * CS; i += kWave * NW) {
            const int a = i / CS, c = i - a * CS;
            if (c0 + c < C)
                dst[static_cast<int64_t>(a) * C + c0 + c] = st[a * RS + c];
        }
    }
}

template<typename Scalar, int VEC, int EPP, int NW, bool FAST>
hipError_t launch_scan_pair(const SegmentJob &job, const ScanGeom &geo, hipStream_t stream) {
    const unsigned blocks = static_cast<unsigned>(((geo.n_units + 7) / 8) * 8);
    hipLaunchKernelGGL((segment_scan_pair_kernel<Scalar, VEC, EPP, NW, FAST>), dim3(blocks), dim3(kWave * NW),
                       scan_pair_lds_bytes(job.A, VEC, EPP, NW, static_cast<int>(sizeof(Scalar))), stream, job, geo);
    return hipGetLastError();
}

// Paired layouts compiled for every activation dtype: (VEC, EPP, NW).
#define RAMNET_SCAN_PAIR_LAYOUTS(X) X(1, 8, 4) X(1, 8, 8) X(1, 16, 4) X(1, 16, 8) X(2, 8, 4) X(2, 16, 2) X(2, 16, 4)

template<typename Scalar>
hipError_t scan_pair_dispatch(const SegmentJob &job, const ScanGeom &geo, int vec, int epp, int nw,
                              hipStream_t stream) {
    const int cs = nw * (kWave / 2 / epp) * vec;
    const bool fast = job.C % cs == 0;
#define RAMNET_SCAN_PAIR_CASE(V, E, W)                                                                  \
    if (vec == V && epp == E && nw == W)                                                                \
        return fast ? launch_scan_pair<Scalar, V, E, W, true>(job, geo, stream)              \
                    : launch_scan_pair<Scalar, V, E, W, false>(job, geo, stream);
    RAMNET_SCAN_PAIR_LAYOUTS(RAMNET_SCAN_PAIR_CASE)
#undef RAMNET_SCAN_PAIR_CASE
    return hipErrorInvalidValue;
}

inline bool scan_pair_layout_compiled(int vec, int epp, int nw) {
#define RAMNET_SCAN_PAIR_HAS(V, E, W) if (vec == V && epp == E && nw == W) return true;
    RAMNET_SCAN_PAIR_LAYOUTS(RAMNET_SCAN_PAIR_HAS)
#undef RAMNET_SCAN_PAIR_HAS
    return false;
}

hipError_t launch_scan_pair_f32(const SegmentJob &, const ScanGeom &, int, int, int, hipStream_t);
hipError_t launch_scan_pair_f16(const SegmentJob &, const ScanGeom &, int, int, int, hipStream_t);
hipError_t launch_scan_pair_bf16(const SegmentJob &, const ScanGeom &, int, int, int, hipStream_t);

}  // namespace ramnet
