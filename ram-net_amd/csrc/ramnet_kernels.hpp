// Host-side launch interface shared by the kernel translation units and the
// C-ABI layer. Everything here is plain data: raw device pointers, sizes and
// scalars. Shapes are validated by the C-ABI layer before any launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ramnet {

enum DType : int { kF32 = 0, kF16 = 1, kBF16 = 2 };

// One address tensor to decode: logits (B, H, U, P, T) in `dtype`.
struct AddrSource {
    const void *addr;
    int top_k;
    float re_norm;  // top_k_re_norm exponent r in [0, 1]
    float sign;     // +1, or -1 when the weights are returned negated
    int k_off;      // first row of this address in the (B, H, k_total, T) outputs
};

// Per-event records consumed by the segment scan, laid out
// [b*H + h][event][t] with t padded to a multiple of kScanPad (an even
// number of kScanChunk-token chunks, so the scan's two prefetch buffers
// alternate without a tail case). Slots are
// local to the (b, h) head after CAPE. Events that must not act (masked or
// padding tokens, inactive addresses, zero weights) point at dummy LDS rows
// in front of the state: writes at slot -2 (weight 0, alpha 1), reads at
// slot -1 (weight 0). The workspace holds, in order: write records
// (B*H, Kw, T_pad), read records (B*H, Kr, T_pad), then the gain records of
// the precomputed-gain scan (B*H, T_pad, max(Kw, Kr)) of GainRec, token-major
// so that the events of one token, which the scan's lanes load together,
// are contiguous, then the paired scan's flags (B*H, T_pad) of int. The
// decoder records are never modified after they are written, so one set of
// records can be scanned any number of times.
constexpr int kScanChunk = 16;
constexpr int kScanPad = 2 * kScanChunk;
struct WriteRec {
    int slot;
    float w;
    float alpha;
    float overlap;  // int bits, event 0: bit d - 1 set if a slot of this token is also written by token t - d
                    // (d = 1, 2, 3), or if that is not known
};
struct ReadRec {
    int slot;
    float r;
};

// One event of the precomputed-gain scan, written by the mass pre-pass:
// write event e and read event e of one token, for every event below
// max(Kw, Kr) (past Kw a no-op write, past Kr a no-op read) and every token
// below T (the padding tokens are not written).
struct GainRec {
    int wslot;
    float gain;
    int rslot;
    float r;  // effective read weight (mass-aware), else the read weight
};

__host__ __device__ inline int scan_t_pad(int T) { return (T + kScanPad - 1) / kScanPad * kScanPad; }
inline int64_t scan_t_pad64(int64_t T) { return (T + kScanPad - 1) / kScanPad * kScanPad; }

// Workspace bytes: the decoder records alone, and with the gain records.
inline int64_t scan_record_bytes(int64_t B, int64_t H, int64_t T, int64_t Kw, int64_t Kr) {
    return B * H * scan_t_pad64(T) *
           (Kw * static_cast<int64_t>(sizeof(WriteRec)) + Kr * static_cast<int64_t>(sizeof(ReadRec)));
}
inline int64_t scan_gain_bytes(int64_t B, int64_t H, int64_t T, int64_t Kw, int64_t Kr) {
    return B * H * scan_t_pad64(T) * (Kw > Kr ? Kw : Kr) * static_cast<int64_t>(sizeof(GainRec));
}
// The paired scan's read-after-write flags, one int per (b, h, padded token).
inline int64_t scan_flag_bytes(int64_t B, int64_t H, int64_t T) {
    return B * H * scan_t_pad64(T) * static_cast<int64_t>(sizeof(int));
}

// Decode one or two address tensors (write and read) sharing a shape.
struct AddrJob {
    AddrSource src[2];
    int n_src;
    int dtype;
    int B, H, U, P, T, A;
    int embed_num;           // CAPE applies to heads h < embed_num
    int encode_batch_idx;    // idx = (b*H + h)*A + a, else h*A + a
    int k_total;
    const int32_t *position_ids;  // (B, T)
    int32_t *idx_out;             // (B, H, k_total, T)
    float *val_out;               // (B, H, k_total, T)
    // Record mode (both set): instead of idx/val, write scan records for
    // t < T_pad, source 0 as writes, source 1 as reads.
    WriteRec *wrec;               // (B*H, Kw, T_pad)
    ReadRec *rrec;                // (B*H, Kr, T_pad)
    const void *gamma;            // (B, H, T) in dtype, for alpha
    const uint8_t *mask;          // (B, T) or null
};

// Decoder backward for one address source: gradient of the top-K weights
// (positive-weight convention) -> gradient of the logits.
struct AddrBwdJob {
    const void *addr;             // (B, H, U, P, T) logits in dtype
    const int32_t *idx;           // (B, H, k_total, T), this source at k_off .. k_off + K
    const float *val;             // (B, H, k_total, T), stored weights (negated when sign < 0)
    const float *grad_val;        // (B, H, k_total, T), gradient of the positive weights
    void *grad_addr;              // (B, H, U, P, T) in dtype
    const int32_t *position_ids;  // (B, T)
    int dtype;
    int B, H, U, P, T, A;
    int embed_num;
    int k_total, k_off, K;
    float re_norm;
    float sign;
};

// Per-event forward quantities of the segment backward, written by the mass
// pre-pass in its record-keeping mode. Token-major: (B*H, T, K).
struct MassAux {
    int4 *wev;   // (B*H, T, Kw) {slot, or -2 for a no-op; gain g = w / (m + eps); effective weight of
                 //  the read of the same slot in this token, or 0; slot mass before the write} (floats as bits)
    int4 *rev;   // (B*H, T, Kr) {slot, or -1 for a no-op; effective read weight; post-write mass of
                 //  the slot; 0} (floats as bits)
};

// Rows a training forward saves for the segment backward, laid out in the
// backward's channel slices: (B*H*n_sub, T_pad, kp, csw) floats each, n_sub
// slices of csw channels (a power of two), kp padded event slots per token,
// T_pad = scan_t_pad(T) (the padding tokens' rows are written, never read).
struct SavedRows {
    float *w;  // per write event: x_t - s before the write; null: nothing saved
    float *r;  // per read event: the row read, after the token's writes
    int n_sub, kp, csw;
    // the backward's per-event records, written by the forward's mass
    // pre-pass alongside the gains (null: the backward replays it)
    MassAux aux;
};

// Time-sequential gated sparse update + top-K read over a whole sequence.
struct SegmentJob {
    const WriteRec *wrec;     // (B*H, Kw, T_pad) scan records
    const ReadRec *rrec;      // (B*H, Kr, T_pad)
    GainRec *gain;            // (B*H, max(Kw, Kr), T_pad): written by the mass pre-pass, or null
    const void *x;            // (B, H, T, C) in dtype
    const float *init_slot;   // (B, H, A, C)
    const float *init_mass;   // (B, H, A)
    float *slot_out;          // (B, H, A, C); may alias init_slot
    float *mass_out;          // (B, H, A); may alias init_mass
    void *y;                  // (B, H, T, C) in dtype
    // (B, H, T, C) fp32 read sums carried from one slot range to the next
    // when the scan is split into slot ranges: y itself for fp32 y, else a
    // workspace buffer (so y is rounded once, from the full sum)
    float *yacc;
    // (B*H, T_pad) per token: 1 if one of its write slots is a read slot of
    // the token before (or if that is not known), else 0. Written by the mass
    // pre-pass for the paired scan (segment_scan_pair.hpp); null otherwise.
    int *flags;
    SavedRows save;           // rows for the segment backward (save.w null: none)
    int dtype;
    int B, H, T, A, C, Kw, Kr;
    int mass_aware;
    float eps;
};


// Segment backward (gradients of ramnet_topk_segment_forward).
struct SegmentBwdJob {
    SegmentJob fwd;           // records, x, init state, shapes (y, slot_out unused)
    MassAux aux;
    const float *addr_val;    // (B, H, Kw + Kr, T) decoder weights (reads negated)
    const void *gamma;        // (B, H, T) in dtype
    const void *grad_y;       // (B, H, T, C) in dtype
    const float *grad_slot;   // (B, H, A, C) or null (zero)
    const float *grad_mass;   // (B, H, A) or null (zero)
    float *grad_val;          // (B, H, Kw + Kr, T): positive-weight gradients
    float *grad_x;            // (B, H, T, C)
    float *grad_gamma;        // (B, H, T)
    float *grad_init_slot;    // (B, H, A, C)
    float *grad_init_mass;    // (B, H, A)
    float *delta;             // (B*H*n_sub, T_pad, KP, CSW) x - s before each write (KP: padded event count)
    const float *saved_r;     // same layout: the rows read, saved by the forward (then delta too); else null
    int aux_saved;            // 1: `aux` was written by the forward (no replay here)
    float *dr_part;           // (n_sub, B*H, T_pad, KP) per-slice read dot products
    float *dg_part;           // (n_sub, B*H, T_pad, KP) per-slice gain gradients
    float *dr_sum;            // (B*H, T, Kr) read dot products d_j
    float *dg_sum;            // (B*H, T, Kw) gain gradients Dg
    float *mass_scratch;      // (B*H*A)
    void *maps;               // chunk maps of the mass replay
    size_t maps_bytes;
};

// One fused autoregressive step: decode, K writes, then K reads.
struct DecodeJob {
    const void *w_addr;       // (B, H, U, P)
    const void *r_addr;       // (B, H, U, P)
    const void *x;            // (B, H, C)
    const void *gamma;        // (B, H)
    const uint8_t *mask;      // (B) or null
    const int32_t *position_ids;  // (B)
    float *slot;              // (B, H, A, C), updated in place
    float *mass;              // (B, H, A), updated in place
    void *y;                  // (B, H, C)
    int dtype;
    int B, H, U, P, A, C, Kw, Kr;
    int embed_num;
    float w_re_norm, r_re_norm;
    int mass_aware;
    float eps;
};

// Launchers return hipSuccess or the launch error; `why` receives a static
// message when the shape is outside what the kernels were built for.
hipError_t launch_topk_addr(const AddrJob &job, hipStream_t stream, const char **why);
hipError_t launch_topk_addr_backward(const AddrBwdJob &job, hipStream_t stream, const char **why);
hipError_t launch_segment_forward(const SegmentJob &job, hipStream_t stream, const char **why);

// Build scan records from decoder outputs idx/val (B, H, Kw + Kr, T).
struct PackJob {
    const int32_t *addr_idx;
    const float *addr_val;
    const void *gamma;        // (B, H, T) in dtype
    const uint8_t *mask;      // (B, T) or null
    WriteRec *wrec;
    ReadRec *rrec;
    int dtype;
    int B, H, T, A, Kw, Kr;
};
hipError_t launch_pack_records(const PackJob &job, hipStream_t stream, const char **why);
hipError_t launch_autoregressive(const DecodeJob &job, hipStream_t stream, const char **why);
// S consecutive decode steps; the inputs, y, position_ids and mask of a
// DecodeJob carry a leading step dimension (S, ...).
// Candidate buffer (a power of two) of the staircase address search for
// radix P, top-K K and NPD = pow2 >= P.
int stair_buffer(int P, int K, int NPD);
hipError_t launch_autoregressive_steps(const DecodeJob &job, int S, hipStream_t stream, const char **why);

// Channel-slice width, dynamic LDS bytes, form (1: precomputed gains) and
// number of slot ranges that a segment-scan launch of this shape uses on the
// current device.
int segment_plan(int B, int H, int T, int A, int C, int Kw, int Kr, int dtype, int *cs, int *lds_bytes, int *pre,
                 int *ranges = nullptr);

// Mass pre-pass in record-keeping mode: the records stay as they are and
// `aux` receives the per-event quantities. `maps` holds the chunk maps
// (mass_replay_scratch_bytes of it); the final masses go to job.mass_out.
int64_t mass_replay_scratch_bytes(int B, int H, int T, int A);
// Time chunks (and their length) the pre-pass uses with maps_bytes of maps.
int mass_replay_chunks(const SegmentJob &job, size_t maps_bytes, int *chunk_len);
hipError_t launch_mass_replay(const SegmentJob &job, const MassAux &aux, void *maps, size_t maps_bytes,
                              hipStream_t stream);

// Segment backward. segment_backward_layout places the backward's buffers
// (everything in SegmentBwdJob past `fwd` and the inputs/outputs) in `base`
// and returns their total size in bytes (-1: shape not supported); with a
// null `base` it only sizes. The launch expects the scan records already
// packed into job.fwd's workspace.
// With `saved`, the rows x - s come from the forward (SavedRows) and the
// layout holds no buffer for them.
int64_t segment_backward_layout(int B, int H, int T, int A, int C, int Kw, int Kr, char *base, SegmentBwdJob *job,
                                bool saved = false);
// The channel slices (n_sub, kp, csw) in which a forward saves rows for the
// backward of this shape; false where the backward takes no saved rows.
bool segment_saved_slices(int A, int C, int Kw, int Kr, SavedRows *geo);
// Whether a forward of this shape can save rows in those slices on the
// current device (a one-token precomputed-gain scan over the whole slot
// space, with whole channel slices).
bool segment_forward_can_save(int B, int H, int T, int A, int C, int Kw, int Kr, int dtype, const SavedRows &geo);
// Whether a saving forward also keeps the backward's per-event records
// (MassAux): the record-keeping pre-pass holds the slot space in one piece.
bool segment_saved_aux(int A);
hipError_t launch_segment_backward(const SegmentBwdJob &job, hipStream_t stream, const char **why);

}  // namespace ramnet
