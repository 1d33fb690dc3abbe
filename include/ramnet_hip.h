/*
 * ramnet_hip.h - C ABI of the MI355X (gfx950) RAM-Net operator library.
 *
 * Each entry point replaces one native operator of the reference extension
 * (packages/ramnet-ops/csrc/ram_attn_bind.cpp:22-113, implemented in
 * ram_attn_ops.cpp). Arguments are raw device pointers, element counts and
 * scalars; no framework types cross this boundary. All tensors are dense,
 * row-major (C-contiguous) in the layouts given below, on the current HIP
 * device. Work is enqueued on `stream` (a hipStream_t; NULL = default
 * stream) and never synchronised; nothing is allocated or freed.
 *
 * Shape symbols: B batch, H heads, U address digits, P radix, A = P**U slots,
 * K top-k, T tokens, C value channels.
 *
 * Return value: RAMNET_OK, or a nonzero RAMNET_E* code with a message
 * available from ramnet_last_error() on the calling thread.
 */
#ifndef RAMNET_HIP_H
#define RAMNET_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RAMNET_ABI_VERSION 3

enum {
    RAMNET_OK = 0,
    RAMNET_EINVAL = 1,  /* bad argument: shape, range, dtype, null pointer, aliasing */
    RAMNET_ELAUNCH = 2, /* the HIP runtime rejected the launch */
};

/* Activation dtypes (logits, values, gamma, y). Slot state is always fp32. */
enum { RAMNET_F32 = 0, RAMNET_F16 = 1, RAMNET_BF16 = 2 };

/* ABI revision of this header. */
int ramnet_abi_version(void);

/* Width of the index type used on device (32). Replaces the `_C.INT_BITS`
 * module constant exported by the reference extension
 * (ram_attn_bind.cpp:115-129; read by impl/_cuda_config.py:4). */
int ramnet_int_bits(void);

/* Message of the last failed call on this thread ("" if none). */
const char *ramnet_last_error(void);

/*
 * Top-K address decoder for one address tensor.
 * Replaces ramnet_ops::topk_addr_single_forward
 * (ram_attn_bind.cpp:27-35, ram_attn_ops.cpp:63-95).
 *   addr          (B, H, U, P, T) logits, `dtype`
 *   position_ids  (B, T) int32, used by heads h < embed_num (CAPE)
 *   idx_out       (B, H, top_k, T) int32: (b*H + h)*A + slot, or h*A + slot
 *                 when encode_batch_idx == 0
 *   val_out       (B, H, top_k, T) fp32 weights, negated if addr_val_neg
 * Requires A == P**U, 0 < top_k <= A, 0 <= embed_num <= H,
 * 0 <= top_k_re_norm <= 1.
 */
int ramnet_topk_addr_single_forward(const void *addr, int dtype, int64_t B, int64_t H, int64_t U, int64_t P,
                                    int64_t T, int64_t embed_num, int64_t A, const int32_t *position_ids,
                                    int64_t top_k, float top_k_re_norm, int addr_val_neg, int encode_batch_idx,
                                    int32_t *idx_out, float *val_out, void *stream);

/*
 * Write and read address decoders in one launch.
 * Replaces ramnet_ops::topk_addr_forward
 * (ram_attn_bind.cpp:46-54, ram_attn_ops.cpp:137-172).
 *   w_addr, r_addr  (B, H, U, P, T) logits, `dtype`
 *   idx_out         (B, H, w_top_k + r_top_k, T) int32; write rows first
 *   val_out         (B, H, w_top_k + r_top_k, T) fp32; write weights
 *                   positive, read weights negated (the sign tells the
 *                   segment scan which events read)
 */
int ramnet_topk_addr_forward(const void *w_addr, const void *r_addr, int dtype, int64_t B, int64_t H, int64_t U,
                             int64_t P, int64_t T, int64_t embed_num, int64_t A, const int32_t *position_ids,
                             int64_t w_top_k, int64_t r_top_k, float w_re_norm, float r_re_norm,
                             int encode_batch_idx, int32_t *idx_out, float *val_out, void *stream);

/*
 * Gradient of one address decoder with respect to its logits (the selection
 * carries none). Replaces ramnet_ops::topk_addr_single_backward
 * (ram_attn_bind.cpp:36-45, ram_attn_ops.cpp:97-135).
 *   idx, val    (B, H, top_k, T): the forward's outputs (either index
 *               encoding; val negated when addr_val_neg)
 *   addr        (B, H, U, P, T) logits, `dtype`
 *   grad_val    (B, H, top_k, T) fp32: gradient with respect to the positive
 *               weights
 *   grad_addr   (B, H, U, P, T) `dtype`, written in full
 */
int ramnet_topk_addr_single_backward(const int32_t *idx, const float *val, const void *addr, const float *grad_val,
                                     int dtype, int64_t B, int64_t H, int64_t U, int64_t P, int64_t T,
                                     int64_t embed_num, int64_t A, const int32_t *position_ids, int64_t top_k,
                                     float top_k_re_norm, int addr_val_neg, void *grad_addr, void *stream);

/*
 * Gradients of both decoders of ramnet_topk_addr_forward (write rows first;
 * read weights stored negated, their gradients with respect to the positive
 * weights). Replaces ramnet_ops::topk_addr_backward
 * (ram_attn_bind.cpp:55-64, ram_attn_ops.cpp:177-224).
 */
int ramnet_topk_addr_backward(const int32_t *idx, const float *val, const void *w_addr, const void *r_addr,
                              const float *grad_val, int dtype, int64_t B, int64_t H, int64_t U, int64_t P, int64_t T,
                              int64_t embed_num, int64_t A, const int32_t *position_ids, int64_t w_top_k,
                              int64_t r_top_k, float w_re_norm, float r_re_norm, void *grad_w_addr,
                              void *grad_r_addr, void *stream);

/*
 * Bytes of device workspace the segment scan needs for B x H heads, T tokens
 * and the given top-k when it keeps a head's slot slice resident in one
 * piece (every shape up to A = 8190 slots): the decoder's per-event records
 * (T padded to 32), then the gain records the precomputed-gain form writes,
 * then one int per token of the read-after-write flags its paired layout
 * uses. A scan only reads the decoder records, so the same records can be
 * scanned again. The 32-bit form returns -1 when the size does not fit an int. No
 * counterpart in the reference, which allocates inside its ops
 * (ram_attn_ops.cpp:251-253); ramnet_segment_workspace_bytes sizes any shape.
 */
int ramnet_scan_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t w_top_k, int64_t r_top_k);
int64_t ramnet_scan_workspace_bytes64(int64_t B, int64_t H, int64_t T, int64_t w_top_k, int64_t r_top_k);

/*
 * Bytes of device workspace of the segment forward entry points
 * (ramnet_topk_segment_forward(_), ramnet_segment_scan,
 * ramnet_ram_attn_forward) for this exact shape and activation dtype: the
 * records above, plus, when the slot space is too wide for one resident
 * slice and is scanned in slot ranges with 16-bit activations,
 * B*H*T*C fp32 read sums carried from range to range (y is rounded once,
 * from the whole sum). -1 for shapes the scan does not take. No counterpart
 * in the reference (it allocates inside its ops, ram_attn_ops.cpp:251-253).
 */
int64_t ramnet_segment_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t A, int64_t C, int64_t w_top_k,
                                       int64_t r_top_k, int dtype);

/*
 * Gated sparse update and top-K read over a whole sequence, returning a new
 * state. Replaces ramnet_ops::topk_segment_forward
 * (ram_attn_bind.cpp:65-73, ram_attn_ops.cpp:226-265). The reference op
 * also takes event-grouping metadata built by a global sort; this library
 * scans time in order and needs none.
 *   addr_idx, addr_val  output of ramnet_topk_addr_forward with
 *                       encode_batch_idx = 1
 *   x                   (B, H, T, C) `dtype`;  gamma (B, H, T) `dtype`
 *   mask                (B, T) uint8/bool (nonzero = valid) or NULL
 *   init_slot/mass      (B, H, A, C) / (B, H, A) fp32
 *   slot_out/mass_out   (B, H, A, C) / (B, H, A) fp32; slot_out may alias
 *                       init_slot, mass_out must not alias init_mass
 *   y                   (B, H, T, C) `dtype`; masked tokens get 0
 *   workspace           >= ramnet_segment_workspace_bytes(B, H, T, A, C, w, r,
 *                       dtype) bytes of device memory, overwritten by the
 *                       call
 */
int ramnet_topk_segment_forward(const int32_t *addr_idx, const float *addr_val, const void *x, const void *gamma,
                                int dtype, const uint8_t *mask, const float *init_slot, const float *init_mass,
                                float *slot_out, float *mass_out, void *y, int64_t B, int64_t H, int64_t T, int64_t A,
                                int64_t C, int64_t w_top_k, int64_t r_top_k, int mass_aware, float eps,
                                void *workspace, int64_t workspace_bytes, void *stream);

/*
 * In-place variant: updates slot and mass. Replaces
 * ramnet_ops::topk_segment_forward_ (ram_attn_bind.cpp:83-91,
 * ram_attn_ops.cpp:312-347). `mass_in` is a copy of the mass state taken
 * before the call (B*H*A fp32, must not alias `mass`): channel slices of one
 * head may start after another slice has already stored the new masses.
 */
int ramnet_topk_segment_forward_(const int32_t *addr_idx, const float *addr_val, const void *x, const void *gamma,
                                 int dtype, const uint8_t *mask, float *slot, float *mass, const float *mass_in,
                                 void *y, int64_t B, int64_t H, int64_t T, int64_t A, int64_t C, int64_t w_top_k,
                                 int64_t r_top_k, int mass_aware, float eps, void *workspace, int64_t workspace_bytes,
                                 void *stream);

/*
 * Gradients of ramnet_topk_segment_forward. Replaces
 * ramnet_ops::topk_segment_backward (ram_attn_bind.cpp:74-82,
 * ram_attn_ops.cpp:267-310); like the forward it takes the decoder outputs
 * instead of event-grouping metadata.
 *   addr_idx, addr_val, x, gamma, mask, init_slot, init_mass
 *                       the forward's inputs
 *   grad_y              (B, H, T, C) `dtype` (the reference casts it to x's
 *                       dtype too); masked tokens' entries are ignored
 *   grad_slot/mass      (B, H, A, C) / (B, H, A) fp32 gradients of the final
 *                       state, or NULL for zero
 *   grad_addr_val       (B, H, Kw + Kr, T) fp32: gradients of the positive
 *                       write and read weights (0 for events that do not act)
 *   grad_x              (B, H, T, C) fp32;  grad_gamma (B, H, T) fp32
 *   grad_init_slot/mass (B, H, A, C) / (B, H, A) fp32
 *   workspace           >= ramnet_segment_backward_workspace_bytes(...) bytes
 * Deterministic: no atomics.
 */
int ramnet_topk_segment_backward(const int32_t *addr_idx, const float *addr_val, const void *x, const void *gamma,
                                 int dtype, const uint8_t *mask, const float *init_slot, const float *init_mass,
                                 const void *grad_y, const float *grad_slot, const float *grad_mass,
                                 float *grad_addr_val, float *grad_x, float *grad_gamma, float *grad_init_slot,
                                 float *grad_init_mass, int64_t B, int64_t H, int64_t T, int64_t A, int64_t C,
                                 int64_t w_top_k, int64_t r_top_k, int mass_aware, float eps, void *workspace,
                                 int64_t workspace_bytes, void *stream);

/* Device workspace bytes of ramnet_topk_segment_backward; -1 for shapes it does not take. */
int64_t ramnet_segment_backward_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t A, int64_t C,
                                                int64_t w_top_k, int64_t r_top_k);

/*
 * Training pair with saved rows: a forward that keeps what the backward
 * would otherwise recompute, and the backward that uses it. No counterpart
 * in the reference, whose backward reconstructs the forward
 * (ram_attn_segment_parallel.cu:418-606); the outputs are those of
 * ramnet_topk_segment_forward and ramnet_topk_segment_backward
 * (ram_attn_bind.cpp:65-82) on the same inputs, to fp32 rounding. For
 * training callers with memory to spare: the saved buffer holds the scan
 * records, the backward's per-event mass records (16 bytes per event), and
 * two fp32 arrays of B*H*T_pad*kp*C*4 bytes (x - s before each write, the
 * row of each read; kp = max(Kw, Kr) rounded up to the backward's event
 * slots, T_pad = T rounded up to 32): 4.5 GB at B=8, H=16, T=4096, C=128,
 * K=8. One backward pass over the sequence, with no replay of the mass
 * pre-pass, then replaces the backward's replay of the forward.
 *
 * ramnet_segment_saved_bytes: bytes of the saved buffer, or -1 where the pair
 * does not apply (the forward must run a one-token precomputed-gain scan
 * over the whole slot space with whole channel slices; B, T > 0). Callers
 * fall back to ramnet_topk_segment_forward/_backward there.
 * ramnet_topk_segment_forward_save: arguments of ramnet_topk_segment_forward
 * plus `saved` (written; kept unchanged until the backward).
 * ramnet_topk_segment_backward_saved: arguments of
 * ramnet_topk_segment_backward without addr_idx and mask (the records are in
 * `saved`), plus `saved`; its workspace is
 * ramnet_segment_backward_saved_workspace_bytes(...) bytes.
 */
int64_t ramnet_segment_saved_bytes(int64_t B, int64_t H, int64_t T, int64_t A, int64_t C, int64_t w_top_k,
                                   int64_t r_top_k, int dtype);
int ramnet_topk_segment_forward_save(const int32_t *addr_idx, const float *addr_val, const void *x,
                                     const void *gamma, int dtype, const uint8_t *mask, const float *init_slot,
                                     const float *init_mass, float *slot_out, float *mass_out, void *y, int64_t B,
                                     int64_t H, int64_t T, int64_t A, int64_t C, int64_t w_top_k, int64_t r_top_k,
                                     int mass_aware, float eps, void *workspace, int64_t workspace_bytes, void *saved,
                                     int64_t saved_bytes, void *stream);
int64_t ramnet_segment_backward_saved_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t A, int64_t C,
                                                      int64_t w_top_k, int64_t r_top_k);
int ramnet_topk_segment_backward_saved(const float *addr_val, const void *x, const void *gamma, int dtype,
                                       const float *init_slot, const float *init_mass, const void *grad_y,
                                       const float *grad_slot, const float *grad_mass, float *grad_addr_val,
                                       float *grad_x, float *grad_gamma, float *grad_init_slot, float *grad_init_mass,
                                       int64_t B, int64_t H, int64_t T, int64_t A, int64_t C, int64_t w_top_k,
                                       int64_t r_top_k, int mass_aware, float eps, const void *saved,
                                       int64_t saved_bytes, void *workspace, int64_t workspace_bytes, void *stream);

/*
 * The two stages of ramnet_ram_attn_forward, for callers that schedule or
 * time them separately. ramnet_topk_addr_records runs both address decoders
 * and writes the scan's per-event records into `workspace` (CAPE, mask,
 * inactive addresses and the forget coefficients from gamma folded in);
 * ramnet_segment_scan runs the scan from those records. Arguments as for
 * ramnet_ram_attn_forward.
 */
int ramnet_topk_addr_records(const void *w_addr, const void *r_addr, const void *gamma, int dtype,
                             const uint8_t *mask, int64_t embed_num, const int32_t *position_ids, int64_t B, int64_t H,
                             int64_t U, int64_t P, int64_t T, int64_t A, int64_t w_top_k, int64_t r_top_k,
                             float w_re_norm, float r_re_norm, void *workspace, int64_t workspace_bytes,
                             void *stream);
int ramnet_segment_scan(const void *x, int dtype, const float *init_slot, const float *init_mass, float *slot_out,
                        float *mass_out, void *y, int64_t B, int64_t H, int64_t T, int64_t A, int64_t C,
                        int64_t w_top_k, int64_t r_top_k, int mass_aware, float eps, void *workspace,
                        int64_t workspace_bytes, void *stream);

/*
 * Whole parallel (prefill) forward: both address decoders and the segment
 * scan, with the decoder writing the scan's per-event records directly (no
 * idx/val round trip). Replaces the parallel branch of the reference's
 * _cuda_ram_attn (packages/ramnet-ops/src/ramnet_ops/impl/cuda_impl.py:
 * 240-271: topk_addr_forward, gather_segment, topk_segment_forward).
 *   w_addr, r_addr  (B, H, U, P, T) logits;  other arguments as for
 *                   ramnet_topk_addr_forward and ramnet_topk_segment_forward
 * For an in-place update pass slot_out == init_slot and a snapshot copy of
 * the masses as init_mass (mass_out must not alias init_mass).
 */
int ramnet_ram_attn_forward(const void *w_addr, const void *r_addr, const void *x, const void *gamma, int dtype,
                            const uint8_t *mask, int64_t embed_num, const int32_t *position_ids,
                            const float *init_slot, const float *init_mass, float *slot_out, float *mass_out, void *y,
                            int64_t B, int64_t H, int64_t U, int64_t P, int64_t T, int64_t A, int64_t C,
                            int64_t w_top_k, int64_t r_top_k, float w_re_norm, float r_re_norm, int mass_aware,
                            float eps, void *workspace, int64_t workspace_bytes, void *stream);

/*
 * One fused decode step on a persistent state, updated in place.
 * Replaces ramnet_ops::topk_autoregressive_ (ram_attn_bind.cpp:92-101,
 * ram_attn_ops.cpp:349-394).
 *   w_addr, r_addr  (B, H, U, P) `dtype`;  x (B, H, C);  gamma (B, H)
 *   slot, mass      (B, H, A, C), (B, H, A) fp32, read-modify-write
 *   mask            (B) uint8/bool or NULL: masked rows keep their state
 *                   and get y = 0
 *   position_ids    (B) int32
 *   y               (B, H, C) `dtype`
 */
int ramnet_topk_autoregressive_(const void *w_addr, const void *r_addr, const void *x, const void *gamma, int dtype,
                                float *slot, float *mass, const uint8_t *mask, int64_t embed_num,
                                const int32_t *position_ids, int64_t B, int64_t H, int64_t U, int64_t P, int64_t A,
                                int64_t C, int64_t w_top_k, int64_t r_top_k, float w_re_norm, float r_re_norm,
                                int mass_aware, float eps, void *y, void *stream);

/*
 * S consecutive decode steps in one call, the same as S calls of
 * ramnet_topk_autoregressive_ on the step slices of the inputs. No
 * counterpart in the reference: a multi-step form of topk_autoregressive_
 * for callers that hold the inputs of several steps at once (replay,
 * benchmarking, speculative verification). Shapes that take the half-wave
 * fast path (P <= 32, top-k <= 11, C <= 256) run as one persistent launch
 * in which step s + 1's addresses are decoded while step s's rows are in
 * flight; other shapes run one launch per step.
 *   w_addr, r_addr  (S, B, H, U, P) `dtype`;  x (S, B, H, C);  gamma (S, B, H)
 *   position_ids    (S, B) int32;  mask (S, B) uint8/bool or NULL
 *   slot, mass      (B, H, A, C), (B, H, A) fp32, read-modify-write
 *   y               (S, B, H, C) `dtype`
 */
int ramnet_topk_autoregressive_steps_(const void *w_addr, const void *r_addr, const void *x, const void *gamma,
                                      int dtype, float *slot, float *mass, const uint8_t *mask, int64_t embed_num,
                                      const int32_t *position_ids, int64_t S, int64_t B, int64_t H, int64_t U,
                                      int64_t P, int64_t A, int64_t C, int64_t w_top_k, int64_t r_top_k,
                                      float w_re_norm, float r_re_norm, int mass_aware, float eps, void *y,
                                      void *stream);

/* Bytes of the per-GPU scratch of ramnet_ram_attn_forward_noalloc (192 MiB:
 * config 2, B=8 H=16 T=4096 K=8 in the precomputed-gain form, needs 162 MiB). */
#define RAMNET_NOALLOC_SCRATCH_BYTES (192LL << 20)

/*
 * ramnet_ram_attn_forward without a workspace argument. No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). It allocates nothing: the per-event records live in a
 * file-scope device array of RAMNET_NOALLOC_SCRATCH_BYTES, one per GPU the
 * library runs on, held until the process ends. A shape whose records
 * (B*H*T_pad*(16*w_top_k + 8*r_top_k) bytes, plus B*H*T_pad*(16*max(w_top_k,
 * r_top_k) + 4) when the scan uses the precomputed-gain form) exceed it returns
 * RAMNET_EINVAL. The array is part of the library's device code: loading
 * the library's code on a GPU reserves RAMNET_NOALLOC_SCRATCH_BYTES of that
 * GPU's memory until the process ends, whether or not this entry point is
 * ever called. Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (other streams, other threads) race, and the caller
 * must order them. Other arguments and results as ramnet_ram_attn_forward.
 */
int ramnet_ram_attn_forward_noalloc(const void *w_addr, const void *r_addr, const void *x, const void *gamma,
                                    int dtype, const uint8_t *mask, int64_t embed_num, const int32_t *position_ids,
                                    const float *init_slot, const float *init_mass, float *slot_out, float *mass_out,
                                    void *y, int64_t B, int64_t H, int64_t U, int64_t P, int64_t T, int64_t A,
                                    int64_t C, int64_t w_top_k, int64_t r_top_k, float w_re_norm, float r_re_norm,
                                    int mass_aware, float eps, void *stream);

/*
 * Planning query (no device work beyond reading the device's CU count): the
 * layout a segment-scan launch of this shape uses on the current device --
 * channel-slice width, LDS bytes per workgroup, and whether it is the
 * precomputed-gain form (a mass pre-pass writes the gain records of the
 * workspace first). Honours RAMNET_SCAN_LAYOUT like the launch does. The
 * answer is for a 4096-token call: a much shorter call may take the
 * mass-wave form instead (the workspace size does not depend on the form).
 * Returns 1 if the shape is supported (top-k <= 128; A <= 8190 in one
 * resident slice, wider slot spaces in the precomputed-gain form split into
 * at most 4096 slot ranges scanned one launch each, within the int32 limits
 * B*H*A*C < 2**31), else 0.
 */
int ramnet_segment_plan(int64_t B, int64_t H, int64_t A, int64_t C, int64_t w_top_k, int64_t r_top_k, int dtype,
                        int *slice_channels, int *lds_bytes, int *precomputed_gains);

#ifdef __cplusplus
}
#endif

#endif /* RAMNET_HIP_H */
