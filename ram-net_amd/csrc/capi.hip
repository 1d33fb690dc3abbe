// C-ABI entry points: argument validation, then one launch on the caller's
// stream. Errors never abort: they set a thread-local message and return a
// nonzero code (the reference raises RuntimeError from the same checks,
// csrc/cuda_utils.cuh:375-391 and ram_attn_topk_addr.cu:241-246).
#include "ramnet_hip.h"
#include "ramnet_kernels.hpp"
#include "ramnet_search.hpp"

#include <atomic>
#include <mutex>
#include <stdio.h>
#include <string>

namespace {

thread_local std::string g_last_error;

constexpr int64_t kIntMax = 0x7fffffffLL;
constexpr int64_t kAddressLimit = 1LL << 30;  // headroom bit for index arithmetic

int fail(int code, const std::string &msg) {
    g_last_error = msg;
    return code;
}

#define RAMNET_REQUIRE(cond, msg)              \
    do {                                       \
        if (!(cond))                           \
            return fail(RAMNET_EINVAL, (msg)); \
    } while (0)

bool valid_dtype(int d) { return d == RAMNET_F32 || d == RAMNET_F16 || d == RAMNET_BF16; }

// A == P**U without overflow.
bool is_power(int64_t P, int64_t U, int64_t A) {
    int64_t v = 1;
    for (int64_t u = 0; u < U; ++u) {
        v *= P;
        if (v > kAddressLimit)
            return false;
    }
    return v == A;
}

bool fits_int(std::initializer_list<int64_t> prods) {
    for (int64_t p : prods)
        if (p < 0 || p >= kIntMax)
            return false;
    return true;
}

int finish(hipError_t err, const char *why, const char *what) {
    if (err == hipSuccess) {
        g_last_error.clear();
        return RAMNET_OK;
    }
    if (why)
        return fail(RAMNET_EINVAL, why);
    return fail(RAMNET_ELAUNCH, std::string(what) + ": " + hipGetErrorString(err));
}

int check_addr_shape(int64_t B, int64_t H, int64_t U, int64_t P, int64_t T, int64_t embed_num, int64_t A) {
    RAMNET_REQUIRE(B >= 0 && H > 0 && U > 0 && P > 0 && T >= 0, "address shape must have B, T >= 0 and H, U, P > 0");
    RAMNET_REQUIRE(A > 0 && A < kAddressLimit, "Address space overflow: A must be in (0, 2**30)");
    RAMNET_REQUIRE(is_power(P, U, A), "A must equal P**U");
    RAMNET_REQUIRE(embed_num >= 0 && embed_num <= H, "embed_num must be in [0, H]");
    return RAMNET_OK;
}


// One decoder source of a backward call (the k rows k_off .. k_off + top_k).
int addr_backward(const int32_t *idx, const float *val, const void *addr, const float *grad_val, int dtype,
                  int64_t B, int64_t H, int64_t U, int64_t P, int64_t T, int64_t embed_num, int64_t A,
                  const int32_t *position_ids, int64_t k_total, int64_t k_off, int64_t top_k, float re_norm,
                  float sign, void *grad_addr, void *stream) {
    ramnet::AddrBwdJob job{};
    job.addr = addr;
    job.idx = idx;
    job.val = val;
    job.grad_val = grad_val;
    job.grad_addr = grad_addr;
    job.position_ids = position_ids;
    job.dtype = dtype;
    job.B = static_cast<int>(B);
    job.H = static_cast<int>(H);
    job.U = static_cast<int>(U);
    job.P = static_cast<int>(P);
    job.T = static_cast<int>(T);
    job.A = static_cast<int>(A);
    job.embed_num = static_cast<int>(embed_num);
    job.k_total = static_cast<int>(k_total);
    job.k_off = static_cast<int>(k_off);
    job.K = static_cast<int>(top_k);
    job.re_norm = re_norm;
    job.sign = sign;
    const char *why = nullptr;
    const hipError_t err = ramnet::launch_topk_addr_backward(job, static_cast<hipStream_t>(stream), &why);
    return finish(err, why, "topk_addr backward launch");
}

}  // namespace

extern "C" {

int ramnet_abi_version(void) { return RAMNET_ABI_VERSION; }

int ramnet_int_bits(void) { return 32; }

const char *ramnet_last_error(void) { return g_last_error.c_str(); }

int ramnet_topk_addr_single_forward(const void *addr, int dtype, int64_t B, int64_t H, int64_t U, int64_t P,
                                    int64_t T, int64_t embed_num, int64_t A, const int32_t *position_ids,
                                    int64_t top_k, float top_k_re_norm, int addr_val_neg, int encode_batch_idx,
                                    int32_t *idx_out, float *val_out, void *stream) {
    if (int rc = check_addr_shape(B, H, U, P, T, embed_num, A))
        return rc;
    RAMNET_REQUIRE(valid_dtype(dtype), "addr dtype must be float32, float16 or bfloat16");
    RAMNET_REQUIRE(top_k > 0 && top_k <= A, "top_k must be in [1, A]");
    RAMNET_REQUIRE(top_k_re_norm >= 0.f && top_k_re_norm <= 1.f, "top_k_re_norm must be in [0, 1]");
    RAMNET_REQUIRE(fits_int({B * H * U * P * T, B * H * A, B * H * top_k * T}), "CUDA index overflow: sizes exceed int32");
    if (B * T == 0)
        return RAMNET_OK;
    RAMNET_REQUIRE(addr && position_ids && idx_out && val_out, "null tensor pointer");
    ramnet::AddrJob job{};
    job.src[0] = {addr, static_cast<int>(top_k), top_k_re_norm, addr_val_neg ? -1.f : 1.f, 0};
    job.n_src = 1;
    job.dtype = dtype;
    job.B = static_cast<int>(B);
    job.H = static_cast<int>(H);
    job.U = static_cast<int>(U);
    job.P = static_cast<int>(P);
    job.T = static_cast<int>(T);
    job.A = static_cast<int>(A);
    job.embed_num = static_cast<int>(embed_num);
    job.encode_batch_idx = encode_batch_idx ? 1 : 0;
    job.k_total = static_cast<int>(top_k);
    job.position_ids = position_ids;
    job.idx_out = idx_out;
    job.val_out = val_out;
    const char *why = nullptr;
    const hipError_t err = ramnet::launch_topk_addr(job, static_cast<hipStream_t>(stream), &why);
    return finish(err, why, "topk_addr_single_forward launch");
}

int ramnet_topk_addr_single_backward(const int32_t *idx, const float *val, const void *addr, const float *grad_val,
                                     int dtype, int64_t B, int64_t H, int64_t U, int64_t P, int64_t T,
                                     int64_t embed_num, int64_t A, const int32_t *position_ids, int64_t top_k,
                                     float top_k_re_norm, int addr_val_neg, void *grad_addr, void *stream) {
    if (int rc = check_addr_shape(B, H, U, P, T, embed_num, A))
        return rc;
    RAMNET_REQUIRE(valid_dtype(dtype), "addr dtype must be float32, float16 or bfloat16");
    RAMNET_REQUIRE(top_k > 0 && top_k <= A, "top_k must be in [1, A]");
    RAMNET_REQUIRE(top_k_re_norm >= 0.f && top_k_re_norm <= 1.f, "top_k_re_norm must be in [0, 1]");
    RAMNET_REQUIRE(fits_int({B * H * U * P * T, B * H * A, B * H * top_k * T}), "CUDA index overflow: sizes exceed int32");
    if (B * H * T == 0)
        return RAMNET_OK;
    RAMNET_REQUIRE(idx && val && addr && grad_val && position_ids && grad_addr, "null tensor pointer");
    return addr_backward(idx, val, addr, grad_val, dtype, B, H, U, P, T, embed_num, A, position_ids, top_k, 0, top_k,
                         top_k_re_norm, addr_val_neg ? -1.f : 1.f, grad_addr, stream);
}

int ramnet_topk_addr_backward(const int32_t *idx, const float *val, const void *w_addr, const void *r_addr,
                              const float *grad_val, int dtype, int64_t B, int64_t H, int64_t U, int64_t P, int64_t T,
                              int64_t embed_num, int64_t A, const int32_t *position_ids, int64_t w_top_k,
                              int64_t r_top_k, float w_re_norm, float r_re_norm, void *grad_w_addr,
                              void *grad_r_addr, void *stream) {
    if (int rc = check_addr_shape(B, H, U, P, T, embed_num, A))
        return rc;
    RAMNET_REQUIRE(valid_dtype(dtype), "addr dtype must be float32, float16 or bfloat16");
    RAMNET_REQUIRE(w_top_k > 0 && w_top_k <= A && r_top_k > 0 && r_top_k <= A, "top_k values must be in [1, A]");
    RAMNET_REQUIRE(w_re_norm >= 0.f && w_re_norm <= 1.f && r_re_norm >= 0.f && r_re_norm <= 1.f,
                   "top_k_re_norm exponents must be in [0, 1]");
    RAMNET_REQUIRE(fits_int({B * H * U * P * T, B * H * A, B * H * (w_top_k + r_top_k) * T}),
                   "CUDA index overflow: sizes exceed int32");
    if (B * H * T == 0)
        return RAMNET_OK;
    RAMNET_REQUIRE(idx && val && w_addr && r_addr && grad_val && position_ids && grad_w_addr && grad_r_addr,
                   "null tensor pointer");
    const int64_t kt = w_top_k + r_top_k;
    if (int rc = addr_backward(idx, val, w_addr, grad_val, dtype, B, H, U, P, T, embed_num, A, position_ids, kt, 0,
                               w_top_k, w_re_norm, 1.f, grad_w_addr, stream))
        return rc;
    return addr_backward(idx, val, r_addr, grad_val, dtype, B, H, U, P, T, embed_num, A, position_ids, kt, w_top_k,
                         r_top_k, r_re_norm, -1.f, grad_r_addr, stream);
}

int ramnet_topk_addr_forward(const void *w_addr, const void *r_addr, int dtype, int64_t B, int64_t H, int64_t U,
                             int64_t P, int64_t T, int64_t embed_num, int64_t A, const int32_t *position_ids,
                             int64_t w_top_k, int64_t r_top_k, float w_re_norm, float r_re_norm,
                             int encode_batch_idx, int32_t *idx_out, float *val_out, void *stream) {
    if (int rc = check_addr_shape(B, H, U, P, T, embed_num, A))
        return rc;
    RAMNET_REQUIRE(valid_dtype(dtype), "addr dtype must be float32, float16 or bfloat16");
    RAMNET_REQUIRE(w_top_k > 0 && w_top_k <= A && r_top_k > 0 && r_top_k <= A, "top_k values must be in [1, A]");
    RAMNET_REQUIRE(w_re_norm >= 0.f && w_re_norm <= 1.f && r_re_norm >= 0.f && r_re_norm <= 1.f,
                   "top_k_re_norm exponents must be in [0, 1]");
    RAMNET_REQUIRE(fits_int({B * H * U * P * T, B * H * A, B * H * (w_top_k + r_top_k) * T}),
                   "CUDA index overflow: sizes exceed int32");
    if (B * T == 0)
        return RAMNET_OK;
    RAMNET_REQUIRE(w_addr && r_addr && position_ids && idx_out && val_out, "null tensor pointer");
    ramnet::AddrJob job{};
    job.src[0] = {w_addr, static_cast<int>(w_top_k), w_re_norm, 1.f, 0};
    job.src[1] = {r_addr, static_cast<int>(r_top_k), r_re_norm, -1.f, static_cast<int>(w_top_k)};
    job.n_src = 2;
    job.dtype = dtype;
    job.B = static_cast<int>(B);
    job.H = static_cast<int>(H);
    job.U = static_cast<int>(U);
    job.P = static_cast<int>(P);
    job.T = static_cast<int>(T);
    job.A = static_cast<int>(A);
    job.embed_num = static_cast<int>(embed_num);
    job.encode_batch_idx = encode_batch_idx ? 1 : 0;
    job.k_total = static_cast<int>(w_top_k + r_top_k);
    job.position_ids = position_ids;
    job.idx_out = idx_out;
    job.val_out = val_out;
    const char *why = nullptr;
    const hipError_t err = ramnet::launch_topk_addr(job, static_cast<hipStream_t>(stream), &why);
    return finish(err, why, "topk_addr_forward launch");
}

// Decoder records, then the gain records of the precomputed-gain scan and
// the paired scan's flags.
static int64_t scan_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t Kw, int64_t Kr) {
    return ramnet::scan_record_bytes(B, H, T, Kw, Kr) + ramnet::scan_gain_bytes(B, H, T, Kw, Kr) +
           ramnet::scan_flag_bytes(B, H, T);
}

// fp32 read sums that a scan in slot ranges carries from range to range
// (B*H*T*C floats after the gain records), when y is 16-bit (fp32 y holds
// them itself). `plan_ok` is false for shapes the scan does not take.
static int64_t range_sum_bytes(int64_t B, int64_t H, int64_t T, int64_t A, int64_t C, int64_t Kw, int64_t Kr,
                               int dtype, bool *plan_ok = nullptr) {
    int ranges = 1;
    const bool ok = B > 0 && H > 0 && T >= 0 && A > 0 && A < kAddressLimit && C > 0 && Kw > 0 && Kr > 0 &&
                    valid_dtype(dtype) && fits_int({B * H * A * C, B * H * (A + 2), B * H * T * C}) &&
                    ramnet::segment_plan(static_cast<int>(B), static_cast<int>(H), static_cast<int>(T),
                                         static_cast<int>(A), static_cast<int>(C), static_cast<int>(Kw),
                                         static_cast<int>(Kr), dtype, nullptr, nullptr, nullptr, &ranges);
    if (plan_ok)
        *plan_ok = ok;
    return ok && ranges > 1 && dtype != RAMNET_F32 ? B * H * T * C * 4 : 0;
}

// The whole workspace of a segment forward of this shape.
static int64_t segment_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t A, int64_t C, int64_t Kw,
                                       int64_t Kr, int dtype) {
    return scan_workspace_bytes(B, H, T, Kw, Kr) + range_sum_bytes(B, H, T, A, C, Kw, Kr, dtype);
}

// Checks shared by the segment entry points; fills the scan job.
// `need` is the workspace the caller's entry point requires (-1: the scan's).
static int segment_checks(const void *x, const void *gamma, int dtype, const float *init_slot, const float *init_mass,
                          float *slot_out, float *mass_out, void *y, int64_t B, int64_t H, int64_t T, int64_t A,
                          int64_t C, int64_t w_top_k, int64_t r_top_k, float eps, void *workspace,
                          int64_t workspace_bytes, int64_t need = -1) {
    RAMNET_REQUIRE(B >= 0 && H > 0 && T >= 0 && C > 0, "segment shape must have B, T >= 0 and H, C > 0");
    RAMNET_REQUIRE(A > 0 && A < kAddressLimit, "Address space overflow: A must be in (0, 2**30)");
    RAMNET_REQUIRE(valid_dtype(dtype), "x dtype must be float32, float16 or bfloat16");
    RAMNET_REQUIRE(w_top_k > 0 && w_top_k <= A && r_top_k > 0 && r_top_k <= A, "top_k values must be in [1, A]");
    RAMNET_REQUIRE(eps > 0.f, "eps must be > 0");
    RAMNET_REQUIRE(fits_int({B * H * A * C, B * H * (A + 2), B * H * T * C, B * H * (T + ramnet::kScanPad) * (w_top_k + r_top_k)}),
                   "CUDA index overflow: sizes exceed int32");
    if (B == 0)
        return RAMNET_OK;
    RAMNET_REQUIRE(init_slot && init_mass && slot_out && mass_out, "null state pointer");
    RAMNET_REQUIRE(static_cast<const void *>(init_mass) != static_cast<const void *>(mass_out),
                   "mass_out must not alias init_mass");
    RAMNET_REQUIRE(T == 0 || (x && gamma && y), "null tensor pointer");
    if (need < 0)
        need = segment_workspace_bytes(B, H, T, A, C, w_top_k, r_top_k, dtype);
    RAMNET_REQUIRE(workspace_bytes >= need && (T == 0 || workspace),
                   "workspace too small: see ramnet_segment_workspace_bytes");
    return RAMNET_OK;
}

static ramnet::SegmentJob make_segment_job(const void *x, int dtype, const float *init_slot, const float *init_mass,
                                           float *slot_out, float *mass_out, void *y, int64_t B, int64_t H,
                                           int64_t T, int64_t A, int64_t C, int64_t w_top_k, int64_t r_top_k,
                                           int mass_aware, float eps, void *workspace) {
    ramnet::SegmentJob job{};
    const int64_t t_pad = ramnet::scan_t_pad64(T);
    job.wrec = static_cast<const ramnet::WriteRec *>(workspace);
    const char *ws = static_cast<const char *>(workspace);
    const int64_t w_bytes = B * H * t_pad * w_top_k * static_cast<int64_t>(sizeof(ramnet::WriteRec));
    const int64_t r_bytes = B * H * t_pad * r_top_k * static_cast<int64_t>(sizeof(ramnet::ReadRec));
    job.rrec = reinterpret_cast<const ramnet::ReadRec *>(ws + w_bytes);
    job.gain = reinterpret_cast<ramnet::GainRec *>(const_cast<char *>(ws) + w_bytes + r_bytes);
    job.flags = reinterpret_cast<int *>(const_cast<char *>(ws) + w_bytes + r_bytes +
                                        ramnet::scan_gain_bytes(B, H, T, w_top_k, r_top_k));
    // fp32 read sums of a scan in slot ranges: y itself, or after the gain records
    if (y && B * T > 0)
        job.yacc = dtype == RAMNET_F32 ? static_cast<float *>(y)
                                       : reinterpret_cast<float *>(const_cast<char *>(ws) +
                                                                   scan_workspace_bytes(B, H, T, w_top_k, r_top_k));
    job.x = x;
    job.init_slot = init_slot;
    job.init_mass = init_mass;
    job.slot_out = slot_out;
    job.mass_out = mass_out;
    job.y = y;
    job.dtype = dtype;
    job.B = static_cast<int>(B);
    job.H = static_cast<int>(H);
    job.T = static_cast<int>(T);
    job.A = static_cast<int>(A);
    job.C = static_cast<int>(C);
    job.Kw = static_cast<int>(w_top_k);
    job.Kr = static_cast<int>(r_top_k);
    job.mass_aware = mass_aware ? 1 : 0;
    job.eps = eps;
    return job;
}

// Scan records from decoder outputs, into the job's workspace.
static hipError_t pack_decoded(const ramnet::SegmentJob &job, const int32_t *addr_idx, const float *addr_val,
                               const void *gamma, const uint8_t *mask, hipStream_t s, const char **why) {
    ramnet::PackJob pack{};
    pack.addr_idx = addr_idx;
    pack.addr_val = addr_val;
    pack.gamma = gamma;
    pack.mask = mask;
    pack.wrec = const_cast<ramnet::WriteRec *>(job.wrec);
    pack.rrec = const_cast<ramnet::ReadRec *>(job.rrec);
    pack.dtype = job.dtype;
    pack.B = job.B;
    pack.H = job.H;
    pack.T = job.T;
    pack.A = job.A;
    pack.Kw = job.Kw;
    pack.Kr = job.Kr;
    return ramnet::launch_pack_records(pack, s, why);
}

static int segment_from_decoded(const int32_t *addr_idx, const float *addr_val, const void *x, const void *gamma,
                                int dtype, const uint8_t *mask, const float *init_slot, const float *init_mass,
                                float *slot_out, float *mass_out, void *y, int64_t B, int64_t H, int64_t T, int64_t A,
                                int64_t C, int64_t w_top_k, int64_t r_top_k, int mass_aware, float eps,
                                void *workspace, int64_t workspace_bytes, void *stream, const char *what) {
    if (int rc = segment_checks(x, gamma, dtype, init_slot, init_mass, slot_out, mass_out, y, B, H, T, A, C, w_top_k,
                                r_top_k, eps, workspace, workspace_bytes))
        return rc;
    if (B == 0)
        return RAMNET_OK;
    RAMNET_REQUIRE(T == 0 || (addr_idx && addr_val), "null tensor pointer");
    ramnet::SegmentJob job = make_segment_job(x, dtype, init_slot, init_mass, slot_out, mass_out, y, B, H, T, A, C,
                                              w_top_k, r_top_k, mass_aware, eps, workspace);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const char *why = nullptr;
    if (T > 0) {
        const hipError_t err = pack_decoded(job, addr_idx, addr_val, gamma, mask, s, &why);
        if (err != hipSuccess)
            return finish(err, why, what);
    }
    const hipError_t err = ramnet::launch_segment_forward(job, s, &why);
    return finish(err, why, what);
}

int ramnet_scan_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t w_top_k, int64_t r_top_k) {
    if (B < 0 || H < 0 || T < 0 || w_top_k < 0 || r_top_k < 0)
        return -1;
    const int64_t n = scan_workspace_bytes(B, H, T, w_top_k, r_top_k);
    return n > 0x7fffffffLL ? -1 : static_cast<int>(n);
}

int64_t ramnet_scan_workspace_bytes64(int64_t B, int64_t H, int64_t T, int64_t w_top_k, int64_t r_top_k) {
    if (B < 0 || H < 0 || T < 0 || w_top_k < 0 || r_top_k < 0)
        return -1;
    return scan_workspace_bytes(B, H, T, w_top_k, r_top_k);
}

int64_t ramnet_segment_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t A, int64_t C, int64_t w_top_k,
                                       int64_t r_top_k, int dtype) {
    if (B < 0 || H < 0 || T < 0 || w_top_k < 0 || r_top_k < 0 || A <= 0 || C <= 0 || !valid_dtype(dtype))
        return -1;
    if (B * H * T == 0)
        return scan_workspace_bytes(B, H, T, w_top_k, r_top_k);
    bool ok = false;
    const int64_t extra = range_sum_bytes(B, H, T, A, C, w_top_k, r_top_k, dtype, &ok);
    return ok ? scan_workspace_bytes(B, H, T, w_top_k, r_top_k) + extra : -1;
}

int ramnet_topk_segment_forward(const int32_t *addr_idx, const float *addr_val, const void *x, const void *gamma,
                                int dtype, const uint8_t *mask, const float *init_slot, const float *init_mass,
                                float *slot_out, float *mass_out, void *y, int64_t B, int64_t H, int64_t T, int64_t A,
                                int64_t C, int64_t w_top_k, int64_t r_top_k, int mass_aware, float eps,
                                void *workspace, int64_t workspace_bytes, void *stream) {
    return segment_from_decoded(addr_idx, addr_val, x, gamma, dtype, mask, init_slot, init_mass, slot_out, mass_out, y,
                                B, H, T, A, C, w_top_k, r_top_k, mass_aware, eps, workspace, workspace_bytes, stream,
                                "topk_segment_forward launch");
}

int ramnet_topk_segment_forward_(const int32_t *addr_idx, const float *addr_val, const void *x, const void *gamma,
                                 int dtype, const uint8_t *mask, float *slot, float *mass, const float *mass_in,
                                 void *y, int64_t B, int64_t H, int64_t T, int64_t A, int64_t C, int64_t w_top_k,
                                 int64_t r_top_k, int mass_aware, float eps, void *workspace, int64_t workspace_bytes,
                                 void *stream) {
    return segment_from_decoded(addr_idx, addr_val, x, gamma, dtype, mask, slot, mass_in, slot, mass, y, B, H, T, A,
                                C, w_top_k, r_top_k, mass_aware, eps, workspace, workspace_bytes, stream,
                                "topk_segment_forward_ launch");
}

// Bodies of the record decoder, the scan and the fused forward; `need` is
// the workspace the calling entry point requires (-1: the scan workspace).
static int addr_records(const void *w_addr, const void *r_addr, const void *gamma, int dtype, const uint8_t *mask,
                        int64_t embed_num, const int32_t *position_ids, int64_t B, int64_t H, int64_t U, int64_t P,
                        int64_t T, int64_t A, int64_t w_top_k, int64_t r_top_k, float w_re_norm, float r_re_norm,
                        void *workspace, int64_t workspace_bytes, int64_t need, void *stream) {
    if (int rc = check_addr_shape(B, H, U, P, T, embed_num, A))
        return rc;
    RAMNET_REQUIRE(valid_dtype(dtype), "addr dtype must be float32, float16 or bfloat16");
    RAMNET_REQUIRE(w_top_k > 0 && w_top_k <= A && r_top_k > 0 && r_top_k <= A, "top_k values must be in [1, A]");
    RAMNET_REQUIRE(w_re_norm >= 0.f && w_re_norm <= 1.f && r_re_norm >= 0.f && r_re_norm <= 1.f,
                   "top_k_re_norm exponents must be in [0, 1]");
    RAMNET_REQUIRE(fits_int({B * H * U * P * T, B * H * (T + ramnet::kScanPad) * (w_top_k + r_top_k)}),
                   "CUDA index overflow: sizes exceed int32");
    if (need < 0)
        need = scan_workspace_bytes(B, H, T, w_top_k, r_top_k);
    RAMNET_REQUIRE(workspace_bytes >= need && workspace, "workspace too small: see ramnet_scan_workspace_bytes");
    if (B * T == 0)
        return RAMNET_OK;
    RAMNET_REQUIRE(w_addr && r_addr && gamma && position_ids, "null tensor pointer");
    ramnet::SegmentJob lay = make_segment_job(nullptr, dtype, nullptr, nullptr, nullptr, nullptr, nullptr, B, H, T,
                                              A, 1, w_top_k, r_top_k, 0, 1.f, workspace);
    ramnet::AddrJob dec{};
    dec.src[0] = {w_addr, static_cast<int>(w_top_k), w_re_norm, 1.f, 0};
    dec.src[1] = {r_addr, static_cast<int>(r_top_k), r_re_norm, 1.f, 0};
    dec.n_src = 2;
    dec.dtype = dtype;
    dec.B = static_cast<int>(B);
    dec.H = static_cast<int>(H);
    dec.U = static_cast<int>(U);
    dec.P = static_cast<int>(P);
    dec.T = static_cast<int>(T);
    dec.A = static_cast<int>(A);
    dec.embed_num = static_cast<int>(embed_num);
    dec.encode_batch_idx = 1;
    dec.k_total = static_cast<int>(w_top_k + r_top_k);
    dec.position_ids = position_ids;
    dec.wrec = const_cast<ramnet::WriteRec *>(lay.wrec);
    dec.rrec = const_cast<ramnet::ReadRec *>(lay.rrec);
    dec.gamma = gamma;
    dec.mask = mask;
    const char *why = nullptr;
    const hipError_t err = ramnet::launch_topk_addr(dec, static_cast<hipStream_t>(stream), &why);
    return finish(err, why, "topk_addr_records launch");
}

static int segment_scan(const void *x, int dtype, const float *init_slot, const float *init_mass, float *slot_out,
                        float *mass_out, void *y, int64_t B, int64_t H, int64_t T, int64_t A, int64_t C,
                        int64_t w_top_k, int64_t r_top_k, int mass_aware, float eps, void *workspace,
                        int64_t workspace_bytes, int64_t need, void *stream) {
    if (int rc = segment_checks(x, x, dtype, init_slot, init_mass, slot_out, mass_out, y, B, H, T, A, C, w_top_k,
                                r_top_k, eps, workspace, workspace_bytes, need))
        return rc;
    if (B == 0)
        return RAMNET_OK;
    ramnet::SegmentJob job = make_segment_job(x, dtype, init_slot, init_mass, slot_out, mass_out, y, B, H, T, A, C,
                                              w_top_k, r_top_k, mass_aware, eps, workspace);
    const char *why = nullptr;
    const hipError_t err = ramnet::launch_segment_forward(job, static_cast<hipStream_t>(stream), &why);
    return finish(err, why, "segment_scan launch");
}

static int ram_attn_forward(const void *w_addr, const void *r_addr, const void *x, const void *gamma, int dtype,
                            const uint8_t *mask, int64_t embed_num, const int32_t *position_ids,
                            const float *init_slot, const float *init_mass, float *slot_out, float *mass_out, void *y,
                            int64_t B, int64_t H, int64_t U, int64_t P, int64_t T, int64_t A, int64_t C,
                            int64_t w_top_k, int64_t r_top_k, float w_re_norm, float r_re_norm, int mass_aware,
                            float eps, void *workspace, int64_t workspace_bytes, int64_t need, void *stream) {
    if (int rc = segment_checks(x, gamma, dtype, init_slot, init_mass, slot_out, mass_out, y, B, H, T, A, C, w_top_k,
                                r_top_k, eps, workspace, workspace_bytes, need))
        return rc;
    if (B > 0 && T > 0) {
        if (int rc = addr_records(w_addr, r_addr, gamma, dtype, mask, embed_num, position_ids, B, H, U, P, T, A,
                                  w_top_k, r_top_k, w_re_norm, r_re_norm, workspace, workspace_bytes, need, stream))
            return rc;
    }
    return segment_scan(x, dtype, init_slot, init_mass, slot_out, mass_out, y, B, H, T, A, C, w_top_k, r_top_k,
                        mass_aware, eps, workspace, workspace_bytes, need, stream);
}

int ramnet_topk_addr_records(const void *w_addr, const void *r_addr, const void *gamma, int dtype,
                             const uint8_t *mask, int64_t embed_num, const int32_t *position_ids, int64_t B, int64_t H,
                             int64_t U, int64_t P, int64_t T, int64_t A, int64_t w_top_k, int64_t r_top_k,
                             float w_re_norm, float r_re_norm, void *workspace, int64_t workspace_bytes,
                             void *stream) {
    return addr_records(w_addr, r_addr, gamma, dtype, mask, embed_num, position_ids, B, H, U, P, T, A, w_top_k,
                        r_top_k, w_re_norm, r_re_norm, workspace, workspace_bytes, -1, stream);
}

int ramnet_segment_scan(const void *x, int dtype, const float *init_slot, const float *init_mass, float *slot_out,
                        float *mass_out, void *y, int64_t B, int64_t H, int64_t T, int64_t A, int64_t C,
                        int64_t w_top_k, int64_t r_top_k, int mass_aware, float eps, void *workspace,
                        int64_t workspace_bytes, void *stream) {
    return segment_scan(x, dtype, init_slot, init_mass, slot_out, mass_out, y, B, H, T, A, C, w_top_k, r_top_k,
                        mass_aware, eps, workspace, workspace_bytes, -1, stream);
}

int ramnet_ram_attn_forward(const void *w_addr, const void *r_addr, const void *x, const void *gamma, int dtype,
                            const uint8_t *mask, int64_t embed_num, const int32_t *position_ids,
                            const float *init_slot, const float *init_mass, float *slot_out, float *mass_out, void *y,
                            int64_t B, int64_t H, int64_t U, int64_t P, int64_t T, int64_t A, int64_t C,
                            int64_t w_top_k, int64_t r_top_k, float w_re_norm, float r_re_norm, int mass_aware,
                            float eps, void *workspace, int64_t workspace_bytes, void *stream) {
    return ram_attn_forward(w_addr, r_addr, x, gamma, dtype, mask, embed_num, position_ids, init_slot, init_mass,
                            slot_out, mass_out, y, B, H, U, P, T, A, C, w_top_k, r_top_k, w_re_norm, r_re_norm,
                            mass_aware, eps, workspace, workspace_bytes, -1, stream);
}

static int64_t backward_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t A, int64_t C, int64_t Kw,
                                        int64_t Kr) {
    if (B < 0 || H <= 0 || T < 0 || A <= 0 || C <= 0 || Kw <= 0 || Kr <= 0 || A >= kAddressLimit ||
        !fits_int({B * H * A * C, B * H * (A + 2), B * H * T * C, B * H * (T + ramnet::kScanPad) * (Kw + Kr)}))
        return -1;
    const int64_t rec = (ramnet::scan_record_bytes(B, H, T, Kw, Kr) + 255) / 256 * 256;
    const int64_t extra = ramnet::segment_backward_layout(static_cast<int>(B), static_cast<int>(H), static_cast<int>(T),
                                                          static_cast<int>(A), static_cast<int>(C), static_cast<int>(Kw),
                                                          static_cast<int>(Kr), nullptr, nullptr);
    return extra < 0 ? -1 : rec + extra;
}

int64_t ramnet_segment_backward_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t A, int64_t C,
                                                int64_t w_top_k, int64_t r_top_k) {
    return backward_workspace_bytes(B, H, T, A, C, w_top_k, r_top_k);
}

int ramnet_topk_segment_backward(const int32_t *addr_idx, const float *addr_val, const void *x, const void *gamma,
                                 int dtype, const uint8_t *mask, const float *init_slot, const float *init_mass,
                                 const void *grad_y, const float *grad_slot, const float *grad_mass,
                                 float *grad_addr_val, float *grad_x, float *grad_gamma, float *grad_init_slot,
                                 float *grad_init_mass, int64_t B, int64_t H, int64_t T, int64_t A, int64_t C,
                                 int64_t w_top_k, int64_t r_top_k, int mass_aware, float eps, void *workspace,
                                 int64_t workspace_bytes, void *stream) {
    const int64_t need = backward_workspace_bytes(B, H, T, A, C, w_top_k, r_top_k);
    if (int rc = segment_checks(x, gamma, dtype, init_slot, init_mass, grad_init_slot, grad_init_mass, grad_x, B, H,
                                T, A, C, w_top_k, r_top_k, eps, workspace, workspace_bytes, need < 0 ? 0 : need))
        return rc;
    if (B == 0)
        return RAMNET_OK;
    RAMNET_REQUIRE(need >= 0, "segment backward: shape outside the LDS-resident scan (top_k <= 128 and a slot "
                              "slice in LDS: A <= 37870, or 34798 beyond 64 events)");
    RAMNET_REQUIRE(workspace_bytes >= need && workspace,
                   "workspace too small: see ramnet_segment_backward_workspace_bytes");
    RAMNET_REQUIRE(T == 0 || (addr_idx && addr_val && grad_y && grad_addr_val && grad_gamma), "null tensor pointer");
    ramnet::SegmentJob fj = make_segment_job(x, dtype, init_slot, init_mass, nullptr, nullptr, nullptr, B, H, T, A, C,
                                             w_top_k, r_top_k, mass_aware, eps, workspace);
    fj.gain = nullptr;  // the backward's own buffers follow the records
    fj.flags = nullptr;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const char *why = nullptr;
    if (T > 0) {
        const hipError_t err = pack_decoded(fj, addr_idx, addr_val, gamma, mask, s, &why);
        if (err != hipSuccess)
            return finish(err, why, "topk_segment_backward launch");
    }
    ramnet::SegmentBwdJob job{};
    job.fwd = fj;
    job.addr_val = addr_val;
    job.gamma = gamma;
    job.grad_y = grad_y;
    job.grad_slot = grad_slot;
    job.grad_mass = grad_mass;
    job.grad_val = grad_addr_val;
    job.grad_x = grad_x;
    job.grad_gamma = grad_gamma;
    job.grad_init_slot = grad_init_slot;
    job.grad_init_mass = grad_init_mass;
    const int64_t rec = (ramnet::scan_record_bytes(B, H, T, w_top_k, r_top_k) + 255) / 256 * 256;
    ramnet::segment_backward_layout(static_cast<int>(B), static_cast<int>(H), static_cast<int>(T), static_cast<int>(A),
                                    static_cast<int>(C), static_cast<int>(w_top_k), static_cast<int>(r_top_k),
                                    static_cast<char *>(workspace) + rec, &job);
    const hipError_t err = ramnet::launch_segment_backward(job, s, &why);
    return finish(err, why, "topk_segment_backward launch");
}

// ---- training pair with saved rows. The saved buffer holds the scan
// records, the backward's per-event records (MassAux: where its
// record-keeping pre-pass holds the slot space in one piece), then x - s of
// every write row and every read row in the backward's channel slices
// (SavedRows), each part 256-byte aligned.
struct SavedParts {
    int64_t rec, aux_w, aux_r, rows;
    int64_t total() const { return rec + aux_w + aux_r + 2 * rows; }
};
static bool saved_layout(int64_t B, int64_t H, int64_t T, int64_t A, int64_t C, int64_t Kw, int64_t Kr, int dtype,
                         ramnet::SavedRows *geo, SavedParts *parts) {
    if (B <= 0 || H <= 0 || T <= 0 || A <= 0 || A >= kAddressLimit || C <= 0 || Kw <= 0 || Kr <= 0 || Kw > A ||
        Kr > A || !valid_dtype(dtype) ||
        !fits_int({B * H * A * C, B * H * (A + 2), B * H * T * C, B * H * (T + ramnet::kScanPad) * (Kw + Kr)}))
        return false;
    if (backward_workspace_bytes(B, H, T, A, C, Kw, Kr) < 0 ||
        !ramnet::segment_saved_slices(static_cast<int>(A), static_cast<int>(C), static_cast<int>(Kw),
                                      static_cast<int>(Kr), geo) ||
        !ramnet::segment_forward_can_save(static_cast<int>(B), static_cast<int>(H), static_cast<int>(T),
                                          static_cast<int>(A), static_cast<int>(C), static_cast<int>(Kw),
                                          static_cast<int>(Kr), dtype, *geo))
        return false;
    auto al = [](int64_t n) { return (n + 255) / 256 * 256; };
    const bool aux = ramnet::segment_saved_aux(static_cast<int>(A));
    parts->rec = al(ramnet::scan_record_bytes(B, H, T, Kw, Kr));
    parts->aux_w = aux ? al(B * H * T * Kw * 16) : 0;
    parts->aux_r = aux ? al(B * H * T * Kr * 16) : 0;
    parts->rows = al(B * H * geo->n_sub * ramnet::scan_t_pad64(T) * geo->kp * geo->csw * 4);
    return true;
}

// The parts of a saved buffer at `base`.
static void saved_pointers(char *base, const SavedParts &parts, ramnet::SavedRows *geo) {
    char *aw = base + parts.rec, *ar = aw + parts.aux_w, *rw = ar + parts.aux_r;
    geo->aux = parts.aux_w ? ramnet::MassAux{reinterpret_cast<int4 *>(aw), reinterpret_cast<int4 *>(ar)}
                           : ramnet::MassAux{};
    geo->w = reinterpret_cast<float *>(rw);
    geo->r = reinterpret_cast<float *>(rw + parts.rows);
}

int64_t ramnet_segment_saved_bytes(int64_t B, int64_t H, int64_t T, int64_t A, int64_t C, int64_t w_top_k,
                                   int64_t r_top_k, int dtype) {
    ramnet::SavedRows geo{};
    SavedParts parts{};
    return saved_layout(B, H, T, A, C, w_top_k, r_top_k, dtype, &geo, &parts) ? parts.total() : -1;
}

int ramnet_topk_segment_forward_save(const int32_t *addr_idx, const float *addr_val, const void *x,
                                     const void *gamma, int dtype, const uint8_t *mask, const float *init_slot,
                                     const float *init_mass, float *slot_out, float *mass_out, void *y, int64_t B,
                                     int64_t H, int64_t T, int64_t A, int64_t C, int64_t w_top_k, int64_t r_top_k,
                                     int mass_aware, float eps, void *workspace, int64_t workspace_bytes, void *saved,
                                     int64_t saved_bytes, void *stream) {
    if (int rc = segment_checks(x, gamma, dtype, init_slot, init_mass, slot_out, mass_out, y, B, H, T, A, C, w_top_k,
                                r_top_k, eps, workspace, workspace_bytes))
        return rc;
    ramnet::SavedRows geo{};
    SavedParts parts{};
    RAMNET_REQUIRE(saved_layout(B, H, T, A, C, w_top_k, r_top_k, dtype, &geo, &parts),
                   "topk_segment_forward_save: no saved-row form for this shape (ramnet_segment_saved_bytes < 0)");
    RAMNET_REQUIRE(saved && saved_bytes >= parts.total(), "saved buffer too small: see ramnet_segment_saved_bytes");
    RAMNET_REQUIRE(addr_idx && addr_val, "null tensor pointer");
    ramnet::SegmentJob job = make_segment_job(x, dtype, init_slot, init_mass, slot_out, mass_out, y, B, H, T, A, C,
                                              w_top_k, r_top_k, mass_aware, eps, workspace);
    char *sv = static_cast<char *>(saved);
    job.wrec = reinterpret_cast<const ramnet::WriteRec *>(sv);
    job.rrec = reinterpret_cast<const ramnet::ReadRec *>(sv + B * H * ramnet::scan_t_pad64(T) * w_top_k *
                                                               static_cast<int64_t>(sizeof(ramnet::WriteRec)));
    saved_pointers(sv, parts, &geo);
    job.save = geo;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const char *why = nullptr;
    hipError_t err = pack_decoded(job, addr_idx, addr_val, gamma, mask, s, &why);
    if (err == hipSuccess)
        err = ramnet::launch_segment_forward(job, s, &why);
    return finish(err, why, "topk_segment_forward_save launch");
}

int64_t ramnet_segment_backward_saved_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t A, int64_t C,
                                                      int64_t w_top_k, int64_t r_top_k) {
    if (backward_workspace_bytes(B, H, T, A, C, w_top_k, r_top_k) < 0)
        return -1;
    return ramnet::segment_backward_layout(static_cast<int>(B), static_cast<int>(H), static_cast<int>(T),
                                           static_cast<int>(A), static_cast<int>(C), static_cast<int>(w_top_k),
                                           static_cast<int>(r_top_k), nullptr, nullptr, true);
}

int ramnet_topk_segment_backward_saved(const float *addr_val, const void *x, const void *gamma, int dtype,
                                       const float *init_slot, const float *init_mass, const void *grad_y,
                                       const float *grad_slot, const float *grad_mass, float *grad_addr_val,
                                       float *grad_x, float *grad_gamma, float *grad_init_slot, float *grad_init_mass,
                                       int64_t B, int64_t H, int64_t T, int64_t A, int64_t C, int64_t w_top_k,
                                       int64_t r_top_k, int mass_aware, float eps, const void *saved,
                                       int64_t saved_bytes, void *workspace, int64_t workspace_bytes, void *stream) {
    const int64_t need = ramnet_segment_backward_saved_workspace_bytes(B, H, T, A, C, w_top_k, r_top_k);
    if (int rc = segment_checks(x, gamma, dtype, init_slot, init_mass, grad_init_slot, grad_init_mass, grad_x, B, H,
                                T, A, C, w_top_k, r_top_k, eps, workspace, workspace_bytes, need < 0 ? 0 : need))
        return rc;
    ramnet::SavedRows geo{};
    SavedParts parts{};
    RAMNET_REQUIRE(need >= 0 && saved_layout(B, H, T, A, C, w_top_k, r_top_k, dtype, &geo, &parts),
                   "topk_segment_backward_saved: no saved-row form for this shape (ramnet_segment_saved_bytes < 0)");
    RAMNET_REQUIRE(saved && saved_bytes >= parts.total(), "saved buffer too small: see ramnet_segment_saved_bytes");
    RAMNET_REQUIRE(workspace_bytes >= need && workspace,
                   "workspace too small: see ramnet_segment_backward_saved_workspace_bytes");
    RAMNET_REQUIRE(addr_val && grad_y && grad_addr_val && grad_gamma, "null tensor pointer");
    // the records were packed into the saved buffer by the forward
    ramnet::SegmentJob fj = make_segment_job(x, dtype, init_slot, init_mass, nullptr, nullptr, nullptr, B, H, T, A, C,
                                             w_top_k, r_top_k, mass_aware, eps, const_cast<void *>(saved));
    fj.gain = nullptr;
    fj.flags = nullptr;
    ramnet::SegmentBwdJob job{};
    job.fwd = fj;
    job.addr_val = addr_val;
    job.gamma = gamma;
    job.grad_y = grad_y;
    job.grad_slot = grad_slot;
    job.grad_mass = grad_mass;
    job.grad_val = grad_addr_val;
    job.grad_x = grad_x;
    job.grad_gamma = grad_gamma;
    job.grad_init_slot = grad_init_slot;
    job.grad_init_mass = grad_init_mass;
    ramnet::segment_backward_layout(static_cast<int>(B), static_cast<int>(H), static_cast<int>(T), static_cast<int>(A),
                                    static_cast<int>(C), static_cast<int>(w_top_k), static_cast<int>(r_top_k),
                                    static_cast<char *>(workspace), &job, true);
    saved_pointers(static_cast<char *>(const_cast<void *>(saved)), parts, &geo);
    job.delta = geo.w;
    job.saved_r = geo.r;
    if (geo.aux.wev) {
        job.aux = geo.aux;
        job.aux_saved = 1;
    }
    const char *why = nullptr;
    const hipError_t err = ramnet::launch_segment_backward(job, static_cast<hipStream_t>(stream), &why);
    return finish(err, why, "topk_segment_backward_saved launch");
}

// Checks and job of one decode step (S = 1) or S steps of one shape.
static int decode_job(const void *w_addr, const void *r_addr, const void *x, const void *gamma, int dtype,
                      float *slot, float *mass, const uint8_t *mask, int64_t embed_num, const int32_t *position_ids,
                      int64_t S, int64_t B, int64_t H, int64_t U, int64_t P, int64_t A, int64_t C, int64_t w_top_k,
                      int64_t r_top_k, float w_re_norm, float r_re_norm, int mass_aware, float eps, void *y,
                      ramnet::DecodeJob &job) {
    if (int rc = check_addr_shape(B, H, U, P, 1, embed_num, A))
        return rc;
    RAMNET_REQUIRE(S >= 0, "the step count must be >= 0");
    RAMNET_REQUIRE(C > 0, "C must be > 0");
    RAMNET_REQUIRE(valid_dtype(dtype), "x dtype must be float32, float16 or bfloat16");
    RAMNET_REQUIRE(w_top_k > 0 && w_top_k <= A && r_top_k > 0 && r_top_k <= A, "top_k values must be in [1, A]");
    RAMNET_REQUIRE(w_re_norm >= 0.f && w_re_norm <= 1.f && r_re_norm >= 0.f && r_re_norm <= 1.f,
                   "top_k_re_norm exponents must be in [0, 1]");
    RAMNET_REQUIRE(eps > 0.f, "eps must be > 0");
    RAMNET_REQUIRE(fits_int({B * H * U * P, B * H * A * C, B * H * A, B * H * C, S}),
                   "CUDA index overflow: sizes exceed int32");
    job = ramnet::DecodeJob{};
    job.w_addr = w_addr;
    job.r_addr = r_addr;
    job.x = x;
    job.gamma = gamma;
    job.mask = mask;
    job.position_ids = position_ids;
    job.slot = slot;
    job.mass = mass;
    job.y = y;
    job.dtype = dtype;
    job.B = static_cast<int>(B);
    job.H = static_cast<int>(H);
    job.U = static_cast<int>(U);
    job.P = static_cast<int>(P);
    job.A = static_cast<int>(A);
    job.C = static_cast<int>(C);
    job.Kw = static_cast<int>(w_top_k);
    job.Kr = static_cast<int>(r_top_k);
    job.embed_num = static_cast<int>(embed_num);
    job.w_re_norm = w_re_norm;
    job.r_re_norm = r_re_norm;
    job.mass_aware = mass_aware ? 1 : 0;
    job.eps = eps;
    return RAMNET_OK;
}

int ramnet_topk_autoregressive_(const void *w_addr, const void *r_addr, const void *x, const void *gamma, int dtype,
                                float *slot, float *mass, const uint8_t *mask, int64_t embed_num,
                                const int32_t *position_ids, int64_t B, int64_t H, int64_t U, int64_t P, int64_t A,
                                int64_t C, int64_t w_top_k, int64_t r_top_k, float w_re_norm, float r_re_norm,
                                int mass_aware, float eps, void *y, void *stream) {
    ramnet::DecodeJob job;
    if (int rc = decode_job(w_addr, r_addr, x, gamma, dtype, slot, mass, mask, embed_num, position_ids, 1, B, H, U, P,
                            A, C, w_top_k, r_top_k, w_re_norm, r_re_norm, mass_aware, eps, y, job))
        return rc;
    if (B == 0)
        return RAMNET_OK;
    RAMNET_REQUIRE(w_addr && r_addr && x && gamma && slot && mass && position_ids && y, "null tensor pointer");
    const char *why = nullptr;
    const hipError_t err = ramnet::launch_autoregressive(job, static_cast<hipStream_t>(stream), &why);
    return finish(err, why, "topk_autoregressive_ launch");
}

int ramnet_topk_autoregressive_steps_(const void *w_addr, const void *r_addr, const void *x, const void *gamma,
                                      int dtype, float *slot, float *mass, const uint8_t *mask, int64_t embed_num,
                                      const int32_t *position_ids, int64_t S, int64_t B, int64_t H, int64_t U,
                                      int64_t P, int64_t A, int64_t C, int64_t w_top_k, int64_t r_top_k,
                                      float w_re_norm, float r_re_norm, int mass_aware, float eps, void *y,
                                      void *stream) {
    ramnet::DecodeJob job;
    if (int rc = decode_job(w_addr, r_addr, x, gamma, dtype, slot, mass, mask, embed_num, position_ids, S, B, H, U, P,
                            A, C, w_top_k, r_top_k, w_re_norm, r_re_norm, mass_aware, eps, y, job))
        return rc;
    if (B == 0 || S == 0)
        return RAMNET_OK;
    RAMNET_REQUIRE(w_addr && r_addr && x && gamma && slot && mass && position_ids && y, "null tensor pointer");
    const char *why = nullptr;
    const hipError_t err =
        ramnet::launch_autoregressive_steps(job, static_cast<int>(S), static_cast<hipStream_t>(stream), &why);
    return finish(err, why, "topk_autoregressive_steps_ launch");
}

// The query has no token count: it answers for a call of kPlanQueryTokens
// tokens (the form can differ for much shorter calls, where the mass-wave
// form's saving of the pre-pass launches decides).
constexpr int kPlanQueryTokens = 4096;

int ramnet_segment_plan(int64_t B, int64_t H, int64_t A, int64_t C, int64_t w_top_k, int64_t r_top_k, int dtype,
                        int *slice_channels, int *lds_bytes, int *precomputed_gains) {
    if (B <= 0 || H <= 0 || A <= 0 || A >= kAddressLimit || C <= 0 || w_top_k <= 0 || r_top_k <= 0 ||
        !valid_dtype(dtype) || !fits_int({B * H * A * C, B * H * (A + 2)}))
        return 0;
    return ramnet::segment_plan(static_cast<int>(B), static_cast<int>(H), kPlanQueryTokens, static_cast<int>(A),
                                static_cast<int>(C), static_cast<int>(w_top_k), static_cast<int>(r_top_k), dtype,
                                slice_channels, lds_bytes, precomputed_gains);
}

// ---- prefill forward without a workspace argument
//
// The per-event records (and the gain records of the precomputed-gain form)
// live in `scratch`, one copy per GPU, held by the loaded code object until
// the process ends. Host code never passes the array's name to a kernel (on
// the host it is only a stand-in): each device's address comes from
// hipGetSymbolAddress, looked up once per device with that device current.
// Nothing in it needs to start at zero: the record decoder writes every
// record the scan reads. Calls on one GPU share that GPU's copy.
static __device__ __align__(256) unsigned char scratch[RAMNET_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kScratchDevices = 64;
std::atomic<void *> g_scratch[kScratchDevices];
std::mutex g_scratch_mu;

int scratch_address(void **out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess)
        return fail(RAMNET_ELAUNCH, std::string("ram_attn_forward_noalloc: hipGetDevice: ") + hipGetErrorString(e));
    RAMNET_REQUIRE(dev >= 0 && dev < kScratchDevices, "ram_attn_forward_noalloc: device ordinal beyond 63");
    void *p = g_scratch[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch[dev].load(std::memory_order_relaxed);
        if (!p) {
            e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess || !p)
                return fail(RAMNET_ELAUNCH, std::string("ram_attn_forward_noalloc: hipGetSymbolAddress(scratch): ") +
                                                hipGetErrorString(e));
            g_scratch[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return RAMNET_OK;
}
}  // namespace

int ramnet_ram_attn_forward_noalloc(const void *w_addr, const void *r_addr, const void *x, const void *gamma,
                                    int dtype, const uint8_t *mask, int64_t embed_num, const int32_t *position_ids,
                                    const float *init_slot, const float *init_mass, float *slot_out, float *mass_out,
                                    void *y, int64_t B, int64_t H, int64_t U, int64_t P, int64_t T, int64_t A,
                                    int64_t C, int64_t w_top_k, int64_t r_top_k, float w_re_norm, float r_re_norm,
                                    int mass_aware, float eps, void *stream) {
    void *ws = nullptr;
    int64_t need = 0;
    // sizes the scan's own checks accept (anything else fails there first)
    const bool plausible = B > 0 && H > 0 && T >= 0 && C > 0 && A > 0 && A < kAddressLimit && w_top_k > 0 &&
                           r_top_k > 0 && w_top_k <= A && r_top_k <= A && valid_dtype(dtype) &&
                           fits_int({B * H * A * C, B * H * (A + 2), B * H * T * C,
                                     B * H * (T + ramnet::kScanPad) * (w_top_k + r_top_k)});
    if (plausible) {
        int pre = 0;
        RAMNET_REQUIRE(ramnet::segment_plan(static_cast<int>(B), static_cast<int>(H), static_cast<int>(T),
                                            static_cast<int>(A), static_cast<int>(C), static_cast<int>(w_top_k),
                                            static_cast<int>(r_top_k), dtype, nullptr, nullptr, &pre),
                       "ram_attn_forward_noalloc: shape outside the LDS-resident scan (top_k <= 128)");
        // the decoder records; the precomputed-gain form adds the gain
        // records and, in slot ranges with 16-bit y, the fp32 read sums
        need = pre ? segment_workspace_bytes(B, H, T, A, C, w_top_k, r_top_k, dtype)
                   : ramnet::scan_record_bytes(B, H, T, w_top_k, r_top_k);
        if (need > RAMNET_NOALLOC_SCRATCH_BYTES)
            return fail(RAMNET_EINVAL, "ram_attn_forward_noalloc: this shape needs " + std::to_string(need) +
                                           " bytes of records, more than the " +
                                           std::to_string(static_cast<long long>(RAMNET_NOALLOC_SCRATCH_BYTES)) +
                                           "-byte scratch; use ramnet_ram_attn_forward with a workspace");
        // T == 0 reads no records, but the launch still takes the scratch as
        // its workspace (the precomputed-gain form refuses a null one)
        if (int rc = scratch_address(&ws))
            return rc;
    }
    return ram_attn_forward(w_addr, r_addr, x, gamma, dtype, mask, embed_num, position_ids, init_slot, init_mass,
                            slot_out, mass_out, y, B, H, U, P, T, A, C, w_top_k, r_top_k, w_re_norm, r_re_norm,
                            mass_aware, eps, ws, RAMNET_NOALLOC_SCRATCH_BYTES, need, stream);
}

}  // extern "C"
