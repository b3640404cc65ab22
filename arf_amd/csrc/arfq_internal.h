// arfq_internal.h -- host-side structures and the launchers each kernel file
// exports to the host library (arfq_host.hip).  Not part of the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stddef.h>
#include <stdint.h>
#include <string>

#include "../../include/arfq.h"

struct arfq_ctx {
    int device = 0;
    int cus = 0;  // compute units of the device
    hipStream_t stream = nullptr;
    bool own_stream = false;
    std::string err;
    hipEvent_t ev_start = nullptr, ev_stop = nullptr;
    // growable scratch for the MoE pipeline (routing, grouping, intermediates)
    void *scratch = nullptr;
    size_t scratch_bytes = 0;
};

struct arfq_weight {
    arfq_ctx *ctx = nullptr;
    int qtype = 0;
    int64_t n = 0, k = 0;
    int experts = 1;
    int64_t nblk = 0;  // blocks over all experts
    // device streams (see arfq_common.h for what each holds per qtype)
    void *s0 = nullptr;  // Q4_K hdr | Q8_0 qs | Q6_K qb
    void *s1 = nullptr;  // Q4_K qs  | Q8_0 d  | Q6_K sc
    void *s2 = nullptr;  //                      Q6_K d
    size_t bytes = 0;    // ggml bytes of one expert (what one matmul streams)
};

namespace arfq {

// block geometry
inline int qk_of(int qtype) { return qtype == ARFQ_Q8_0 ? 32 : 256; }
inline int block_bytes_of(int qtype) {
    return qtype == ARFQ_Q8_0 ? 34 : qtype == ARFQ_Q4_K ? 144 : qtype == ARFQ_Q6_K ? 210 : 0;
}

// ---- arfq_dequant.hip ----
// Split raw ggml blocks (device) into the layout streams of `w`.
hipError_t launch_repack(const arfq_weight *w, const uint8_t *raw, hipStream_t s);
// Dequantize all blocks of `w` to f32.
hipError_t launch_dequant(const arfq_weight *w, float *out, hipStream_t s);

// ---- arfq_gemv.hip ----
// Small-m GEMV for expert `e`: y[m, n] = x[m, k] . W_e^T, x f32.  Returns
// hipErrorInvalidValue when (qtype, m) has no GEMV kernel.
hipError_t launch_gemv(const arfq_weight *w, int e, int64_t m, const float *x, float *y,
                       hipStream_t s);
bool gemv_supports(const arfq_weight *w, int64_t m);

// ---- arfq_gemm.hip ----
// Launch shape of the dequant-into-LDS MFMA GEMM.
struct GemmPlan {
    int bm = 128;         // x rows per workgroup tile (64 or 128)
    int splits = 1;       // split-K factor (partials [splits][m][n] then a reduce)
    bool xsplit = false;  // x given as f16 hi + lo (an f32 x split in two)
};
GemmPlan gemm_plan(const arfq_weight *w, int64_t m, bool xsplit);
bool gemm_supports(const arfq_weight *w, int64_t m);
// y[m, n] = x[m, k] . W_e^T with x = xh (+ xl when plan.xsplit), row-major f16.
// `partials` holds splits * m * n floats when plan.splits > 1.
hipError_t launch_gemm(const arfq_weight *w, int e, int64_t m, const _Float16 *xh,
                       const _Float16 *xl, float *y, float *partials, const GemmPlan &p,
                       hipStream_t s);
// x f32 -> f16 (round to nearest), and x f32 -> hi + lo f16 pair.
hipError_t launch_f32_to_f16(const float *x, __half *y, int64_t n, hipStream_t s);
hipError_t launch_split_f32(const float *x, __half *hi, __half *lo, int64_t n, hipStream_t s);

}  // namespace arfq
