// arfq_internal.h -- host-side structures and the launchers each kernel file
// exports to the host library (arfq_host.hip).  Not part of the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stddef.h>
#include <stdint.h>
#include <atomic>
#include <string>

#include "../../include/arfq.h"

struct arfq_ctx {
    int device = 0;
    int cus = 0;  // compute units of the device
    hipStream_t stream = nullptr;
    bool own_stream = false;
    std::string err;
    hipEvent_t ev_start = nullptr, ev_stop = nullptr;
    unsigned options = 0;  // ARFQ_OPT_* bits
    // growable scratch for the GEMM plans, the MoE pipeline and the FFN
    // (stream-ordered allocations: grown without waiting for the stream)
    void *scratch = nullptr;
    size_t scratch_bytes = 0;
    // staging of host uploads, reused across calls (at most UPLOAD_CHUNK bytes)
    void *staging = nullptr;
    size_t staging_bytes = 0;
    // device address of the allocation-free matmul's fixed scratch on this device
    void *noalloc_scratch = nullptr;
    // device words: arfq_stream_read's sink (STREAM_SINK_WORDS), then the
    // upload's flag words (UPLOAD_FLAG_WORDS)
    uint32_t *aux = nullptr;
};

struct arfq_weight {
    arfq_ctx *ctx = nullptr;
    int qtype = 0;
    int64_t n = 0, k = 0;
    int experts = 1;
    int64_t nblk = 0;  // blocks over all experts
    // device streams (see arfq_common.h for what each holds per qtype)
    void *s0 = nullptr;  // Q4_K hdr | Q8_0 qs | Q6_K qb | Q5_K hdr     | IQ4_XS hdr
    void *s1 = nullptr;  // Q4_K qs  | Q8_0 d  | Q6_K sc | Q5_K qh + qs | IQ4_XS qs
    void *s2 = nullptr;  //                      Q6_K d
    size_t bytes = 0;    // ggml bytes of one expert (what one matmul streams)
    bool wide = false;   // Q6_K: some sub-block scale outside [-64, 64] (set by the upload)
    bool over62 = false; // Q6_K: some sub-block scale outside [-62, 62] (set by the upload)
};

namespace arfq {

// words of arfq_ctx::aux that arfq_stream_read's kernel may store to (one per
// thread of a 256-thread workgroup)
constexpr int STREAM_SINK_WORDS = 256;
// words past the sink: the upload's flag (a Q6_K scale outside [-64, 64] seen by the repack)
constexpr int UPLOAD_FLAG_WORDS = 64;
// host uploads go through the context's staging buffer in pieces of at most this many bytes
constexpr size_t UPLOAD_CHUNK = (size_t)64 << 20;

// hipFuncSetAttribute(MaxDynamicSharedMemorySize) for `fn` on the current
// device, once per device: `done` (one per kernel, zero-initialised static)
// holds a bit per device index already set.
inline hipError_t set_max_lds_once(const void *fn, size_t bytes, std::atomic<uint64_t> &done) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const uint64_t bit = dev < 64 ? (uint64_t)1 << dev : 0;
    if (bit && (done.load(std::memory_order_acquire) & bit)) return hipSuccess;
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e == hipSuccess && bit) done.fetch_or(bit, std::memory_order_release);
    return e;
}

// block geometry
inline int qk_of(int qtype) { return qtype == ARFQ_Q8_0 ? 32 : 256; }
inline int block_bytes_of(int qtype) {
    return qtype == ARFQ_Q8_0 ? 34 : qtype == ARFQ_Q4_K ? 144 : qtype == ARFQ_Q6_K ? 210
         : qtype == ARFQ_Q5_K ? 176 : qtype == ARFQ_IQ4_XS ? 136 : 0;
}

// ---- arfq_dequant.hip ----
// Split raw ggml blocks (device) into the layout streams of `w`: blocks
// [b0, b0 + nb) of w (nb < 0: to the end), raw pointing at block b0's bytes.
// Q6_K: a repack that meets a sub-block scale outside [-64, 64] stores 1 to
// wide[0], one outside [-62, 62] stores 1 to wide[1] (when wide is not null).
hipError_t launch_repack(const arfq_weight *w, const uint8_t *raw, hipStream_t s, int64_t b0 = 0,
                         int64_t nb = -1, uint32_t *wide = nullptr);
// Dequantize all blocks of `w` to f32.
hipError_t launch_dequant(const arfq_weight *w, float *out, hipStream_t s);

// ---- arfq_gemv.hip ----
// Small-m GEMV for expert `e`: y[m, n] = x[m, k] . W_e^T, x f32.  Returns
// hipErrorInvalidValue when (qtype, m) has no GEMV kernel.
// x16: m = 1 takes the 16-bit fixed-point x kernel instead of f32 arithmetic
// (ARFQ_OPT_GEMV_X16).
hipError_t launch_gemv(const arfq_weight *w, int e, int64_t m, const float *x, float *y,
                       hipStream_t s, bool x16 = false);
bool gemv_supports(const arfq_weight *w, int64_t m, bool x16 = false);
// MoE decode GEMVs over P (token, expert) pairs, Q4_K: y[p] (w->n floats) = W_ids[p] .
// x_p, where x_p is row p / x_div of x (f32 or f16, [*, w->k]) or, when g is
// set, silu(g[p]) * u[p] (g, u: [P, w->k] f32).  Pairs with an out-of-range id
// are skipped.
// The FFN's down projection: y[m, n] = W . (act(g) * u), g and u [m, w->k] f32
// (Q4_K, m <= 4); act ARFQ_ACT_SILU or ARFQ_ACT_GELU_TANH.
bool gemv_glu_supports(const arfq_weight *w, int64_t m, bool x16 = false);
hipError_t launch_gemv_glu(const arfq_weight *w, int64_t m, const float *g, const float *u, float *y, int act,
                           hipStream_t s, bool x16 = false);
// The FFN's gate and up projections of one x row in one launch: ya = A . x,
// yb = B . x (Q4_K, same shape, f32 arithmetic).
bool gemv_dual_supports(const arfq_weight *a, const arfq_weight *b, int64_t m);
hipError_t launch_gemv_dual(const arfq_weight *a, const arfq_weight *b, const float *x, float *ya, float *yb,
                            hipStream_t s);
// h = act(g) * u elementwise (n floats; act ARFQ_ACT_*)
hipError_t launch_glu(const float *g, const float *u, float *h, int64_t n, int act, hipStream_t s);
bool gemv_pairs_supports(const arfq_weight *w);
hipError_t launch_gemv_pairs(const arfq_weight *w, int64_t P, const int32_t *ids, const void *x,
                             int x_dtype, int x_div, const float *g, const float *u, float *y,
                             hipStream_t s);
// MoE decode gate and up in one launch (same qtype, shape and expert count).
bool gemv_pairs_dual_supports(const arfq_weight *w0, const arfq_weight *w1);
hipError_t launch_gemv_pairs_dual(const arfq_weight *w0, const arfq_weight *w1, int64_t P, const int32_t *ids,
                                  const void *x, int x_dtype, int x_div, float *y0, float *y1, hipStream_t s);

// ---- arfq_gemm.hip ----
// Launch shape and scratch layout of the dequant-into-LDS MFMA GEMM.
struct GemmPlan {
    int bm = 128;          // x rows per workgroup tile (64 or 128)
    int splits = 1;        // split-K factor (partials [splits][m][n] then a reduce)
    bool xsplit = false;   // x as f16 hi + lo (an f32 x split in two)
    bool convert = false;  // x arrives as f32 and is converted into scratch
    bool sums = false;     // the format needs x sub-block sums (Q4_K)
    bool skinny = false;   // m <= 64: the weight-streaming kernel (arfq_skinny.h)
    bool bd = false;       // Q4_K prefill: weights straight into MFMA operands (arfq_gemm_bd.h)
    // skinny and bd, f32 x: the f16 parts x enters as (1: x rounded to f16 (f16
    // x, or ARFQ_OPT_GEMV_X16); 2: hi + lo, ~22 bits, skinny m = 9..64 and the bd
    // prefill; 3: hi + mid + lo, skinny m <= 8, which represents every f32 x
    // within 2^15 of its row's max exactly), stored as row blocks [parts][m][k]
    int parts = 1;
    bool fx = false;       // skinny, parts 3: the kernel splits the f32 x (and sums its parts) itself
    int bd_full = 0;       // bd: whole tiles; the rest are split into bd_chunks K ranges
    int bd_chunks = 1;
    size_t off_xh = 0, off_xl = 0, off_xs = 0, off_rs = 0, off_part = 0, scratch_bytes = 0;
};
// x16: ARFQ_OPT_GEMV_X16 is set (the skinny and prefill kernels take an f32 x as one f16 part)
GemmPlan gemm_plan(const arfq_weight *w, int64_t m, int x_dtype, bool x16 = false);
bool gemm_supports(const arfq_weight *w, int64_t m);
// y[m, n] = x[m, k] . W_e^T; `scratch` holds plan.scratch_bytes.
hipError_t launch_gemm(const arfq_weight *w, int e, int64_t m, const void *x, int x_dtype,
                       float *y, void *scratch,
                       const GemmPlan &p, hipStream_t s);
// Activation preparation: x (f32 or f16, [m, k]) -> f16 copy (xh), f16
// remainder (xl), bf16 sub-block sums (xs, [m][k / 256][16]); null outputs are
// skipped.  With rs (f32 x only) each row is stored divided by a power of two
// rs[row] that puts its max |x| in [2^14, 2^15); products of it must be
// multiplied back by rs[row].
// With parts = 2 or 3 (xl == xh + m * k) the lo rows (parts 2: x - hi; parts
// 3: the mid rows, then the lo rows x - hi - mid) follow the hi rows, and xs
// holds each part's row sums in the same row order.
// rs_splits: with rs, one scale per row and per K range of the skinny
// kernel's split-K (rs[split * m + row]; 1: one per row)
hipError_t launch_xprep(const void *x, int x_dtype, int64_t m, int64_t k, _Float16 *xh,
                        _Float16 *xl, uint16_t *xs, float *rs, hipStream_t s, int parts = 1,
                        int rs_splits = 1);

// ---- arfq_moe.hip ----
// Routing: ids/weights [tokens, top_k] from logits [tokens, E] (E <= 1024, top_k <= 64).
// With xs, the same launch also writes the bf16 sub-block sums of the f16 x
// [tokens, k] (what launch_xprep writes for an f16 x and xs alone).
hipError_t launch_moe_route(const float *logits, int64_t tokens, int E, int top_k, int norm,
                            int32_t *ids, float *wts, hipStream_t s, const _Float16 *x = nullptr,
                            int64_t k = 0, uint16_t *xs = nullptr);
// Grouping of P = tokens * top_k pairs by expert (E <= MOE_MAX_EXPERTS): off[E + 1],
// sorted[P] (pair indices), tiles[moe_max_tiles] (int2 expert, first row), *ntiles.
hipError_t launch_moe_group(const int32_t *ids, int64_t P, int E, int32_t *off, int32_t *sorted,
                            void *tiles, int32_t *ntiles, hipStream_t s);
int64_t moe_max_tiles(int64_t P, int E);
// h[P, inter] (f32, sorted order) = silu(x . gate^T) * (x . up^T) per pair;
// xs: x sub-block sums (Q4_K weights only, else null).
// xrs: row scales of a prepared f32 x (null for f16 x); g and u are multiplied
// back by the token's scale before the SwiGLU.
hipError_t launch_moe_gateup(const arfq_weight *gate, const arfq_weight *up, const _Float16 *x,
                             const uint16_t *xs, const float *xrs, int top_k, const int32_t *off,
                             const int32_t *sorted, const void *tiles, const int32_t *ntiles,
                             int64_t max_tiles, float *h, hipStream_t s);
// h (f32) -> h16 = h / rs[row] (rs a power of two keeping h16 in f16 range)
// and, when hs is set, the bf16 sub-block sums of h16.
hipError_t launch_moe_hprep(const float *h, int64_t P, int inter, _Float16 *h16, uint16_t *hs,
                            float *rs, hipStream_t s);
// o[pair, hidden] (f32) = rs[row] * (h16[sorted row] . down^T).
hipError_t launch_moe_down(const arfq_weight *down, const _Float16 *h, const uint16_t *hs,
                           const float *rs, const int32_t *off,
                           const int32_t *sorted, const void *tiles, const int32_t *ntiles,
                           int64_t max_tiles, float *o, hipStream_t s);
// y[t] = sum_j w[t, j] * o[t * top_k + j] in slot order.
hipError_t launch_moe_combine(const float *o, const int32_t *ids, const float *wts, int64_t tokens,
                              int top_k, int E, int64_t hidden, float *y, bool accumulate, hipStream_t s);
constexpr int MOE_EXPERTS_MAX = 512;
constexpr int MOE_ROUTE_EXPERTS_MAX = 1024;
constexpr int MOE_TOPK_MAX = 64;
// at most this many (token, expert) pairs take the indirect-GEMV decode path
constexpr int64_t MOE_DECODE_PAIRS_MAX = 128;

}  // namespace arfq
