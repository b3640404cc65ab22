/*
 * arfq.h -- C ABI of the MI355X (gfx950) GGUF quantized-matmul library.
 *
 * The library replaces the GPU side of Arf's quantized matmul path: the weight
 * upload for GGUF Q8_0 / Q4_K / Q6_K tensors, the matmul entry point that picks
 * a GEMV or a tiled GEMM by the activation row count, and the expert-grouped
 * MoE block.  Each declaration cites the reference interface it replaces
 * (paths relative to the joydle/Arf source tree).
 *
 * Conventions (shared by every entry point):
 *   - Every call returns an int status: ARFQ_OK (0) or a negative ARFQ_E_*
 *     code; arfq_last_error(ctx) holds a message for the last failure.  No C++
 *     exception crosses this boundary.  (The reference panics on shape
 *     mismatches, crates/arf-ml/src/matmul.rs:180-183,374-386; here the same
 *     checks return ARFQ_E_SHAPE.)
 *   - A weight matrix is [n rows = outputs, k cols = inputs], row-major, ggml
 *     blocks running along k; y[m, n] = sum_k x[m, k] * W[n, k]
 *     (crates/arf-ml/src/matmul.rs:84-99, crates/arf-core/src/model/gguf.rs:780-782).
 *   - x, y, ids and other activations are DEVICE pointers owned by the caller.
 *     Weights are owned by their arfq_weight handle.
 *   - Work is enqueued asynchronously on the context's HIP stream; one context
 *     is used by one thread at a time (the reference's single-owner model,
 *     crates/arf-gpu/src/gpu/metal/island.rs:968-971).
 *   - Accumulation is fp32.  Dequantized weights are bit-identical to the
 *     reference's CPU dequant (arfq_dequant_f32 is the hook that proves it).
 */
#ifndef ARFQ_H
#define ARFQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ARFQ_VERSION 100 /* 1.0.0 */

/* status codes */
#define ARFQ_OK 0
#define ARFQ_E_INVALID -1   /* null handle / pointer, unknown enum */
#define ARFQ_E_SHAPE -2     /* dimension or byte-count mismatch */
#define ARFQ_E_DEVICE -3    /* HIP runtime error */
#define ARFQ_E_NOMEM -4     /* device allocation failed */
#define ARFQ_E_UNSUPPORTED -5 /* valid request this build does not implement */
#define ARFQ_E_FORMAT -6    /* file is not a well-formed GGUF v3 */
#define ARFQ_E_IO -7        /* file cannot be opened or mapped */
#define ARFQ_E_NOT_FOUND -8 /* no tensor of that name */

/* ggml type ids, crates/arf-core/src/model/gguf.rs:36-90 (GgmlType). */
typedef enum {
    ARFQ_Q8_0 = 8,  /* 34 B per 32 weights: f16 d, 32 x i8 */
    ARFQ_Q4_K = 12, /* 144 B per 256 weights: f16 d, f16 dmin, 12 B 6-bit scales/mins, 128 B nibbles */
    ARFQ_Q5_K = 13, /* 176 B per 256 weights: Q4_K's d, dmin, scales, then qh[32] 5th bits, qs[128];
                       every m (decode GEMV at m <= 4), MoE experts, dequant */
    ARFQ_Q6_K = 14, /* 210 B per 256 weights: ql[128], qh[64], i8 scales[16], f16 d */
    ARFQ_IQ4_XS = 23 /* 136 B per 256 weights: f16 d, u16 scales_h, scales_l[4], qs[128] codebook
                        indices; every m (decode GEMV at m <= 4), MoE experts, dequant */
} arfq_qtype;

/* activation element type */
typedef enum { ARFQ_F32 = 0, ARFQ_F16 = 1 } arfq_dtype;

typedef struct arfq_ctx arfq_ctx;
typedef struct arfq_weight arfq_weight;

/* Library version (ARFQ_VERSION). */
int arfq_version(void);

/* Static text for a status code. */
const char *arfq_status_string(int status);

/* Create a context on HIP device `device`.  `stream` is a hipStream_t to enqueue
 * on, or NULL for a stream the context creates (default priority) and owns.
 * Replaces the reference's GpuContext/CommandPass pair as the owner of the
 * queue (crates/arf-gpu/src/gpu/context.rs:28-120, command.rs:169-243). */
int arfq_ctx_create(int device, void *stream, arfq_ctx **out);
int arfq_ctx_destroy(arfq_ctx *ctx);
/* The hipStream_t the context enqueues on. */
void *arfq_ctx_stream(arfq_ctx *ctx);
/* Message for the last failed call on this context ("" if none).  A NULL ctx
 * returns the message of the last failed arfq_ctx_create on this thread. */
const char *arfq_last_error(const arfq_ctx *ctx);
/* Block until all work enqueued on the context's stream has finished. */
int arfq_ctx_sync(arfq_ctx *ctx);

/* Context options (bit set; default 0).
 * ARFQ_OPT_GEMV_X16: the Q4_K, Q5_K, Q6_K and IQ4_XS decode GEMVs at m <= 4
 *   (Q6_K at m <= 2; arfq_matmul, arfq_ffn_act) round each 32-element block
 *   of f32 x to 16-bit fixed point (relative to the block's max |x|) and take
 *   exact integer dots; faster, max relative error ~1e-4 of the output's rms.
 *   Only where those kernels' LDS fits 64 KiB: longer x keeps the default
 *   path.  The skinny MFMA kernel and the prefill GEMM (below) then take an
 *   f32 x as one f16 part (11 bits) instead of two or three.
 *   By default every GEMV multiplies f32 x by the exact weights in f32,
 *   as the reference GEMVs do
 *   (crates/arf-gpu/src/shaders/metal/matmul_vec_q4ks_msl.metal:46-165,
 *   matmul_vec_q4ks_batch_msl.metal:104-288).
 * No counterpart in the reference (which has only the f32 form). */
#define ARFQ_OPT_GEMV_X16 1u
int arfq_ctx_set_options(arfq_ctx *ctx, unsigned options);

/* Upload `n_experts` stacked [n_rows, k_cols] matrices of raw ggml blocks from
 * HOST memory.  `nbytes` must equal n_experts * n_rows * k_cols / QK *
 * block_bytes (QK = 32 / 256; block_bytes = 34 / 144 / 210).  Experts are
 * concatenated in expert-major order, the PackedExperts layout
 * (crates/arf-gpu/src/gpu/types.rs:89-112).  The upload is a lossless repack
 * into 16-byte-aligned device streams.  Replaces the Q4KS/Q8_0 upload in
 * crates/arf-gpu/src/weights.rs:1140-1236 and crates/arf-gpu/src/gpu/flux/t5.rs:106-140
 * (which transcode first; here the GPU reads ggml's own bit layout).
 * Synchronous: returns after the data is on the device. */
int arfq_weight_upload(arfq_ctx *ctx, int qtype, const void *host_blocks, size_t nbytes,
                       int64_t n_rows, int64_t k_cols, int n_experts, arfq_weight **out);
/* Same, from raw ggml blocks already in DEVICE memory (e.g. a GGUF tensor
 * copied as-is); the source is only read, and may be freed after the call. */
int arfq_weight_upload_device(arfq_ctx *ctx, int qtype, const void *dev_blocks, size_t nbytes,
                              int64_t n_rows, int64_t k_cols, int n_experts, arfq_weight **out);
int arfq_weight_free(arfq_weight *w);
/* Shape and type of an uploaded weight; any out-pointer may be NULL.
 * `device_bytes` is the bytes one full matmul streams (GpuMatWeight::bytes_num,
 * crates/arf-gpu/src/gpu/types.rs:69-82). */
int arfq_weight_info(const arfq_weight *w, int *qtype, int64_t *n_rows, int64_t *k_cols,
                     int *n_experts, size_t *device_bytes);

/* y[m, n_rows] (f32) = x[m, k_cols] . W^T for expert `expert` of `w` (0 for a
 * plain matrix).  x is f32 or f16 per `x_dtype`.  The library picks the kernel
 * by (qtype, m): wave-per-rows GEMV for small m, dequant-into-LDS MFMA GEMM
 * otherwise.  Arithmetic, f32 x:
 *   - m = 1: f32 x times the exact weights in f32 (Q4_K, Q5_K, IQ4_XS and Q6_K
 *     while x fits the kernels' LDS: k up to about 37K for Q4_K and 38K for the
 *     others; longer x takes the m <= 8 path below).
 *   - m <= 4: Q6_K and Q8_0 GEMVs in f32.
 *   - m <= 8 (Q4_K / Q5_K / IQ4_XS from m = 2, Q6_K / Q8_0 from m = 5): the
 *     skinny MFMA kernel with x as three f16 parts (hi + mid + lo) of x scaled
 *     per row (and per K range) by a power of two that puts the row's max |x|
 *     in [2^14, 2^15), so every x within 2^15 of that max is represented
 *     exactly; exact codes, f32 sums, the output scaled back.
 *   - m = 9..64: the same with two parts (hi + lo, ~22 bits).
 *   - Above 64 rows: hi + lo of x scaled per row, in the prefill GEMM (twice
 *     the MFMAs of an f16 x).
 * f16 x enters as is.  The weights are exact at every m for Q4_K, Q5_K, Q6_K
 * and Q8_0 (Q6_K scales beyond +-64 and Q8_0's d * q as two f16 operands
 * above 64 rows), except in the tile loop that takes the shapes the direct
 * prefill kernel does not (Q8_0 with k not a multiple of 256, streams past
 * 2 GiB) and IQ4_XS above 64 rows at f32 x: there the dequant is rounded once
 * to f16.
 * Replaces add_matmul_m / add_matmul
 * (crates/arf-gpu/src/gpu/dispatch.rs:169-202, Q4KS arms :517-630) and the
 * island's gemv_q4ks / gemv_q4ks_batch / matmul_mm_q4ks selection
 * (crates/arf-gpu/src/gpu/metal/island.rs:4289-4333). */
int arfq_matmul(arfq_ctx *ctx, const arfq_weight *w, int expert, int64_t m, const void *x,
                int x_dtype, float *y);

/* Bytes of the fixed device scratch behind arfq_matmul_noalloc (one array per
 * GPU, resident from the library's load until the process ends). */
#define ARFQ_NOALLOC_SCRATCH_BYTES (32u << 20)

/* As arfq_matmul, but allocates nothing: no hipMalloc/hipFree or allocating
 * library call, on the first call or any other.  The GEMM paths take their
 * scratch (x preparation, split-K partials) from a fixed 32 MiB device array
 * per GPU instead of the context's growable buffer; a product that would need
 * more returns ARFQ_E_UNSUPPORTED (decode shapes, m <= 64 at k, n up to ~20K,
 * fit; the GEMVs need none).  Every call on a GPU shares that GPU's array:
 * calls that overlap on one GPU (two streams, two threads) race and must be
 * ordered by the caller.  No counterpart in the reference: for callers that
 * cannot allocate -- code under HIP graph capture, tight serving loops,
 * harnesses that forbid device allocation. */
int arfq_matmul_noalloc(arfq_ctx *ctx, const arfq_weight *w, int expert, int64_t m, const void *x,
                        int x_dtype, float *y);

/* Dequantize every expert of `w` into out[n_experts * n_rows * k_cols] (device,
 * f32) with the same device dequant code the matmuls use.  Bit-identical to
 * dequant_q8_0 / dequant_q4_k / dequant_q6_k
 * (crates/arf-core/src/model/gguf.rs:1633-1649,2004-2035,2092-2131) and to
 * Q4KSMatrix::to_f32 (crates/arf-ml/src/weight.rs:1110-1136). */
int arfq_dequant_f32(arfq_ctx *ctx, const arfq_weight *w, float *out);

/* Top-k routing for `tokens` rows of router logits [tokens, n_experts] (device
 * f32): full softmax, the top_k largest probabilities (ties -> lower index),
 * renormalised to sum 1 when norm_topk != 0.  Writes ids[tokens, top_k] (i32)
 * and weights[tokens, top_k] (f32), both device.  Replaces the moe_route(_b)
 * kernels (crates/arf-gpu/src/shaders/metal/moe_route_msl.metal:18-98,
 * moe_batch_msl.metal:371-449); oracle top_k_softmax
 * (crates/arf-core/src/model/moe.rs:89-121). */
int arfq_moe_route(arfq_ctx *ctx, const float *logits, int64_t tokens, int n_experts, int top_k,
                   int norm_topk, int32_t *ids, float *weights);

/* The MoE feed-forward block on `tokens` rows of x [tokens, hidden]:
 * route (as arfq_moe_route), group (token, slot) pairs by expert, run each
 * expert's SwiGLU  down(silu(gate . x) * (up . x)), and scatter-add the results
 * weighted by the router weights into y[tokens, hidden] (f32, overwritten).
 * gate/up hold n_experts x [inter, hidden]; down holds n_experts x [hidden,
 * inter]; Q4_K, Q5_K, Q6_K, Q8_0 or IQ4_XS (gate and up alike).  Replaces add_moe_block_batched
 * (crates/arf-gpu/src/gpu/batch.rs:355-460) and the island's sorted mm_id chain
 * (crates/arf-gpu/src/gpu/metal/island.rs:4033-4134); oracle MoeMlp::forward
 * (crates/arf-core/src/model/moe.rs:53-86).  Scratch memory is owned by the
 * context and grows on demand. */
int arfq_moe(arfq_ctx *ctx, const arfq_weight *gate, const arfq_weight *up,
             const arfq_weight *down, const float *router_logits, int64_t tokens, int top_k,
             int norm_topk, const void *x, int x_dtype, float *y);

/* As arfq_moe, with routing already done: ids/weights [tokens, top_k] (device). */
int arfq_moe_ids(arfq_ctx *ctx, const arfq_weight *gate, const arfq_weight *up,
                 const arfq_weight *down, const int32_t *ids, const float *weights,
                 int64_t tokens, int top_k, const void *x, int x_dtype, float *y);

/* As arfq_moe / arfq_moe_ids, adding into y instead of overwriting it: y holds
 * the shared experts' output on entry (e.g. from arfq_ffn on the same x), and
 * each token's routed contributions are added to it in slot order,
 * y[t] = ((y[t] + w_0 * y_0) + w_1 * y_1) + ...  That is MoeMlp::forward with
 * shared experts (crates/arf-core/src/model/moe.rs:62-67: out starts at 0, the
 * shared experts' outputs are added first, then the routed experts'). */
int arfq_moe_add(arfq_ctx *ctx, const arfq_weight *gate, const arfq_weight *up,
                 const arfq_weight *down, const float *router_logits, int64_t tokens, int top_k,
                 int norm_topk, const void *x, int x_dtype, float *y);
int arfq_moe_ids_add(arfq_ctx *ctx, const arfq_weight *gate, const arfq_weight *up,
                     const arfq_weight *down, const int32_t *ids, const float *weights,
                     int64_t tokens, int top_k, const void *x, int x_dtype, float *y);

/* ---- device-memory and timing helpers -------------------------------------
 * For callers without their own HIP allocator (the FFI host, tests, the bench).
 * The reference's equivalents are GpuContext buffer init / readback
 * (crates/arf-gpu/src/gpu/context.rs:505-611) and its per-kernel timestamp
 * queries (crates/arf-gpu/src/gpu/command.rs:186-243). */
int arfq_dev_malloc(arfq_ctx *ctx, size_t bytes, void **out);
int arfq_dev_free(arfq_ctx *ctx, void *p);
/* Synchronous copies (they wait for the context's stream first). */
int arfq_copy_h2d(arfq_ctx *ctx, void *dst, const void *src, size_t bytes);
int arfq_copy_d2h(arfq_ctx *ctx, void *dst, const void *src, size_t bytes);
/* Enqueue a device-to-device copy on the context's stream (asynchronous).  It
 * runs a plain 16-byte-per-lane copy kernel when both pointers and `bytes` are
 * 16-byte aligned (hipMemcpyAsync otherwise); the kernel doubles as the
 * known-size reference for HBM byte counters.  No counterpart in the
 * reference (its buffers are copied by the wgpu/Metal runtime). */
int arfq_copy_d2d(arfq_ctx *ctx, void *dst, const void *src, size_t bytes);
/* Enqueue one read-only pass over `bytes` (a multiple of 16, 16-byte aligned)
 * of device memory at `src`: grid-stride 16-byte loads, eight 256-thread
 * workgroups per CU.  The practical HBM read ceiling the
 * GEMV roofline is judged against (the bench times it beside the datasheet
 * peak).  When `stamps` is not NULL (device memory, room for 4 * `nstamps`
 * uint64), the first wave of each of the first `nstamps` workgroups writes
 * (s_memrealtime, s_memtime) at its start and at its end there; their ratio
 * against the device's wall-clock rate (hipDeviceAttributeWallClockRate) is
 * the shader clock while the stream ran.  No counterpart in the reference
 * (its roofline probe reads through a wgpu kernel,
 * crates/arf-gpu/examples/gemv_roofline_probe.rs:15-45). */
int arfq_stream_read(arfq_ctx *ctx, const void *src, size_t bytes, uint64_t *stamps, int nstamps);
/* The context device's compute units, peak shader clock and the frequency of
 * s_memrealtime (both kHz, hipDeviceAttributeClockRate and
 * hipDeviceAttributeWallClockRate); any pointer may be NULL.  No counterpart
 * in the reference (its adapter info comes from wgpu). */
int arfq_ctx_device_info(arfq_ctx *ctx, int *cus, int *shader_clock_khz, int *wall_clock_khz);
/* The device scratch the context holds (grown on demand by arfq_matmul,
 * arfq_moe* and arfq_ffn*; never by arfq_matmul_noalloc) and the device's free
 * and total memory (hipMemGetInfo); any pointer may be NULL.  No counterpart
 * in the reference. */
int arfq_ctx_memory(arfq_ctx *ctx, size_t *scratch_bytes, size_t *device_free, size_t *device_total);
/* Record a start event / a stop event on the context's stream; elapsed time in
 * ms between the last start and stop (waits for the stop event). */
int arfq_timer_start(arfq_ctx *ctx);
int arfq_timer_stop(arfq_ctx *ctx, float *ms);
/* Enqueue `iters` arfq_matmul calls back to back, call i using ws[i % n_ws]
 * (distinct weight copies, so a timing loop streams from HBM rather than from
 * a cache), all with the same x and y.  For timing loops only. */
int arfq_matmul_repeat(arfq_ctx *ctx, const arfq_weight *const *ws, int n_ws, int iters,
                       int64_t m, const void *x, int x_dtype, float *y);

/* Gate activation of the dense FFN (GateAct, crates/arf-core/src/config.rs:58):
 * SwiGLU silu(g) * u (crates/arf-ml/src/lib.rs:160-162) or GeGLU
 * gelu_tanh(g) * u with the tanh argument clamped to [-15, 15]
 * (crates/arf-gpu/src/shaders/metal/decode_ops_msl.metal:15-27). */
typedef enum { ARFQ_ACT_SILU = 0, ARFQ_ACT_GELU_TANH = 1 } arfq_act;

/* The dense FFN of one decode/prefill step on already-normalised x (f32,
 * [m, hidden], device): y = down . (act(gate . x) * (up . x)), f32 [m, hidden];
 * gate/up [inter, hidden], down [hidden, inter], single matrices of any qtype
 * the matmul takes; act an arfq_act.  Replaces the island's ffn_dispatch (gate
 * GEMV, up GEMV, the geglu kernel, down GEMV on one queue;
 * crates/arf-gpu/src/gpu/metal/island.rs:13436-13529), its activation choice
 * in the decode and batch paths (crates/arf-gpu/src/gpu/decode.rs:123,
 * batch.rs:6953) and Mlp::forward (crates/arf-core/src/model/mlp.rs:20-24).
 * At m = 1 with Q4_K gate and up of one shape, gate and up run as one launch;
 * with Q4_K down weights at m = 1 and inter <= 8192 (m <= 4 and inter <= 4096
 * under ARFQ_OPT_GEMV_X16) the activation is applied as the down GEMV reads
 * its x (no intermediate), otherwise it runs as a kernel of its own between
 * them.  Either way h = act(g) * u is the same f32 value. */
int arfq_ffn_act(arfq_ctx *ctx, const arfq_weight *gate, const arfq_weight *up, const arfq_weight *down,
                 int64_t m, const float *x, float *y, int act);
/* arfq_ffn_act with ARFQ_ACT_SILU (Mlp::forward). */
int arfq_ffn(arfq_ctx *ctx, const arfq_weight *gate, const arfq_weight *up, const arfq_weight *down,
             int64_t m, const float *x, float *y);

/* ---- GGUF reader ---------------------------------------------------------
 * A GGUF v3 file opened read-only and memory-mapped; tensors are read in place
 * (LazyGguf, crates/arf-core/src/model/gguf.rs:365-564).  Errors of
 * arfq_gguf_open are read with arfq_gguf_last_error(NULL); those of calls on an
 * open file with arfq_gguf_last_error(g). */
typedef struct arfq_gguf arfq_gguf;
/* 1 when `path` is a regular file starting with the GGUF magic, else 0
 * (is_gguf_file, gguf.rs:1115-1125). */
int arfq_gguf_is_gguf(const char *path);
/* Parse the header, the key/value section (general.alignment is kept, other
 * values skipped) and the tensor table (LazyGguf::open_raw, gguf.rs:509-564;
 * Reader::skip_value, gguf.rs:323-360).  Unknown ggml type ids fail the open
 * as GgmlType::from_id does (gguf.rs:60-90).  ARFQ_E_IO / ARFQ_E_FORMAT. */
int arfq_gguf_open(const char *path, arfq_gguf **out);
int arfq_gguf_close(arfq_gguf *g);
const char *arfq_gguf_last_error(const arfq_gguf *g);
/* Tensor table: count, and entry `index` in file order (tensor_names,
 * shape_raw, raw_ggml_type_id, gguf.rs:720-760,830-842).  dims are ggml's,
 * fastest-varying first (up to max_dims are written); file_offset is absolute;
 * nbytes is ggml_byte_len (gguf.rs:1678-1705).  Any out-pointer may be NULL. */
int arfq_gguf_tensor_count(const arfq_gguf *g, int64_t *n);
int arfq_gguf_tensor_info(const arfq_gguf *g, int64_t index, const char **name, int *ggml_type,
                          int *n_dims, int64_t *dims, int max_dims, uint64_t *file_offset,
                          uint64_t *nbytes);
int arfq_gguf_find(const arfq_gguf *g, const char *name, int64_t *index);
/* The raw blocks of tensor `name` when it is stored as ggml type `ggml_type`:
 * a pointer into the mapping (valid until arfq_gguf_close), its byte length,
 * rows = elements / ne0 and cols = ne0 (get_q4k_blocks_raw,
 * get_q8_0_blocks_raw, gguf.rs:774-828; any type id).  ARFQ_E_UNSUPPORTED
 * when stored as another type (the reference returns None). */
int arfq_gguf_blocks(const arfq_gguf *g, const char *name, int ggml_type, const void **blocks,
                     size_t *nbytes, int64_t *rows, int64_t *cols);
/* Upload tensor `name` (Q8_0, Q4_K, Q5_K, Q6_K or IQ4_XS) as a weight:
 *   - 2-D [ne0 = k, ne1 = n]: rows [row0, row0 + n_rows) (n_rows < 0: to the
 *     end) as one matrix (the fused-qkv row slice, Entry::RowSlice,
 *     gguf.rs:125-140); rows start on block boundaries because blocks run along
 *     k;
 *   - 3-D [ne0 = k, ne1 = n, ne2 = experts] (`*_exps`): every expert, in
 *     order (index_experts, gguf.rs:1479-1523); row0 = 0, n_rows = -1 or ne1.
 * k must be a whole number of blocks.  Synchronous, as arfq_weight_upload. */
int arfq_gguf_upload(arfq_ctx *ctx, const arfq_gguf *g, const char *name, int64_t row0,
                     int64_t n_rows, arfq_weight **out);

#ifdef __cplusplus
}
#endif
#endif /* ARFQ_H */
