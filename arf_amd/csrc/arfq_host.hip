// arfq_host.hip -- the C ABI (include/arfq.h): contexts, weight upload,
// kernel selection by (qtype, m), MoE orchestration and the memory / timing
// helpers.  All device work goes to the context's stream.
#include <stdio.h>
#include <string.h>

#include <new>
#include <string>

#include "arfq_common.h"
#include "arfq_internal.h"

#include <algorithm>

// ---- scratch of the allocation-free matmul (arfq_matmul_noalloc) ----
// One fixed array per GPU, in the library's code object: resident from the
// module load until the process ends.  Host code never passes `scratch`
// itself (in host code the name is a stand-in, not a device address); its
// device address on each GPU is read once with hipGetSymbolAddress when the
// first context on that GPU is created and kept in g_noalloc_ptr[device].
static __device__ __align__(256) uint8_t scratch[ARFQ_NOALLOC_SCRATCH_BYTES];

namespace {

thread_local std::string g_create_err;

constexpr int NOALLOC_DEVICES = 64;
std::atomic<void *> g_noalloc_ptr[NOALLOC_DEVICES];

// The device address of `scratch` on the current device `device` (looked up
// once per device); null when the lookup fails.
hipError_t noalloc_scratch_of(int device, void **out) {
    *out = nullptr;
    if (device < 0 || device >= NOALLOC_DEVICES) return hipErrorInvalidDevice;
    void *p = g_noalloc_ptr[device].load(std::memory_order_acquire);
    if (!p) {
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_noalloc_ptr[device].store(p, std::memory_order_release);
    }
    *out = p;
    return hipSuccess;
}

int fail(arfq_ctx *ctx, int code, const std::string &msg) {
    if (ctx) ctx->err = msg;
    return code;
}

int hip_fail(arfq_ctx *ctx, hipError_t e, const char *what) {
    std::string m = std::string(what) + ": " + hipGetErrorString(e);
    return fail(ctx, ARFQ_E_DEVICE, m);
}

#define HIP_TRY(ctx, expr)                                   \
    do {                                                     \
        hipError_t _e = (expr);                              \
        if (_e != hipSuccess) return hip_fail(ctx, _e, #expr); \
    } while (0)

// Make the context's device current for this thread.
int use_device(arfq_ctx *ctx) {
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipSetDevice");
    return ARFQ_OK;
}

}  // namespace

extern "C" {

int arfq_version(void) { return ARFQ_VERSION; }

const char *arfq_status_string(int status) {
    switch (status) {
    case ARFQ_OK: return "ok";
    case ARFQ_E_INVALID: return "invalid argument";
    case ARFQ_E_SHAPE: return "shape mismatch";
    case ARFQ_E_DEVICE: return "HIP device error";
    case ARFQ_E_NOMEM: return "device out of memory";
    case ARFQ_E_UNSUPPORTED: return "unsupported";
    case ARFQ_E_FORMAT: return "malformed GGUF file";
    case ARFQ_E_IO: return "file I/O error";
    case ARFQ_E_NOT_FOUND: return "no such tensor";
    default: return "unknown status";
    }
}

int arfq_ctx_create(int device, void *stream, arfq_ctx **out) {
    if (!out) {
        g_create_err = "arfq_ctx_create: out is NULL";
        return ARFQ_E_INVALID;
    }
    *out = nullptr;
    int ndev = 0;
    hipError_t e = hipGetDeviceCount(&ndev);
    if (e != hipSuccess || ndev == 0) {
        g_create_err = std::string("arfq_ctx_create: no HIP device (") +
                       (e != hipSuccess ? hipGetErrorString(e) : "count 0") + ")";
        return ARFQ_E_DEVICE;
    }
    if (device < 0 || device >= ndev) {
        g_create_err = "arfq_ctx_create: device index out of range";
        return ARFQ_E_INVALID;
    }
    arfq_ctx *ctx = new (std::nothrow) arfq_ctx();
    if (!ctx) return ARFQ_E_NOMEM;
    ctx->device = device;
    e = hipSetDevice(device);
    if (e == hipSuccess) {
        if (stream) {
            ctx->stream = (hipStream_t)stream;
        } else {
            e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
            ctx->own_stream = (e == hipSuccess);
        }
    }
    if (e == hipSuccess) e = hipDeviceGetAttribute(&ctx->cus, hipDeviceAttributeMultiprocessorCount, device);
    // the allocation-free entry point's scratch on this device (resolved here, at set-up)
    if (e == hipSuccess) e = noalloc_scratch_of(device, &ctx->noalloc_scratch);
    if (e == hipSuccess) e = hipEventCreate(&ctx->ev_start);
    if (e == hipSuccess) e = hipEventCreate(&ctx->ev_stop);
    if (e == hipSuccess) {
        // STREAM_SINK_WORDS words of arfq_stream_read's sink, then the upload's
        // flag words
        e = hipMalloc(&ctx->aux, ((size_t)arfq::STREAM_SINK_WORDS + arfq::UPLOAD_FLAG_WORDS) * sizeof(uint32_t));
    }
    if (e == hipSuccess)
        e = hipMemsetAsync(ctx->aux, 0, ((size_t)arfq::STREAM_SINK_WORDS + arfq::UPLOAD_FLAG_WORDS) * sizeof(uint32_t),
                           ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        g_create_err = std::string("arfq_ctx_create: ") + hipGetErrorString(e);
        arfq_ctx_destroy(ctx);
        return ARFQ_E_DEVICE;
    }
    *out = ctx;
    return ARFQ_OK;
}

int arfq_ctx_destroy(arfq_ctx *ctx) {
    if (!ctx) return ARFQ_E_INVALID;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream && ctx->scratch) (void)hipFreeAsync(ctx->scratch, ctx->stream);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    if (ctx->staging) (void)hipFree(ctx->staging);
    if (ctx->aux) (void)hipFree(ctx->aux);
    if (ctx->ev_start) (void)hipEventDestroy(ctx->ev_start);
    if (ctx->ev_stop) (void)hipEventDestroy(ctx->ev_stop);
    if (ctx->own_stream && ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return ARFQ_OK;
}

void *arfq_ctx_stream(arfq_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

const char *arfq_last_error(const arfq_ctx *ctx) {
    return ctx ? ctx->err.c_str() : g_create_err.c_str();
}

int arfq_ctx_sync(arfq_ctx *ctx) {
    if (!ctx) return ARFQ_E_INVALID;
    if (int rc = use_device(ctx)) return rc;
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    return ARFQ_OK;
}

int arfq_ctx_set_options(arfq_ctx *ctx, unsigned options) {
    if (!ctx) return ARFQ_E_INVALID;
    if (options & ~ARFQ_OPT_GEMV_X16) return fail(ctx, ARFQ_E_INVALID, "set_options: unknown option bits");
    ctx->options = options;
    return ARFQ_OK;
}

// ---------------------------------------------------------------- weights ----

static int weight_create(arfq_ctx *ctx, int qtype, size_t nbytes, int64_t n_rows, int64_t k_cols,
                         int n_experts, arfq_weight **out) {
    if (!ctx || !out) return fail(ctx, ARFQ_E_INVALID, "weight upload: null argument");
    *out = nullptr;
    const int bb = arfq::block_bytes_of(qtype);
    if (bb == 0) return fail(ctx, ARFQ_E_INVALID, "weight upload: unknown qtype");
    const int qk = arfq::qk_of(qtype);
    if (n_rows <= 0 || k_cols <= 0 || n_experts <= 0)
        return fail(ctx, ARFQ_E_SHAPE, "weight upload: non-positive dimension");
    if (k_cols % qk != 0)
        return fail(ctx, ARFQ_E_SHAPE,
                    "weight upload: k_cols must be a multiple of " + std::to_string(qk));
    if (n_rows > (int64_t)1 << 30 || k_cols > (int64_t)1 << 30)
        return fail(ctx, ARFQ_E_SHAPE, "weight upload: dimension too large");
    const int64_t nblk = (int64_t)n_experts * n_rows * (k_cols / qk);
    if ((size_t)nblk * (size_t)bb != nbytes)
        return fail(ctx, ARFQ_E_SHAPE,
                    "weight upload: nbytes " + std::to_string(nbytes) + " != expected " +
                        std::to_string((size_t)nblk * bb));
    if (int rc = use_device(ctx)) return rc;
    arfq_weight *w = new (std::nothrow) arfq_weight();
    if (!w) return fail(ctx, ARFQ_E_NOMEM, "weight upload: host allocation");
    w->ctx = ctx;
    w->qtype = qtype;
    w->n = n_rows;
    w->k = k_cols;
    w->experts = n_experts;
    w->nblk = nblk;
    w->bytes = (size_t)n_rows * (size_t)(k_cols / qk) * (size_t)bb;
    size_t sz[3] = {0, 0, 0};
    switch (qtype) {
    case ARFQ_Q4_K: sz[0] = nblk * 16; sz[1] = nblk * 128; break;
    case ARFQ_Q8_0: sz[0] = nblk * 32; sz[1] = nblk * 2; break;
    case ARFQ_Q6_K: sz[0] = nblk * 192; sz[1] = nblk * 16; sz[2] = nblk * 2; break;
    case ARFQ_Q5_K: sz[0] = nblk * 16; sz[1] = nblk * 160; break;
    case ARFQ_IQ4_XS: sz[0] = nblk * 8; sz[1] = nblk * 128; break;
    }
    void **dst[3] = {&w->s0, &w->s1, &w->s2};
    for (int i = 0; i < 3; i++) {
        if (!sz[i]) continue;
        // round up so 16-byte vector loads of the last element stay in bounds
        hipError_t e = hipMalloc(dst[i], (sz[i] + 255) & ~(size_t)255);
        if (e != hipSuccess) {
            arfq_weight_free(w);
            return fail(ctx, ARFQ_E_NOMEM, std::string("weight upload: hipMalloc: ") +
                                               hipGetErrorString(e));
        }
    }
    *out = w;
    return ARFQ_OK;
}

// Q6_K uploads: the repack flags a sub-block scale outside [-64, 64] and one
// outside [-62, 62] in two words of the context's counter allocation (cleared
// first); read back once the repacks are done, they select the prefill GEMM's
// two-operand weights and the skinny kernel's operand form.
static uint32_t *upload_flag(arfq_ctx *ctx, const arfq_weight *w) {
    return w->qtype == ARFQ_Q6_K && ctx->aux ? ctx->aux + arfq::STREAM_SINK_WORDS : nullptr;
}
static hipError_t upload_flag_clear(arfq_ctx *ctx, uint32_t *flag) {
    return flag ? hipMemsetAsync(flag, 0, 2 * sizeof(uint32_t), ctx->stream) : hipSuccess;
}
static hipError_t upload_flag_read(arfq_ctx *ctx, uint32_t *flag, arfq_weight *w) {
    if (!flag) return hipSuccess;
    uint32_t h[2] = {0, 0};
    hipError_t e = hipMemcpyAsync(h, flag, sizeof(h), hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    w->wide = h[0] != 0;
    w->over62 = h[1] != 0;
    return e;
}

int arfq_weight_upload_device(arfq_ctx *ctx, int qtype, const void *dev_blocks, size_t nbytes,
                              int64_t n_rows, int64_t k_cols, int n_experts, arfq_weight **out) {
    if (!dev_blocks) return fail(ctx, ARFQ_E_INVALID, "weight upload: null blocks");
    arfq_weight *w = nullptr;
    if (int rc = weight_create(ctx, qtype, nbytes, n_rows, k_cols, n_experts, &w)) return rc;
    uint32_t *flag = upload_flag(ctx, w);
    hipError_t e = upload_flag_clear(ctx, flag);
    if (e == hipSuccess) e = arfq::launch_repack(w, (const uint8_t *)dev_blocks, ctx->stream, 0, -1, flag);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e == hipSuccess) e = upload_flag_read(ctx, flag, w);
    if (e != hipSuccess) {
        arfq_weight_free(w);
        return hip_fail(ctx, e, "weight upload: repack");
    }
    *out = w;
    return ARFQ_OK;
}

int arfq_weight_upload(arfq_ctx *ctx, int qtype, const void *host_blocks, size_t nbytes,
                       int64_t n_rows, int64_t k_cols, int n_experts, arfq_weight **out) {
    if (!ctx || !host_blocks || !out) return fail(ctx, ARFQ_E_INVALID, "weight upload: null argument");
    arfq_weight *w = nullptr;
    if (int rc = weight_create(ctx, qtype, nbytes, n_rows, k_cols, n_experts, &w)) return rc;
    // through the context's staging buffer, UPLOAD_CHUNK bytes of whole blocks at a
    // time (copy and repack are ordered on the stream); the buffer is allocated
    // once, on the first upload that needs it
    const int64_t bb = arfq::block_bytes_of(qtype);
    const int64_t per = std::max<int64_t>(1, (int64_t)arfq::UPLOAD_CHUNK / bb);
    const size_t need = (size_t)std::min<int64_t>(w->nblk, per) * (size_t)bb;
    hipError_t e = hipSuccess;
    if (ctx->staging_bytes < need) {
        e = hipStreamSynchronize(ctx->stream);  // an earlier upload's copies are done
        if (e == hipSuccess && ctx->staging) (void)hipFree(ctx->staging);
        ctx->staging = nullptr;
        ctx->staging_bytes = 0;
        if (e == hipSuccess) e = hipMalloc(&ctx->staging, std::max(need, (size_t)1 << 20));
        if (e != hipSuccess) {
            arfq_weight_free(w);
            return fail(ctx, ARFQ_E_NOMEM, std::string("weight upload: staging: ") + hipGetErrorString(e));
        }
        ctx->staging_bytes = std::max(need, (size_t)1 << 20);
    }
    uint32_t *flag = upload_flag(ctx, w);
    if (e == hipSuccess) e = upload_flag_clear(ctx, flag);
    for (int64_t b0 = 0; e == hipSuccess && b0 < w->nblk; b0 += per) {
        const int64_t nb = std::min(per, w->nblk - b0);
        e = hipMemcpyAsync(ctx->staging, (const uint8_t *)host_blocks + b0 * bb, (size_t)(nb * bb),
                           hipMemcpyHostToDevice, ctx->stream);
        if (e == hipSuccess) e = arfq::launch_repack(w, (const uint8_t *)ctx->staging, ctx->stream, b0, nb, flag);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e == hipSuccess) e = upload_flag_read(ctx, flag, w);
    if (e != hipSuccess) {
        arfq_weight_free(w);
        return hip_fail(ctx, e, "weight upload");
    }
    *out = w;
    return ARFQ_OK;
}

int arfq_weight_free(arfq_weight *w) {
    if (!w) return ARFQ_E_INVALID;
    if (w->ctx) (void)hipSetDevice(w->ctx->device);
    if (w->s0) (void)hipFree(w->s0);
    if (w->s1) (void)hipFree(w->s1);
    if (w->s2) (void)hipFree(w->s2);
    delete w;
    return ARFQ_OK;
}

int arfq_weight_info(const arfq_weight *w, int *qtype, int64_t *n_rows, int64_t *k_cols,
                     int *n_experts, size_t *device_bytes) {
    if (!w) return ARFQ_E_INVALID;
    if (qtype) *qtype = w->qtype;
    if (n_rows) *n_rows = w->n;
    if (k_cols) *k_cols = w->k;
    if (n_experts) *n_experts = w->experts;
    if (device_bytes) *device_bytes = w->bytes;
    return ARFQ_OK;
}

// ----------------------------------------------------------------- matmul ----

static int check_matmul(arfq_ctx *ctx, const arfq_weight *w, int expert, int64_t m,
                        const void *x, int x_dtype, const float *y) {
    if (!ctx) return ARFQ_E_INVALID;
    if (!w || !x || !y) return fail(ctx, ARFQ_E_INVALID, "matmul: null argument");
    if (x_dtype != ARFQ_F32 && x_dtype != ARFQ_F16)
        return fail(ctx, ARFQ_E_INVALID, "matmul: unknown x dtype");
    if (expert < 0 || expert >= w->experts)
        return fail(ctx, ARFQ_E_SHAPE, "matmul: expert index out of range");
    if (m <= 0 || m > (int64_t)1 << 24) return fail(ctx, ARFQ_E_SHAPE, "matmul: bad m");
    return ARFQ_OK;
}

// Grow the context scratch to at least `bytes`.  Stream-ordered: the old block
// is freed after the work already enqueued on the stream (which may still use
// it) and the new one is allocated in stream order, so the host does not wait.
static int ensure_scratch(arfq_ctx *ctx, size_t bytes) {
    if (ctx->scratch_bytes >= bytes) return ARFQ_OK;
    if (ctx->scratch) HIP_TRY(ctx, hipFreeAsync(ctx->scratch, ctx->stream));
    ctx->scratch = nullptr;
    ctx->scratch_bytes = 0;
    const size_t sz = (bytes + 0xFFFFF) & ~(size_t)0xFFFFF;
    hipError_t e = hipMallocAsync(&ctx->scratch, sz, ctx->stream);
    if (e != hipSuccess) return fail(ctx, ARFQ_E_NOMEM, std::string("scratch: ") + hipGetErrorString(e));
    ctx->scratch_bytes = sz;
    return ARFQ_OK;
}

static int matmul_enqueue(arfq_ctx *ctx, const arfq_weight *w, int expert, int64_t m,
                          const void *x, int x_dtype, float *y) {
    hipError_t e;
    const bool x16 = (ctx->options & ARFQ_OPT_GEMV_X16) != 0;
    if (x_dtype == ARFQ_F32 && arfq::gemv_supports(w, m, x16)) {
        e = arfq::launch_gemv(w, expert, m, (const float *)x, y, ctx->stream, x16);
    } else if (arfq::gemm_supports(w, m)) {
        const arfq::GemmPlan plan = arfq::gemm_plan(w, m, x_dtype, x16);
        if (int rc = ensure_scratch(ctx, plan.scratch_bytes)) return rc;
        e = arfq::launch_gemm(w, expert, m, x, x_dtype, y, ctx->scratch, plan, ctx->stream);
    } else {
        return fail(ctx, ARFQ_E_UNSUPPORTED,
                    "matmul: no kernel for qtype " + std::to_string(w->qtype) + " at m=" +
                        std::to_string(m) + (x_dtype == ARFQ_F16 ? " (f16 x)" : " (f32 x)"));
    }
    if (e != hipSuccess) return hip_fail(ctx, e, "matmul launch");
    return ARFQ_OK;
}

int arfq_matmul(arfq_ctx *ctx, const arfq_weight *w, int expert, int64_t m, const void *x,
                int x_dtype, float *y) {
    if (int rc = check_matmul(ctx, w, expert, m, x, x_dtype, y)) return rc;
    if (int rc = use_device(ctx)) return rc;
    return matmul_enqueue(ctx, w, expert, m, x, x_dtype, y);
}

int arfq_matmul_noalloc(arfq_ctx *ctx, const arfq_weight *w, int expert, int64_t m, const void *x,
                        int x_dtype, float *y) {
    if (int rc = check_matmul(ctx, w, expert, m, x, x_dtype, y)) return rc;
    if (int rc = use_device(ctx)) return rc;
    if (!ctx->noalloc_scratch) return fail(ctx, ARFQ_E_DEVICE, "matmul_noalloc: no scratch on this device");
    hipError_t e;
    const bool x16 = (ctx->options & ARFQ_OPT_GEMV_X16) != 0;
    if (x_dtype == ARFQ_F32 && arfq::gemv_supports(w, m, x16)) {
        // the decode GEMVs use no scratch
        e = arfq::launch_gemv(w, expert, m, (const float *)x, y, ctx->stream, x16);
    } else if (arfq::gemm_supports(w, m)) {
        const arfq::GemmPlan plan = arfq::gemm_plan(w, m, x_dtype, x16);
        if (plan.scratch_bytes > ARFQ_NOALLOC_SCRATCH_BYTES)
            return fail(ctx, ARFQ_E_UNSUPPORTED,
                        "matmul_noalloc: this product needs " + std::to_string(plan.scratch_bytes) +
                            " bytes of scratch, above the " + std::to_string(ARFQ_NOALLOC_SCRATCH_BYTES) +
                            "-byte limit (use arfq_matmul)");
        // every scratch byte a plan reads is written earlier in the same call
        // (x preparation, then the split-K partials before the launch that adds them)
        e = arfq::launch_gemm(w, expert, m, x, x_dtype, y, ctx->noalloc_scratch, plan, ctx->stream);
    } else {
        return fail(ctx, ARFQ_E_UNSUPPORTED,
                    "matmul_noalloc: no kernel for qtype " + std::to_string(w->qtype) + " at m=" +
                        std::to_string(m));
    }
    if (e != hipSuccess) return hip_fail(ctx, e, "matmul_noalloc launch");
    return ARFQ_OK;
}

int arfq_matmul_repeat(arfq_ctx *ctx, const arfq_weight *const *ws, int n_ws, int iters,
                       int64_t m, const void *x, int x_dtype, float *y) {
    if (!ctx) return ARFQ_E_INVALID;
    if (!ws || n_ws <= 0 || iters < 0) return fail(ctx, ARFQ_E_INVALID, "matmul_repeat: bad args");
    for (int i = 0; i < n_ws; i++) {
        if (int rc = check_matmul(ctx, ws[i], 0, m, x, x_dtype, y)) return rc;
        if (ws[i]->n != ws[0]->n || ws[i]->k != ws[0]->k || ws[i]->qtype != ws[0]->qtype)
            return fail(ctx, ARFQ_E_SHAPE, "matmul_repeat: weights differ in shape");
    }
    if (int rc = use_device(ctx)) return rc;
    for (int i = 0; i < iters; i++)
        if (int rc = matmul_enqueue(ctx, ws[i % n_ws], 0, m, x, x_dtype, y)) return rc;
    return ARFQ_OK;
}

// -------------------------------------------------------------------- MoE ----

static size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

int arfq_moe_route(arfq_ctx *ctx, const float *logits, int64_t tokens, int n_experts, int top_k,
                   int norm_topk, int32_t *ids, float *weights) {
    if (!ctx) return ARFQ_E_INVALID;
    if (tokens < 0) return fail(ctx, ARFQ_E_SHAPE, "moe_route: tokens < 0");
    if (tokens > 0 && (!logits || !ids || !weights))
        return fail(ctx, ARFQ_E_INVALID, "moe_route: null argument");
    if (n_experts < 1 || n_experts > arfq::MOE_ROUTE_EXPERTS_MAX)
        return fail(ctx, ARFQ_E_SHAPE, "moe_route: n_experts must be in [1, 1024]");
    if (top_k < 1 || top_k > n_experts || top_k > arfq::MOE_TOPK_MAX)
        return fail(ctx, ARFQ_E_SHAPE, "moe_route: top_k must be in [1, min(n_experts, 64)]");
    if (int rc = use_device(ctx)) return rc;
    hipError_t e = arfq::launch_moe_route(logits, tokens, n_experts, top_k, norm_topk ? 1 : 0, ids,
                                          weights, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "moe_route launch");
    return ARFQ_OK;
}

// Shapes: gate/up n_experts x [inter, hidden]; down n_experts x [hidden, inter].
static int check_moe(arfq_ctx *ctx, const arfq_weight *gate, const arfq_weight *up,
                     const arfq_weight *down, int64_t tokens, int top_k, const void *x,
                     int x_dtype, const float *y) {
    if (!ctx) return ARFQ_E_INVALID;
    if (!gate || !up || !down) return fail(ctx, ARFQ_E_INVALID, "moe: null weight");
    if (tokens < 0) return fail(ctx, ARFQ_E_SHAPE, "moe: tokens < 0");
    if (tokens > 0 && (!x || !y)) return fail(ctx, ARFQ_E_INVALID, "moe: null x or y");
    if (x_dtype != ARFQ_F32 && x_dtype != ARFQ_F16)
        return fail(ctx, ARFQ_E_INVALID, "moe: unknown x dtype");
    const int E = gate->experts;
    if (up->experts != E || down->experts != E)
        return fail(ctx, ARFQ_E_SHAPE, "moe: gate/up/down expert counts differ");
    if (E > arfq::MOE_EXPERTS_MAX) return fail(ctx, ARFQ_E_UNSUPPORTED, "moe: more than 512 experts");
    if (up->qtype != gate->qtype) return fail(ctx, ARFQ_E_UNSUPPORTED, "moe: gate and up differ in qtype");
    if (up->n != gate->n || up->k != gate->k || down->n != gate->k || down->k != gate->n)
        return fail(ctx, ARFQ_E_SHAPE,
                    "moe: want gate/up [inter, hidden] and down [hidden, inter]");
    if (gate->k % 256 != 0 || down->k % 256 != 0)
        return fail(ctx, ARFQ_E_UNSUPPORTED, "moe: hidden and inter must be multiples of 256");
    if (top_k < 1 || top_k > E || top_k > arfq::MOE_TOPK_MAX)
        return fail(ctx, ARFQ_E_SHAPE, "moe: top_k must be in [1, min(n_experts, 64)]");
    if (tokens * top_k > (int64_t)1 << 24) return fail(ctx, ARFQ_E_SHAPE, "moe: too many tokens");
    return ARFQ_OK;
}

// Route (when ids == NULL) + group + grouped GEMMs + combine, all on the stream.
// Scratch layout: [x f16] [ids] [weights] [off] [sorted] [tiles] [ntiles] [h f16] [o f32].
static int moe_enqueue(arfq_ctx *ctx, const arfq_weight *gate, const arfq_weight *up,
                       const arfq_weight *down, const float *logits, const int32_t *ids_in,
                       const float *wts_in, int64_t tokens, int top_k, int norm_topk,
                       const void *x, int x_dtype, float *y, bool accumulate) {
    if (tokens == 0) return ARFQ_OK;
    const int E = gate->experts;
    const int64_t hidden = gate->k, inter = gate->n, P = tokens * top_k;
    // Few (token, expert) pairs: one indirect GEMV per weight over the pairs (route ->
    // gate -> up -> down with SwiGLU on its x -> combine), instead of grouping pairs
    // into expert tiles the grouped GEMMs would mostly leave empty (the reference's
    // mul_mv_id crossover, crates/arf-gpu/src/gpu/metal/island.rs:4048-4070).
    if (P <= arfq::MOE_DECODE_PAIRS_MAX && gate->qtype == ARFQ_Q4_K && down->qtype == ARFQ_Q4_K &&
        arfq::gemv_pairs_supports(gate) && arfq::gemv_pairs_supports(down)) {
        size_t o = 0;
        const size_t o_ids = o;  o += ids_in ? 0 : align256((size_t)P * 4);
        const size_t o_w = o;    o += ids_in ? 0 : align256((size_t)P * 4);
        const size_t o_g = o;    o += align256((size_t)P * inter * 4);
        const size_t o_u = o;    o += align256((size_t)P * inter * 4);
        const size_t o_o = o;    o += align256((size_t)P * hidden * 4);
        if (int rc = ensure_scratch(ctx, o)) return rc;
        char *sc = (char *)ctx->scratch;
        hipError_t e;
        const int32_t *ids = ids_in;
        const float *wts = wts_in;
        if (!ids_in) {
            e = arfq::launch_moe_route(logits, tokens, E, top_k, norm_topk ? 1 : 0,
                                       (int32_t *)(sc + o_ids), (float *)(sc + o_w), ctx->stream);
            if (e != hipSuccess) return hip_fail(ctx, e, "moe: route launch");
            ids = (const int32_t *)(sc + o_ids);
            wts = (const float *)(sc + o_w);
        }
        float *g = (float *)(sc + o_g), *u = (float *)(sc + o_u), *ob = (float *)(sc + o_o);
        if (arfq::gemv_pairs_dual_supports(gate, up)) {
            e = arfq::launch_gemv_pairs_dual(gate, up, P, ids, x, x_dtype, top_k, g, u, ctx->stream);
        } else {
            e = arfq::launch_gemv_pairs(gate, P, ids, x, x_dtype, top_k, nullptr, nullptr, g, ctx->stream);
            if (e == hipSuccess)
                e = arfq::launch_gemv_pairs(up, P, ids, x, x_dtype, top_k, nullptr, nullptr, u, ctx->stream);
        }
        if (e != hipSuccess) return hip_fail(ctx, e, "moe: gate/up GEMV launch");
        e = arfq::launch_gemv_pairs(down, P, ids, nullptr, ARFQ_F32, 1, g, u, ob, ctx->stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "moe: down GEMV launch");
        e = arfq::launch_moe_combine(ob, ids, wts, tokens, top_k, E, hidden, y, accumulate, ctx->stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "moe: combine launch");
        return ARFQ_OK;
    }
    const int64_t max_tiles = arfq::moe_max_tiles(P, E);
    // the formats with a min term read x sub-block sums
    const bool gsums = gate->qtype == ARFQ_Q4_K || gate->qtype == ARFQ_Q5_K;
    const bool dsums = down->qtype == ARFQ_Q4_K || down->qtype == ARFQ_Q5_K;
    size_t o = 0;
    const size_t o_x = o;     o += x_dtype == ARFQ_F32 ? align256((size_t)tokens * hidden * 2) : 0;
    const size_t o_xrs = o;   o += x_dtype == ARFQ_F32 ? align256((size_t)tokens * 4) : 0;
    const size_t o_xs = o;    o += gsums ? align256((size_t)tokens * (hidden / 16) * 2) : 0;
    const size_t o_ids = o;   o += ids_in ? 0 : align256((size_t)P * 4);
    const size_t o_w = o;     o += ids_in ? 0 : align256((size_t)P * 4);
    const size_t o_off = o;   o += align256((size_t)(E + 1) * 4);
    const size_t o_srt = o;   o += align256((size_t)P * 4);
    const size_t o_tl = o;    o += align256((size_t)max_tiles * 8);
    const size_t o_nt = o;    o += 256;
    const size_t o_h = o;     o += align256((size_t)P * inter * 4);
    const size_t o_h16 = o;   o += align256((size_t)P * inter * 2);
    const size_t o_rs = o;    o += align256((size_t)P * 4);
    const size_t o_hs = o;    o += dsums ? align256((size_t)P * (inter / 16) * 2) : 0;
    const size_t o_o = o;     o += align256((size_t)P * hidden * 4);
    if (int rc = ensure_scratch(ctx, o)) return rc;
    char *sc = (char *)ctx->scratch;
    hipError_t e;
    // the grouped GEMMs read f16 activation tiles (as the reference's mm_id
    // kernel stages half tiles, moe_mm_id_q4ks.metal:34-46) and, for Q4_K and
    // Q5_K, the x sub-block sums
    const _Float16 *xh = x_dtype == ARFQ_F32 ? (const _Float16 *)(sc + o_x) : (const _Float16 *)x;
    uint16_t *xs = gsums ? (uint16_t *)(sc + o_xs) : nullptr;
    // an f32 x is stored row-scaled into f16 range; gate|up multiply back
    float *xrs = x_dtype == ARFQ_F32 ? (float *)(sc + o_xrs) : nullptr;
    // an f16 x needing only its sums gets them from the routing launch
    const bool sums_in_route = !ids_in && x_dtype != ARFQ_F32 && xs;
    if (!sums_in_route) {
        e = arfq::launch_xprep(x, x_dtype, tokens, hidden,
                               x_dtype == ARFQ_F32 ? (_Float16 *)(sc + o_x) : nullptr, nullptr, xs, xrs,
                               ctx->stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "moe: x preparation launch");
    }
    const int32_t *ids = ids_in;
    const float *wts = wts_in;
    if (!ids_in) {
        e = arfq::launch_moe_route(logits, tokens, E, top_k, norm_topk ? 1 : 0, (int32_t *)(sc + o_ids),
                                   (float *)(sc + o_w), ctx->stream, sums_in_route ? xh : nullptr, hidden,
                                   sums_in_route ? xs : nullptr);
        if (e != hipSuccess) return hip_fail(ctx, e, "moe: route launch");
        ids = (const int32_t *)(sc + o_ids);
        wts = (const float *)(sc + o_w);
    }
    int32_t *off = (int32_t *)(sc + o_off), *srt = (int32_t *)(sc + o_srt);
    int32_t *nt = (int32_t *)(sc + o_nt);
    void *tiles = sc + o_tl;
    float *h = (float *)(sc + o_h);
    _Float16 *h16 = (_Float16 *)(sc + o_h16);
    float *rs = (float *)(sc + o_rs);
    uint16_t *hs = dsums ? (uint16_t *)(sc + o_hs) : nullptr;
    float *ob = (float *)(sc + o_o);
    e = arfq::launch_moe_group(ids, P, E, off, srt, tiles, nt, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "moe: group launch");
    e = arfq::launch_moe_gateup(gate, up, xh, xs, xrs, top_k, off, srt, tiles, nt, max_tiles, h,
                                ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "moe: gate/up launch");
    e = arfq::launch_moe_hprep(h, P, (int)inter, h16, hs, rs, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "moe: h preparation launch");
    e = arfq::launch_moe_down(down, h16, hs, rs, off, srt, tiles, nt, max_tiles, ob, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "moe: down launch");
    e = arfq::launch_moe_combine(ob, ids, wts, tokens, top_k, E, hidden, y, accumulate, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "moe: combine launch");
    return ARFQ_OK;
}

static int moe_routed(arfq_ctx *ctx, const arfq_weight *gate, const arfq_weight *up, const arfq_weight *down,
                      const float *router_logits, int64_t tokens, int top_k, int norm_topk, const void *x,
                      int x_dtype, float *y, bool accumulate) {
    if (int rc = check_moe(ctx, gate, up, down, tokens, top_k, x, x_dtype, y)) return rc;
    if (tokens > 0 && !router_logits) return fail(ctx, ARFQ_E_INVALID, "moe: null router logits");
    if (int rc = use_device(ctx)) return rc;
    return moe_enqueue(ctx, gate, up, down, router_logits, nullptr, nullptr, tokens, top_k, norm_topk, x,
                       x_dtype, y, accumulate);
}

static int moe_given(arfq_ctx *ctx, const arfq_weight *gate, const arfq_weight *up, const arfq_weight *down,
                     const int32_t *ids, const float *weights, int64_t tokens, int top_k, const void *x,
                     int x_dtype, float *y, bool accumulate) {
    if (int rc = check_moe(ctx, gate, up, down, tokens, top_k, x, x_dtype, y)) return rc;
    if (tokens > 0 && (!ids || !weights)) return fail(ctx, ARFQ_E_INVALID, "moe_ids: null ids or weights");
    if (int rc = use_device(ctx)) return rc;
    return moe_enqueue(ctx, gate, up, down, nullptr, ids, weights, tokens, top_k, 0, x, x_dtype, y, accumulate);
}

int arfq_moe(arfq_ctx *ctx, const arfq_weight *gate, const arfq_weight *up,
             const arfq_weight *down, const float *router_logits, int64_t tokens, int top_k,
             int norm_topk, const void *x, int x_dtype, float *y) {
    return moe_routed(ctx, gate, up, down, router_logits, tokens, top_k, norm_topk, x, x_dtype, y, false);
}

int arfq_moe_add(arfq_ctx *ctx, const arfq_weight *gate, const arfq_weight *up,
                 const arfq_weight *down, const float *router_logits, int64_t tokens, int top_k,
                 int norm_topk, const void *x, int x_dtype, float *y) {
    return moe_routed(ctx, gate, up, down, router_logits, tokens, top_k, norm_topk, x, x_dtype, y, true);
}

int arfq_moe_ids(arfq_ctx *ctx, const arfq_weight *gate, const arfq_weight *up,
                 const arfq_weight *down, const int32_t *ids, const float *weights,
                 int64_t tokens, int top_k, const void *x, int x_dtype, float *y) {
    return moe_given(ctx, gate, up, down, ids, weights, tokens, top_k, x, x_dtype, y, false);
}

int arfq_moe_ids_add(arfq_ctx *ctx, const arfq_weight *gate, const arfq_weight *up,
                     const arfq_weight *down, const int32_t *ids, const float *weights,
                     int64_t tokens, int top_k, const void *x, int x_dtype, float *y) {
    return moe_given(ctx, gate, up, down, ids, weights, tokens, top_k, x, x_dtype, y, true);
}

// -------------------------------------------------------------------- FFN ----

// Scratch bytes a matmul of w at m rows needs (GEMM plans; the GEMV needs none).
static size_t matmul_scratch(const arfq_weight *w, int64_t m, bool x16) {
    if (arfq::gemv_supports(w, m, x16)) return 0;
    return arfq::gemm_supports(w, m) ? arfq::gemm_plan(w, m, ARFQ_F32, x16).scratch_bytes : 0;
}

int arfq_ffn_act(arfq_ctx *ctx, const arfq_weight *gate, const arfq_weight *up, const arfq_weight *down,
                 int64_t m, const float *x, float *y, int act) {
    if (!ctx) return ARFQ_E_INVALID;
    if (act != ARFQ_ACT_SILU && act != ARFQ_ACT_GELU_TANH) return fail(ctx, ARFQ_E_INVALID, "ffn: unknown activation");
    if (!gate || !up || !down) return fail(ctx, ARFQ_E_INVALID, "ffn: null weight");
    if (m < 0) return fail(ctx, ARFQ_E_SHAPE, "ffn: m < 0");
    if (m > 0 && (!x || !y)) return fail(ctx, ARFQ_E_INVALID, "ffn: null x or y");
    if (gate->experts != 1 || up->experts != 1 || down->experts != 1)
        return fail(ctx, ARFQ_E_SHAPE, "ffn: expert-stacked weights (use arfq_moe)");
    if (up->n != gate->n || up->k != gate->k || down->n != gate->k || down->k != gate->n)
        return fail(ctx, ARFQ_E_SHAPE, "ffn: want gate/up [inter, hidden] and down [hidden, inter]");
    if (m == 0) return ARFQ_OK;
    if (int rc = use_device(ctx)) return rc;
    const int64_t inter = gate->n;
    const bool x16 = (ctx->options & ARFQ_OPT_GEMV_X16) != 0;
    // gate and up of one x row in one launch (Q4_K, f32 arithmetic)
    const bool dual = !x16 && arfq::gemv_dual_supports(gate, up, m);
    // the activation applied as the down GEMV reads its x (Q4_K, m <= 4)
    const bool fused = arfq::gemv_glu_supports(down, m, x16);
    // the GEMM plans use the scratch from offset 0; g, u (and h) sit above the largest
    size_t base = std::max({matmul_scratch(gate, m, x16), matmul_scratch(up, m, x16),
                            fused ? (size_t)0 : matmul_scratch(down, m, x16)});
    base = align256(base);
    const size_t gb = align256((size_t)m * inter * 4);
    if (int rc = ensure_scratch(ctx, base + (fused ? 2 : 3) * gb)) return rc;
    char *sc = (char *)ctx->scratch;
    float *g = (float *)(sc + base), *u = (float *)(sc + base + gb), *h = (float *)(sc + base + 2 * gb);
    hipError_t e;
    if (dual) {
        e = arfq::launch_gemv_dual(gate, up, x, g, u, ctx->stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "ffn: gate/up GEMV launch");
    } else {
        if (int rc = matmul_enqueue(ctx, gate, 0, m, x, ARFQ_F32, g)) return rc;
        if (int rc = matmul_enqueue(ctx, up, 0, m, x, ARFQ_F32, u)) return rc;
    }
    if (fused) {
        e = arfq::launch_gemv_glu(down, m, g, u, y, act, ctx->stream, x16);
        if (e != hipSuccess) return hip_fail(ctx, e, "ffn: down GEMV launch");
        return ARFQ_OK;
    }
    e = arfq::launch_glu(g, u, h, m * inter, act, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "ffn: activation launch");
    return matmul_enqueue(ctx, down, 0, m, h, ARFQ_F32, y);
}

int arfq_ffn(arfq_ctx *ctx, const arfq_weight *gate, const arfq_weight *up, const arfq_weight *down,
             int64_t m, const float *x, float *y) {
    return arfq_ffn_act(ctx, gate, up, down, m, x, y, ARFQ_ACT_SILU);
}

int arfq_dequant_f32(arfq_ctx *ctx, const arfq_weight *w, float *out) {
    if (!ctx) return ARFQ_E_INVALID;
    if (!w || !out) return fail(ctx, ARFQ_E_INVALID, "dequant: null argument");
    if (int rc = use_device(ctx)) return rc;
    hipError_t e = arfq::launch_dequant(w, out, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "dequant launch");
    return ARFQ_OK;
}

// ---------------------------------------------------------------- helpers ----

int arfq_dev_malloc(arfq_ctx *ctx, size_t bytes, void **out) {
    if (!ctx || !out) return fail(ctx, ARFQ_E_INVALID, "dev_malloc: null argument");
    if (int rc = use_device(ctx)) return rc;
    hipError_t e = hipMalloc(out, bytes ? bytes : 1);
    if (e != hipSuccess) return fail(ctx, ARFQ_E_NOMEM, std::string("hipMalloc: ") + hipGetErrorString(e));
    return ARFQ_OK;
}

int arfq_dev_free(arfq_ctx *ctx, void *p) {
    if (!ctx) return ARFQ_E_INVALID;
    if (int rc = use_device(ctx)) return rc;
    HIP_TRY(ctx, hipFree(p));
    return ARFQ_OK;
}

int arfq_copy_h2d(arfq_ctx *ctx, void *dst, const void *src, size_t bytes) {
    if (!ctx || (!dst && bytes) || (!src && bytes)) return fail(ctx, ARFQ_E_INVALID, "copy_h2d: null");
    if (int rc = use_device(ctx)) return rc;
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    HIP_TRY(ctx, hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return ARFQ_OK;
}

int arfq_copy_d2h(arfq_ctx *ctx, void *dst, const void *src, size_t bytes) {
    if (!ctx || (!dst && bytes) || (!src && bytes)) return fail(ctx, ARFQ_E_INVALID, "copy_d2h: null");
    if (int rc = use_device(ctx)) return rc;
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    HIP_TRY(ctx, hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return ARFQ_OK;
}

// One 16-byte load and store per lane, grid-stride.
__global__ void copy16_kernel(const uint4 *__restrict__ src, uint4 *__restrict__ dst, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        dst[i] = src[i];
}

int arfq_copy_d2d(arfq_ctx *ctx, void *dst, const void *src, size_t bytes) {
    if (!ctx || (!dst && bytes) || (!src && bytes)) return fail(ctx, ARFQ_E_INVALID, "copy_d2d: null");
    if (int rc = use_device(ctx)) return rc;
    if (bytes == 0) return ARFQ_OK;
    if ((((uintptr_t)dst | (uintptr_t)src | bytes) & 15) == 0) {
        const int64_t n = (int64_t)(bytes / 16);
        const int64_t want = (n + 255) / 256;
        const unsigned grid = (unsigned)std::min<int64_t>(want, (int64_t)std::max(ctx->cus, 1) * 16);
        copy16_kernel<<<grid, 256, 0, ctx->stream>>>((const uint4 *)src, (uint4 *)dst, n);
        HIP_TRY(ctx, hipGetLastError());
    } else {
        HIP_TRY(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
    }
    return ARFQ_OK;
}

// Read-only stream: grid-stride 16-byte loads, folded into one word per lane
// that is stored only if it holds an unlikely value (so the loads cannot be
// dropped).  Wave 0 of workgroups < nstamps records (s_memrealtime,
// s_memtime) at its start and end.
__global__ __launch_bounds__(256) void read_stream_kernel(const uint4 *__restrict__ src, int64_t n,
                                                          uint32_t *__restrict__ sink, uint64_t *__restrict__ stamps,
                                                          int nstamps) {
    const uint64_t r0 = __builtin_amdgcn_s_memrealtime(), c0 = __builtin_readcyclecounter();
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    uint32_t acc = 0;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const uint4 a = arfq::ld_nt(src + i);
        acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    if (acc == 0x9E3779B9u) sink[threadIdx.x] = acc;
    if (stamps && threadIdx.x == 0 && (int)blockIdx.x < nstamps) {
        const uint64_t r1 = __builtin_amdgcn_s_memrealtime(), c1 = __builtin_readcyclecounter();
        uint64_t *o = stamps + 4 * (int64_t)blockIdx.x;
        o[0] = r0;
        o[1] = c0;
        o[2] = r1;
        o[3] = c1;
    }
}

int arfq_stream_read(arfq_ctx *ctx, const void *src, size_t bytes, uint64_t *stamps, int nstamps) {
    if (!ctx) return ARFQ_E_INVALID;
    if (!src || (((uintptr_t)src | bytes) & 15)) return fail(ctx, ARFQ_E_INVALID, "stream_read: need 16-byte alignment");
    if (nstamps < 0 || (nstamps > 0 && !stamps)) return fail(ctx, ARFQ_E_INVALID, "stream_read: bad stamps");
    if (int rc = use_device(ctx)) return rc;
    if (bytes == 0) return ARFQ_OK;
    // the sink (a word per thread of a workgroup) is the start of the context's
    // aux words; nothing reads it
    if (!ctx->aux) return fail(ctx, ARFQ_E_DEVICE, "stream_read: no sink");
    const int64_t n = (int64_t)(bytes / 16);
    // eight 256-thread workgroups per CU (fewer for a short stream: a load per lane at least)
    const unsigned grid = (unsigned)std::min<int64_t>((n + 255) / 256, (int64_t)std::max(ctx->cus, 1) * 8);
    read_stream_kernel<<<grid, 256, 0, ctx->stream>>>((const uint4 *)src, n, ctx->aux, stamps, nstamps);
    HIP_TRY(ctx, hipGetLastError());
    return ARFQ_OK;
}

int arfq_ctx_device_info(arfq_ctx *ctx, int *cus, int *shader_clock_khz, int *wall_clock_khz) {
    if (!ctx) return ARFQ_E_INVALID;
    if (cus) *cus = ctx->cus;
    if (shader_clock_khz) HIP_TRY(ctx, hipDeviceGetAttribute(shader_clock_khz, hipDeviceAttributeClockRate, ctx->device));
    if (wall_clock_khz)
        HIP_TRY(ctx, hipDeviceGetAttribute(wall_clock_khz, hipDeviceAttributeWallClockRate, ctx->device));
    return ARFQ_OK;
}

int arfq_ctx_memory(arfq_ctx *ctx, size_t *scratch_bytes, size_t *device_free, size_t *device_total) {
    if (!ctx) return ARFQ_E_INVALID;
    if (scratch_bytes) *scratch_bytes = ctx->scratch_bytes;
    if (device_free || device_total) {
        if (int rc = use_device(ctx)) return rc;
        size_t f = 0, t = 0;
        HIP_TRY(ctx, hipMemGetInfo(&f, &t));
        if (device_free) *device_free = f;
        if (device_total) *device_total = t;
    }
    return ARFQ_OK;
}

int arfq_timer_start(arfq_ctx *ctx) {
    if (!ctx) return ARFQ_E_INVALID;
    if (int rc = use_device(ctx)) return rc;
    HIP_TRY(ctx, hipEventRecord(ctx->ev_start, ctx->stream));
    return ARFQ_OK;
}

int arfq_timer_stop(arfq_ctx *ctx, float *ms) {
    if (!ctx || !ms) return fail(ctx, ARFQ_E_INVALID, "timer_stop: null");
    if (int rc = use_device(ctx)) return rc;
    HIP_TRY(ctx, hipEventRecord(ctx->ev_stop, ctx->stream));
    HIP_TRY(ctx, hipEventSynchronize(ctx->ev_stop));
    HIP_TRY(ctx, hipEventElapsedTime(ms, ctx->ev_start, ctx->ev_stop));
    return ARFQ_OK;
}

}  // extern "C"
