// arfq_gemm.hip -- dequant-into-LDS MFMA GEMM (prefill / batched decode).
#include "arfq_common.h"
#include "arfq_internal.h"

namespace arfq {

bool gemm_supports(const arfq_weight *, int64_t) { return false; }

hipError_t launch_gemm(const arfq_weight *, int, int64_t, const void *, int, float *, hipStream_t) {
    return hipErrorInvalidValue;
}

__global__ void f32_to_f16_kernel(const float *__restrict__ x, __half *__restrict__ y, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = __float2half_rn(x[i]);
}

hipError_t launch_f32_to_f16(const float *x, __half *y, int64_t n, hipStream_t s) {
    const unsigned grid = (unsigned)((n + 255) / 256);
    f32_to_f16_kernel<<<grid, 256, 0, s>>>(x, y, n);
    return hipGetLastError();
}

}  // namespace arfq
