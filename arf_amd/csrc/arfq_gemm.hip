// arfq_gemm.hip -- dequant-into-LDS MFMA GEMM for prefill and batched decode:
// y[m, n] (f32) = x[m, k] (f16) . W[n, k]^T with W in Q4_K.
//
// Tile: 128 (x rows) x 128 (weight rows) per 256-thread workgroup, K in steps
// of 64 (two Q4_K sub-blocks).  Each step the workgroup
//   * loads the f16 x tile (128 x 64) with 16-byte loads,
//   * loads one 16-byte code chunk (32 nibbles) + the header of 128 weight rows
//     x 2 sub-blocks, dequantizes them to f16 ((d*sc)*q - dmin*m in f32, then
//     round-to-nearest to f16) and stores both tiles in LDS (double buffered,
//     rows padded by 16 bytes so 16-byte LDS reads are conflict-free),
//   * runs 16 v_mfma_f32_32x32x16_f16 per wave (each wave owns 64 x 64 of the
//     output) with f32 accumulation.
// The next step's global loads are issued before the current step's MFMAs.
// Reference behaviour: matmul_mm_q4ks.metal:65-290 (dequant a weight tile into
// threadgroup memory, simdgroup MMA, f32 accumulation); oracle matmul_nt_q4ks
// (crates/arf-ml/src/matmul.rs:363-400) on x widened to f32.
//
// Workgroup -> tile order is XCD-aware: the dispatcher places workgroup b on
// XCD b % 8, so XCD x is given a fixed pair of x tiles (2 x 1.3 MB at k=5120,
// which stays in its L2) and walks all weight tiles, which stream from the
// 256 MB MALL (each weight tile is used twice in a row).
#include "arfq_common.h"
#include "arfq_internal.h"

namespace arfq {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int GM_BM = 128, GM_BN = 128, GM_BK = 64, GM_THREADS = 256;
constexpr int GM_LD = GM_BK + 8;  // halves per LDS row (16 bytes of padding)
constexpr int GM_TILE = GM_BM * GM_LD;
constexpr size_t GM_LDS = 2 * 2 * GM_TILE * sizeof(_Float16);

__device__ __forceinline__ uint32_t pack2h(float a, float b) {
    const __half ha = __float2half_rn(a), hb = __float2half_rn(b);
    return (uint32_t)__half_as_ushort(ha) | ((uint32_t)__half_as_ushort(hb) << 16);
}

__global__ __launch_bounds__(GM_THREADS) void gemm_q4k_f16(
    const uint4 *__restrict__ hdr, const uint4 *__restrict__ qs, const _Float16 *__restrict__ x,
    float *__restrict__ y, int M, int N, int nblk, int mt, int nt, int xcd_order) {
    extern __shared__ _Float16 lds[];
    const int K = nblk * 256;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;

    // tile of this workgroup
    int tm, tn;
    {
        const int b = blockIdx.x;
        if (xcd_order) {
            const int xcd = b & 7, q = b >> 3, per = mt >> 3;
            tm = xcd * per + q % per;
            tn = q / per;
        } else {
            tm = b % mt;
            tn = b / mt;
        }
    }
    const int m0 = tm * GM_BM, n0 = tn * GM_BN;

    // ---- global -> register staging
    // x: 4 x 16 B per thread: row (tid>>3) + 32*i, 8 halves at column 8*(tid&7)
    const int xr = tid >> 3, xc = (tid & 7) * 8;
    // W: weight row n0 + (tid>>1), sub-block 2p + (tid&1) of the current block
    const int wr = tid >> 1, ws = tid & 1;
    const int wrow = min(n0 + wr, N - 1);
    const uint4 *qrow = qs + (int64_t)wrow * nblk * 8;
    const uint4 *hrow = hdr + (int64_t)wrow * nblk;

    uint4 xv[4], cv, hv;
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int row = m0 + xr + 32 * i;
            if (row < M)
                xv[i] = *reinterpret_cast<const uint4 *>(x + (int64_t)row * K + k0 + xc);
            else
                xv[i] = make_uint4(0, 0, 0, 0);
        }
        const int b = k0 >> 8, p = (k0 >> 6) & 3;
        cv = qrow[b * 8 + 2 * p + ws];
        hv = hrow[b];
    };
    auto lstore = [&](int buf, int k0) {
        _Float16 *As = lds + buf * 2 * GM_TILE;
        _Float16 *Bs = As + GM_TILE;
#pragma unroll
        for (int i = 0; i < 4; i++)
            *reinterpret_cast<uint4 *>(As + (xr + 32 * i) * GM_LD + xc) = xv[i];
        // dequantize 32 weights of sub-block j = 2p + ws
        const int j = 2 * ((k0 >> 6) & 3) + ws;
        uint32_t sc, mm;
        q4k_scale_min(hv.y, hv.z, hv.w, j, sc, mm);
        const float d1 = h2f(hv.x) * (float)sc;
        const float m1 = h2f(hv.x >> 16) * (float)mm;
        const uint32_t cw[4] = {cv.x, cv.y, cv.z, cv.w};
        uint32_t o[16];
#pragma unroll
        for (int w = 0; w < 4; w++) {
            // dword w: byte i low nibble = element 8w+i, high nibble = element 8w+4+i
            const uint32_t lo = cw[w] & 0x0F0F0F0Fu, hi = (cw[w] >> 4) & 0x0F0F0F0Fu;
            const float e0 = fmaf(d1, (float)(lo & 0xffu), -m1);
            const float e1 = fmaf(d1, (float)((lo >> 8) & 0xffu), -m1);
            const float e2 = fmaf(d1, (float)((lo >> 16) & 0xffu), -m1);
            const float e3 = fmaf(d1, (float)(lo >> 24), -m1);
            const float e4 = fmaf(d1, (float)(hi & 0xffu), -m1);
            const float e5 = fmaf(d1, (float)((hi >> 8) & 0xffu), -m1);
            const float e6 = fmaf(d1, (float)((hi >> 16) & 0xffu), -m1);
            const float e7 = fmaf(d1, (float)(hi >> 24), -m1);
            o[4 * w + 0] = pack2h(e0, e1);
            o[4 * w + 1] = pack2h(e2, e3);
            o[4 * w + 2] = pack2h(e4, e5);
            o[4 * w + 3] = pack2h(e6, e7);
        }
        uint4 *dst = reinterpret_cast<uint4 *>(Bs + wr * GM_LD + 32 * ws);
#pragma unroll
        for (int q = 0; q < 4; q++) dst[q] = make_uint4(o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]);
    };

    floatx16 acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
            for (int i = 0; i < 16; i++) acc[a][b][i] = 0.f;

    const int nk = K / GM_BK;
    gload(0);
    lstore(0, 0);
    __syncthreads();
    const int lr = lane & 31, lk = (lane >> 5) * 8;
    for (int it = 0; it < nk; it++) {
        const int buf = it & 1;
        if (it + 1 < nk) gload((it + 1) * GM_BK);
        const _Float16 *As = lds + buf * 2 * GM_TILE;
        const _Float16 *Bs = As + GM_TILE;
#pragma unroll
        for (int kk = 0; kk < GM_BK / 16; kk++) {
            half8 af[2], bf[2];
#pragma unroll
            for (int t = 0; t < 2; t++) {
                af[t] = *reinterpret_cast<const half8 *>(As + (wm * 64 + 32 * t + lr) * GM_LD + 16 * kk + lk);
                bf[t] = *reinterpret_cast<const half8 *>(Bs + (wn * 64 + 32 * t + lr) * GM_LD + 16 * kk + lk);
            }
#pragma unroll
            for (int a = 0; a < 2; a++)
#pragma unroll
                for (int b = 0; b < 2; b++)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[a], bf[b], acc[a][b], 0, 0, 0);
        }
        if (it + 1 < nk) lstore(buf ^ 1, (it + 1) * GM_BK);
        __syncthreads();
    }
    // epilogue: lane holds column n = lane%32 of each 32x32 tile, rows 8*(i/4) + 4*(lane/32) + i%4
#pragma unroll
    for (int a = 0; a < 2; a++) {
#pragma unroll
        for (int b = 0; b < 2; b++) {
            const int n = n0 + wn * 64 + 32 * b + lr;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int m = m0 + wm * 64 + 32 * a + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
                if (m < M && n < N) y[(int64_t)m * N + n] = acc[a][b][i];
            }
        }
    }
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

bool gemm_supports(const arfq_weight *w, int64_t m) {
    return w->qtype == ARFQ_Q4_K && m >= 1 && w->n >= 1;
}

hipError_t launch_gemm(const arfq_weight *w, int e, int64_t m, const void *x, int x_dtype, float *y,
                       hipStream_t s) {
    if (w->qtype != ARFQ_Q4_K || x_dtype != ARFQ_F16) return hipErrorInvalidValue;
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t err = hipFuncSetAttribute((const void *)gemm_q4k_f16,
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)GM_LDS);
        if (err != hipSuccess) return err;
        attr_set = true;
    }
    const int nblk = (int)(w->k / 256);
    const int64_t eb = (int64_t)e * w->n * nblk;
    const int mt = (int)((m + GM_BM - 1) / GM_BM), nt = (int)((w->n + GM_BN - 1) / GM_BN);
    const int xcd = (mt % 8 == 0) ? 1 : 0;
    gemm_q4k_f16<<<(unsigned)(mt * nt), GM_THREADS, GM_LDS, s>>>(
        (const uint4 *)w->s0 + eb, (const uint4 *)w->s1 + eb * 8, (const _Float16 *)x, y, (int)m,
        (int)w->n, nblk, mt, nt, xcd);
    return hipGetLastError();
}

}  // namespace arfq
