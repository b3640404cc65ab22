// arfq_gemv.hip -- decode GEMV kernels (m = 1..4 activation rows) for Q4_K,
// Q8_0 and Q6_K weights.  HBM-bound: every weight byte is read exactly once,
// with 128-bit loads, and unpacked in registers.
//
// Thread mapping (all three formats):
//   * one workgroup = one wave64 = two half-waves; half-wave h owns R
//     consecutive output rows;
//   * lane ll (0..31) of a half-wave owns one fixed chunk position inside a
//     block (Q4_K: 16 B of qs = 32 nibbles; Q8_0: 16 B = half a block; Q6_K:
//     one 48-B chunk = 64 codes) and strides over blocks;
//   * the lane loads the x values matching its chunk once per block and reuses
//     them for its R rows (so x traffic is 1/R of the weight traffic through
//     L1), keeps R partial sums, and the half-wave reduces them at the end.
// Reference behaviour: matmul_vec_q4ks_msl.metal:46-165 (simdgroup strides
// sub-blocks, s*sum(q*x) + lo*sum(x) per sub-block, simd_sum), and the oracle
// dot_q4ks (crates/arf-ml/src/matmul.rs:327-358), matmul_nt_q8_0 (:174-204).
#include "arfq_common.h"
#include "arfq_internal.h"

namespace arfq {

namespace {

__device__ __forceinline__ float half_wave_sum(float v) {
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 8);
    v += __shfl_xor(v, 4);
    v += __shfl_xor(v, 2);
    v += __shfl_xor(v, 1);
    return v;
}

__device__ __forceinline__ void load16(const float *p, float *v) {
    const float4 *q = reinterpret_cast<const float4 *>(p);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 t = q[i];
        v[4 * i] = t.x;
        v[4 * i + 1] = t.y;
        v[4 * i + 2] = t.z;
        v[4 * i + 3] = t.w;
    }
}

__device__ __forceinline__ float sum16(const float *v) {
    float a = 0.f, b = 0.f, c = 0.f, d = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
        a += v[i];
        b += v[i + 1];
        c += v[i + 2];
        d += v[i + 3];
    }
    return (a + b) + (c + d);
}

// sum_t x[t] * byte_t(w_i) over 4 dwords whose bytes are small unsigned codes.
__device__ __forceinline__ float dot16_u8(const float *x, uint32_t w0, uint32_t w1, uint32_t w2,
                                          uint32_t w3) {
    const uint32_t w[4] = {w0, w1, w2, w3};
    float a[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        a[0] = fmaf(x[4 * i + 0], (float)(w[i] & 0xffu), a[0]);
        a[1] = fmaf(x[4 * i + 1], (float)((w[i] >> 8) & 0xffu), a[1]);
        a[2] = fmaf(x[4 * i + 2], (float)((w[i] >> 16) & 0xffu), a[2]);
        a[3] = fmaf(x[4 * i + 3], (float)(w[i] >> 24), a[3]);
    }
    return (a[0] + a[1]) + (a[2] + a[3]);
}

// sum_t x[t] * sbyte_t(w_i) for signed i8 codes.
__device__ __forceinline__ float dot16_i8(const float *x, uint4 q) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    float a[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
        for (int j = 0; j < 4; j++)
            a[j] = fmaf(x[4 * i + j], (float)(int8_t)((w[i] >> (8 * j)) & 0xffu), a[j]);
    }
    return (a[0] + a[1]) + (a[2] + a[3]);
}

}  // namespace

// ------------------------------------------------------------------ Q4_K ----
// Lane chunk c (0..7) of a block = qs bytes [16c, 16c+16): group p = c/2 of
// 32 bytes, half hh = c%2.  Low nibble of byte t -> element 64p + 16hh + t
// (sub-block 2p); high nibble -> element 64p + 32 + 16hh + t (sub-block 2p+1).
template <int R, int MX>
__global__ __launch_bounds__(64) void gemv_q4k(const uint4 *__restrict__ hdr,
                                               const uint4 *__restrict__ qs,
                                               const float *__restrict__ x, float *__restrict__ y,
                                               int n, int nblk, int m) {
    const int lane = threadIdx.x;
    const int half = lane >> 5, ll = lane & 31;
    const int c = ll & 7, bq = ll >> 3;
    const int p = c >> 1, hh = c & 1;
    const int64_t row0 = ((int64_t)blockIdx.x * 2 + half) * R;
    const int64_t k = (int64_t)nblk * 256;
    // which header bytes hold sub-blocks 2p, 2p+1 (ggml get_scale_min_k4)
    const bool low = p < 2;
    const int i0 = (2 * p) & 3, i1 = (2 * p + 1) & 3;

    float acc[MX][R];
#pragma unroll
    for (int mi = 0; mi < MX; mi++)
#pragma unroll
        for (int r = 0; r < R; r++) acc[mi][r] = 0.f;

    for (int b = bq; b < nblk; b += 4) {
        uint4 hv[R], qv[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            int64_t row = row0 + r;
            row = row < n ? row : n - 1;  // clamped rows are computed and discarded
            const int64_t blk = row * nblk + b;
            hv[r] = hdr[blk];
            qv[r] = ld_nt(qs + blk * 8 + c);
        }
        float sl[R], sh[R], ml[R], mh[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float d = h2f(hv[r].x), dmin = h2f(hv[r].x >> 16);
            const uint32_t A0 = byte_of(hv[r].y, i0), B0 = byte_of(hv[r].z, i0),
                           C0 = byte_of(hv[r].w, i0);
            const uint32_t A1 = byte_of(hv[r].y, i1), B1 = byte_of(hv[r].z, i1),
                           C1 = byte_of(hv[r].w, i1);
            const uint32_t sc0 = low ? (A0 & 63u) : ((C0 & 15u) | ((A0 >> 6) << 4));
            const uint32_t m0 = low ? (B0 & 63u) : ((C0 >> 4) | ((B0 >> 6) << 4));
            const uint32_t sc1 = low ? (A1 & 63u) : ((C1 & 15u) | ((A1 >> 6) << 4));
            const uint32_t m1 = low ? (B1 & 63u) : ((C1 >> 4) | ((B1 >> 6) << 4));
            sl[r] = d * (float)sc0;
            sh[r] = d * (float)sc1;
            ml[r] = dmin * (float)m0;
            mh[r] = dmin * (float)m1;
        }
#pragma unroll
        for (int mi = 0; mi < MX; mi++) {
            if (mi < m) {
                const float *xb = x + mi * k + (int64_t)b * 256 + 64 * p + 16 * hh;
                float xl[16], xh[16];
                load16(xb, xl);
                load16(xb + 32, xh);
                const float sxl = sum16(xl), sxh = sum16(xh);
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const uint4 q = qv[r];
                    const float dl = dot16_u8(xl, q.x & 0x0F0F0F0Fu, q.y & 0x0F0F0F0Fu,
                                              q.z & 0x0F0F0F0Fu, q.w & 0x0F0F0F0Fu);
                    const float dh =
                        dot16_u8(xh, (q.x >> 4) & 0x0F0F0F0Fu, (q.y >> 4) & 0x0F0F0F0Fu,
                                 (q.z >> 4) & 0x0F0F0F0Fu, (q.w >> 4) & 0x0F0F0F0Fu);
                    acc[mi][r] += (sl[r] * dl + sh[r] * dh) - (ml[r] * sxl + mh[r] * sxh);
                }
            }
        }
    }
#pragma unroll
    for (int mi = 0; mi < MX; mi++) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float v = half_wave_sum(acc[mi][r]);
            const int64_t row = row0 + r;
            if (ll == 0 && mi < m && row < n) y[(int64_t)mi * n + row] = v;
        }
    }
}

// ------------------------------------------------------------------ Q8_0 ----
// Lane chunk c (0..1) = codes [16c, 16c+16) of a 32-weight block.
template <int R, int MX>
__global__ __launch_bounds__(64) void gemv_q80(const uint4 *__restrict__ qs,
                                               const uint16_t *__restrict__ dd,
                                               const float *__restrict__ x, float *__restrict__ y,
                                               int n, int nblk, int m) {
    const int lane = threadIdx.x;
    const int half = lane >> 5, ll = lane & 31;
    const int c = ll & 1, bq = ll >> 1;
    const int64_t row0 = ((int64_t)blockIdx.x * 2 + half) * R;
    const int64_t k = (int64_t)nblk * 32;
    float acc[MX][R];
#pragma unroll
    for (int mi = 0; mi < MX; mi++)
#pragma unroll
        for (int r = 0; r < R; r++) acc[mi][r] = 0.f;

    for (int b = bq; b < nblk; b += 16) {
        uint4 qv[R];
        float dv[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            int64_t row = row0 + r;
            row = row < n ? row : n - 1;
            const int64_t blk = row * nblk + b;
            qv[r] = ld_nt(qs + blk * 2 + c);
            dv[r] = h2f(dd[blk]);
        }
#pragma unroll
        for (int mi = 0; mi < MX; mi++) {
            if (mi < m) {
                float xv[16];
                load16(x + mi * k + (int64_t)b * 32 + 16 * c, xv);
#pragma unroll
                for (int r = 0; r < R; r++) acc[mi][r] += dv[r] * dot16_i8(xv, qv[r]);
            }
        }
    }
#pragma unroll
    for (int mi = 0; mi < MX; mi++) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float v = half_wave_sum(acc[mi][r]);
            const int64_t row = row0 + r;
            if (ll == 0 && mi < m && row < n) y[(int64_t)mi * n + row] = v;
        }
    }
}

// ------------------------------------------------------------------ Q6_K ----
// Lane chunk c (0..3) of a block: 48 B = ql_a[16] | ql_b[16] | qh[16]; code i of
// quadrant t is element 128*(c/2) + 16*(c%2) + 32t + i, scale sc[8*(c/2) + c%2 + 2t].
template <int R, int MX>
__global__ __launch_bounds__(64) void gemv_q6k(const uint4 *__restrict__ qb,
                                               const uint32_t *__restrict__ scw,
                                               const uint16_t *__restrict__ dd,
                                               const float *__restrict__ x, float *__restrict__ y,
                                               int n, int nblk, int m) {
    const int lane = threadIdx.x;
    const int half = lane >> 5, ll = lane & 31;
    const int c = ll & 3, bq = ll >> 2;
    const int n2 = c >> 1, isub = c & 1;
    const int64_t row0 = ((int64_t)blockIdx.x * 2 + half) * R;
    const int64_t k = (int64_t)nblk * 256;
    float acc[MX][R];
#pragma unroll
    for (int mi = 0; mi < MX; mi++)
#pragma unroll
        for (int r = 0; r < R; r++) acc[mi][r] = 0.f;

    for (int b = bq; b < nblk; b += 8) {
        uint4 w0[R], w1[R], w2[R];
        float st[R][4];
#pragma unroll
        for (int r = 0; r < R; r++) {
            int64_t row = row0 + r;
            row = row < n ? row : n - 1;
            const int64_t blk = row * nblk + b;
            const uint4 *src = qb + blk * 12 + c * 3;
            w0[r] = ld_nt(src);
            w1[r] = ld_nt(src + 1);
            w2[r] = ld_nt(src + 2);
            // scales 8*n2 + isub + 2t, t = 0..3 -> bytes of dwords 2*n2 and 2*n2+1
            const uint32_t s_lo = scw[blk * 4 + 2 * n2], s_hi = scw[blk * 4 + 2 * n2 + 1];
            const float d = h2f(dd[blk]);
            st[r][0] = d * (float)(int8_t)(s_lo >> (8 * isub));
            st[r][1] = d * (float)(int8_t)(s_lo >> (8 * (isub + 2)));
            st[r][2] = d * (float)(int8_t)(s_hi >> (8 * isub));
            st[r][3] = d * (float)(int8_t)(s_hi >> (8 * (isub + 2)));
        }
#pragma unroll
        for (int mi = 0; mi < MX; mi++) {
            if (mi < m) {
                const float *xb = x + mi * k + (int64_t)b * 256 + 128 * n2 + 16 * isub;
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    float xv[16];
                    load16(xb + 32 * t, xv);
                    const float sx = sum16(xv);
#pragma unroll
                    for (int r = 0; r < R; r++) {
                        const uint32_t qa[4] = {w0[r].x, w0[r].y, w0[r].z, w0[r].w};
                        const uint32_t qbb[4] = {w1[r].x, w1[r].y, w1[r].z, w1[r].w};
                        const uint32_t qh[4] = {w2[r].x, w2[r].y, w2[r].z, w2[r].w};
                        uint32_t cw[4];
#pragma unroll
                        for (int j = 0; j < 4; j++) {
                            const uint32_t ql = (t & 1) ? qbb[j] : qa[j];
                            const uint32_t nib = (t & 2) ? ((ql >> 4) & 0x0F0F0F0Fu)
                                                         : (ql & 0x0F0F0F0Fu);
                            cw[j] = nib | (((qh[j] >> (2 * t)) & 0x03030303u) << 4);
                        }
                        const float dq = dot16_u8(xv, cw[0], cw[1], cw[2], cw[3]);
                        // sum x*(q-32) = sum x*q - 32*sum x
                        acc[mi][r] += st[r][t] * (dq - 32.f * sx);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int mi = 0; mi < MX; mi++) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float v = half_wave_sum(acc[mi][r]);
            const int64_t row = row0 + r;
            if (ll == 0 && mi < m && row < n) y[(int64_t)mi * n + row] = v;
        }
    }
}

// ---------------------------------------------------------------- launch ----
constexpr int GEMV_MAX_M = 4;

bool gemv_supports(const arfq_weight *w, int64_t m) {
    return m >= 1 && m <= GEMV_MAX_M &&
           (w->qtype == ARFQ_Q4_K || w->qtype == ARFQ_Q8_0 || w->qtype == ARFQ_Q6_K);
}

template <int R, int MX>
static hipError_t launch_gemv_t(const arfq_weight *w, int e, int m, const float *x, float *y,
                                hipStream_t s) {
    const int n = (int)w->n;
    const unsigned grid = (unsigned)((n + 2 * R - 1) / (2 * R));
    const int qk = qk_of(w->qtype);
    const int nblk = (int)(w->k / qk);
    const int64_t eb = (int64_t)e * w->n * nblk;  // first block of expert e
    switch (w->qtype) {
    case ARFQ_Q4_K:
        gemv_q4k<R, MX><<<grid, 64, 0, s>>>((const uint4 *)w->s0 + eb,
                                            (const uint4 *)w->s1 + eb * 8, x, y, n, nblk, m);
        break;
    case ARFQ_Q8_0:
        gemv_q80<R, MX><<<grid, 64, 0, s>>>((const uint4 *)w->s0 + eb * 2,
                                            (const uint16_t *)w->s1 + eb, x, y, n, nblk, m);
        break;
    case ARFQ_Q6_K:
        gemv_q6k<R, MX><<<grid, 64, 0, s>>>((const uint4 *)w->s0 + eb * 12,
                                            (const uint32_t *)w->s1 + eb * 4,
                                            (const uint16_t *)w->s2 + eb, x, y, n, nblk, m);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gemv(const arfq_weight *w, int e, int64_t m, const float *x, float *y,
                       hipStream_t s) {
    if (!gemv_supports(w, m)) return hipErrorInvalidValue;
    if (m == 1) return launch_gemv_t<4, 1>(w, e, 1, x, y, s);
    if (m == 2) return launch_gemv_t<4, 2>(w, e, 2, x, y, s);
    return launch_gemv_t<2, 4>(w, e, (int)m, x, y, s);
}

}  // namespace arfq
