// arfq_dequant.hip -- upload repack (raw ggml blocks -> aligned device streams)
// and the f32 dequant used by arfq_dequant_f32.  Both are one-time / parity
// paths, not hot paths: one thread per block (or per sub-unit), byte reads.
#include "arfq_common.h"
#include "arfq_internal.h"

namespace arfq {

// ---- repack ------------------------------------------------------------------

__global__ void repack_q4k(const uint8_t *__restrict__ raw, uint8_t *__restrict__ hdr,
                           uint8_t *__restrict__ qs, int64_t b0, int64_t nblk) {
    const int64_t lb = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (lb >= nblk) return;
    const int64_t b = b0 + lb;
    const uint8_t *src = raw + lb * 144;
    uint8_t *h = hdr + b * 16;
    for (int i = 0; i < 16; i++) h[i] = src[i];
    // regroup nibbles per sub-block: element 32j+i lives in ggml byte
    // 32*(j/2)+i, low nibble for even j, high nibble for odd j; it goes to
    // dword 4j + i/8, nibble position q4k_sigma_inv(i%8)
    uint32_t *q = reinterpret_cast<uint32_t *>(qs + b * 128);
    for (int j = 0; j < 8; j++) {
        const uint8_t *g = src + 16 + 32 * (j >> 1);
        const int sh = (j & 1) * 4;
        for (int w = 0; w < 4; w++) {
            uint32_t v = 0;
            for (int t = 0; t < 8; t++)
                v |= (uint32_t)((g[8 * w + t] >> sh) & 0xF) << (4 * q4k_sigma_inv(t));
            q[4 * j + w] = v;
        }
    }
}

__global__ void repack_q80(const uint8_t *__restrict__ raw, uint8_t *__restrict__ qs,
                           uint16_t *__restrict__ d, int64_t b0, int64_t nblk) {
    const int64_t lb = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (lb >= nblk) return;
    const int64_t b = b0 + lb;
    const uint8_t *src = raw + lb * 34;
    d[b] = (uint16_t)(src[0] | (src[1] << 8));
    uint8_t *q = qs + b * 32;
    for (int i = 0; i < 32; i++) q[i] = src[2 + i];
}

__global__ void repack_q6k(const uint8_t *__restrict__ raw, uint8_t *__restrict__ qb,
                           uint8_t *__restrict__ sc, uint16_t *__restrict__ d, int64_t b0, int64_t nblk,
                           uint32_t *__restrict__ wide) {
    const int64_t lb = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (lb >= nblk) return;
    const int64_t b = b0 + lb;
    const uint8_t *src = raw + lb * 210;
    const uint8_t *ql = src, *qh = src + 128;
    uint8_t *dst = qb + b * 192;
    for (int c = 0; c < 4; c++) {
        const int n2 = c >> 1, l0 = 16 * (c & 1);
        uint8_t *o = dst + 48 * c;
        for (int i = 0; i < 16; i++) {
            o[i] = ql[64 * n2 + l0 + i];
            o[16 + i] = ql[64 * n2 + 32 + l0 + i];
            o[32 + i] = qh[32 * n2 + l0 + i];
        }
    }
    int amax = 0;
    for (int i = 0; i < 16; i++) {
        sc[b * 16 + i] = src[192 + i];
        const int v = (int8_t)src[192 + i];
        amax = max(amax, v < 0 ? -v : v);
    }
    d[b] = (uint16_t)(src[208] | (src[209] << 8));
    // the prefill GEMM splits sc * (q - 32) into hi + lo past 64, the skinny
    // kernel scales each sub-block in f32 past 62
    if (wide && amax > 64) wide[0] = 1u;
    if (wide && amax > 62) wide[1] = 1u;
}

// Q5_K: the 16-byte header (d, dmin, scales) and ggml's qh[32] + qs[128] as they are.
__global__ void repack_q5k(const uint8_t *__restrict__ raw, uint8_t *__restrict__ hdr,
                           uint8_t *__restrict__ q, int64_t b0, int64_t nblk) {
    const int64_t lb = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (lb >= nblk) return;
    const int64_t b = b0 + lb;
    const uint8_t *src = raw + lb * 176;
    for (int i = 0; i < 16; i++) hdr[b * 16 + i] = src[i];
    for (int i = 0; i < 160; i++) q[b * 160 + i] = src[16 + i];
}

// IQ4_XS: the 8-byte header (d, scales_h, scales_l) and qs[128] as they are.
__global__ void repack_iq4xs(const uint8_t *__restrict__ raw, uint8_t *__restrict__ hdr,
                             uint8_t *__restrict__ qs, int64_t b0, int64_t nblk) {
    const int64_t lb = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (lb >= nblk) return;
    const int64_t b = b0 + lb;
    const uint8_t *src = raw + lb * 136;
    for (int i = 0; i < 8; i++) hdr[b * 8 + i] = src[i];
    for (int i = 0; i < 128; i++) qs[b * 128 + i] = src[8 + i];
}

hipError_t launch_repack(const arfq_weight *w, const uint8_t *raw, hipStream_t s, int64_t b0, int64_t nb,
                         uint32_t *wide) {
    if (nb < 0) nb = w->nblk - b0;
    if (b0 < 0 || nb < 0 || b0 + nb > w->nblk) return hipErrorInvalidValue;
    if (nb == 0) return hipSuccess;
    const int tpb = 256;
    const unsigned grid = (unsigned)((nb + tpb - 1) / tpb);
    switch (w->qtype) {
    case ARFQ_Q4_K:
        repack_q4k<<<grid, tpb, 0, s>>>(raw, (uint8_t *)w->s0, (uint8_t *)w->s1, b0, nb);
        break;
    case ARFQ_Q8_0:
        repack_q80<<<grid, tpb, 0, s>>>(raw, (uint8_t *)w->s0, (uint16_t *)w->s1, b0, nb);
        break;
    case ARFQ_Q6_K:
        repack_q6k<<<grid, tpb, 0, s>>>(raw, (uint8_t *)w->s0, (uint8_t *)w->s1, (uint16_t *)w->s2, b0, nb, wide);
        break;
    case ARFQ_Q5_K:
        repack_q5k<<<grid, tpb, 0, s>>>(raw, (uint8_t *)w->s0, (uint8_t *)w->s1, b0, nb);
        break;
    case ARFQ_IQ4_XS:
        repack_iq4xs<<<grid, tpb, 0, s>>>(raw, (uint8_t *)w->s0, (uint8_t *)w->s1, b0, nb);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---- dequant -----------------------------------------------------------------

// One thread per (block, sub-block j): 32 outputs.
__global__ void dequant_q4k(const uint4 *__restrict__ hdr, const uint32_t *__restrict__ qs,
                            float *__restrict__ out, int64_t nblk) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nblk * 8) return;
    const int64_t b = t >> 3;
    const int j = (int)(t & 7);
    const uint4 h = hdr[b];
    const float d = h2f(h.x), dmin = h2f(h.x >> 16);
    uint32_t sc, m;
    q4k_scale_min(h.y, h.z, h.w, j, sc, m);
    const float d1 = q4k_d1(d, sc);
    const float m1 = q4k_d1(dmin, m);
    const uint32_t *q = qs + b * 32 + j * 4;
    float *o = out + b * 256 + j * 32;
    for (int i = 0; i < 32; i++)
        o[i] = q4k_weight(d1, m1, (q[i >> 3] >> (4 * q4k_sigma_inv(i & 7))) & 0xFu);
}

__global__ void dequant_q80(const int8_t *__restrict__ qs, const uint16_t *__restrict__ d,
                            float *__restrict__ out, int64_t nblk) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblk) return;
    const float dv = h2f(d[b]);
    for (int i = 0; i < 32; i++) out[b * 32 + i] = q80_weight(dv, qs[b * 32 + i]);
}

// One thread per (block, 48-byte chunk c): 64 outputs.
__global__ void dequant_q6k(const uint32_t *__restrict__ qb, const int8_t *__restrict__ sc,
                            const uint16_t *__restrict__ d, float *__restrict__ out,
                            int64_t nblk) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nblk * 4) return;
    const int64_t b = t >> 2;
    const int c = (int)(t & 3);
    uint32_t w[12];
    for (int i = 0; i < 12; i++) w[i] = qb[b * 48 + c * 12 + i];
    const float dv = h2f(d[b]);
    const int n2 = c >> 1, isub = c & 1;
    float *o = out + b * 256 + 128 * n2 + 16 * isub;
    for (int tq = 0; tq < 4; tq++) {
        const int s = sc[b * 16 + 8 * n2 + isub + 2 * tq];
        for (int i = 0; i < 16; i++) o[32 * tq + i] = q6k_weight(dv, s, q6k_code(w, tq, i));
    }
}

// One thread per (block, sub-block j): q = low / high nibble of qs[32 (j / 2) + i]
// | bit j of qh[i] << 4, weight (d * sc) * q - dmin * m as Q4_K
// (crates/arf-core/src/model/gguf.rs:2053-2090).
__global__ void dequant_q5k(const uint4 *__restrict__ hdr, const uint8_t *__restrict__ q,
                            float *__restrict__ out, int64_t nblk) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nblk * 8) return;
    const int64_t b = t >> 3;
    const int j = (int)(t & 7);
    const uint4 h = hdr[b];
    const float d = h2f(h.x), dmin = h2f(h.x >> 16);
    uint32_t sc, m;
    q4k_scale_min(h.y, h.z, h.w, j, sc, m);
    const float d1 = q4k_d1(d, sc);
    const float m1 = q4k_d1(dmin, m);
    const uint8_t *qh = q + b * 160, *qs = qh + 32 + 32 * (j >> 1);
    float *o = out + b * 256 + j * 32;
    for (int i = 0; i < 32; i++)
        o[i] = q4k_weight(d1, m1, ((qs[i] >> (4 * (j & 1))) & 0xFu) | (((qh[i] >> j) & 1u) << 4));
}

// One thread per (block, sub-block j): dl = d * (ls - 32), weight dl * kv with kv
// the codebook value of the nibble (crates/arf-core/src/model/gguf.rs:1937-1976).
__constant__ int8_t IQ4_KV[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                  1,    13,   25,  38,  53,  69,  89,  113};
__global__ void dequant_iq4xs(const uint8_t *__restrict__ hdr, const uint8_t *__restrict__ qs,
                              float *__restrict__ out, int64_t nblk) {
#pragma clang fp contract(off)
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nblk * 8) return;
    const int64_t b = t >> 3;
    const int j = (int)(t & 7);
    const uint8_t *h = hdr + b * 8;
    const float d = h2f((uint32_t)h[0] | ((uint32_t)h[1] << 8));
    const uint32_t sh = (uint32_t)h[2] | ((uint32_t)h[3] << 8);
    const int ls = (int)(((h[4 + j / 2] >> (4 * (j % 2))) & 0xFu) | (((sh >> (2 * j)) & 3u) << 4));
    const float dl = d * (float)(ls - 32);
    const uint8_t *q = qs + b * 128 + 16 * j;
    float *o = out + b * 256 + 32 * j;
    for (int i = 0; i < 16; i++) {
        o[i] = dl * (float)IQ4_KV[q[i] & 0xF];
        o[i + 16] = dl * (float)IQ4_KV[q[i] >> 4];
    }
}

hipError_t launch_dequant(const arfq_weight *w, float *out, hipStream_t s) {
    const int tpb = 256;
    switch (w->qtype) {
    case ARFQ_Q4_K: {
        const unsigned grid = (unsigned)((w->nblk * 8 + tpb - 1) / tpb);
        dequant_q4k<<<grid, tpb, 0, s>>>((const uint4 *)w->s0, (const uint32_t *)w->s1, out,
                                         w->nblk);
        break;
    }
    case ARFQ_Q8_0: {
        const unsigned grid = (unsigned)((w->nblk + tpb - 1) / tpb);
        dequant_q80<<<grid, tpb, 0, s>>>((const int8_t *)w->s0, (const uint16_t *)w->s1, out,
                                         w->nblk);
        break;
    }
    case ARFQ_IQ4_XS: {
        const unsigned grid = (unsigned)((w->nblk * 8 + tpb - 1) / tpb);
        dequant_iq4xs<<<grid, tpb, 0, s>>>((const uint8_t *)w->s0, (const uint8_t *)w->s1, out, w->nblk);
        break;
    }
    case ARFQ_Q5_K: {
        const unsigned grid = (unsigned)((w->nblk * 8 + tpb - 1) / tpb);
        dequant_q5k<<<grid, tpb, 0, s>>>((const uint4 *)w->s0, (const uint8_t *)w->s1, out, w->nblk);
        break;
    }
    case ARFQ_Q6_K: {
        const unsigned grid = (unsigned)((w->nblk * 4 + tpb - 1) / tpb);
        dequant_q6k<<<grid, tpb, 0, s>>>((const uint32_t *)w->s0, (const int8_t *)w->s1,
                                         (const uint16_t *)w->s2, out, w->nblk);
        break;
    }
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace arfq
