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

#include <algorithm>

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
// Integer-dot GEMV.  x is quantized per 32-element block to 16-bit fixed point
// (X = rint(x * 2^(15-e)), e = exponent of the block's max |x|, clamped to
// +-32767; Xu = X + 32768), held in LDS as 4 nibble digits per element, so
// each 32-weight sub-block's sum(q * Xu) is 16 v_dot8_u32_u4 over its four
// code dwords, plus 4 more for sum(q):
//     sum(q*x) = 2^(e-15) * (sum_d 16^d sum(q*digit_d) - 32768*sum(q))   (exact int32)
// and the sub-block contributes  (d*sc) * that - (dmin*m) * sum(x)  as in the
// oracle's dot_q4ks (crates/arf-ml/src/matmul.rs:327-358).  The quantization
// error is at most 2^-15 of the block's max |x| per element (~1e-5 of the
// output's rms).
//
// Work split (persistent, balanced): one 1024-thread workgroup per CU, so x is
// quantized once per CU.  Workgroup w owns rows [w*n/G, (w+1)*n/G).  A "step"
// is one row x 4 consecutive blocks; the workgroup's 32 half-wave groups take
// equal contiguous ranges of its steps (a row may be split between adjacent
// groups; those partials are added in LDS in group order, so the result is
// deterministic).  Lane ll of a group owns sub-block j = ll%8 of block
// 4s + ll/8 of step s and keeps PF steps of code/header loads in flight,
// across row boundaries.  Each lane loads one dword of the block header (dword
// j%4) and gets the other three from its 8-lane block group with ds_swizzle.

namespace {

// DPP quad_perm move (lanes within a quad).
template <int P>
__device__ __forceinline__ float quad_perm(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), P, 0xf, 0xf, true));
}
constexpr int QP_XOR1 = 0xB1;  // [1,0,3,2]
constexpr int QP_XOR2 = 0x4E;  // [2,3,0,1]

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, true));
}

// Sum over the 32 lanes of a half-wave, result in every lane: DPP within
// 16-lane rows (xor 1, xor 2, half-row mirror, row mirror), then a swizzle
// that swaps the two rows of the half-wave.
__device__ __forceinline__ float half_wave_sum_dpp(float v) {
    v += dpp<QP_XOR1>(v);
    v += dpp<QP_XOR2>(v);
    v += dpp<0x141>(v);  // row_half_mirror
    v += dpp<0x140>(v);  // row_mirror
    v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1F | (0x10 << 10)));
    return v;
}

// Quantize `m` rows of x[k] (k = 32*nsub) into LDS:
//   dg (uint4) [(row*4 + q)*nsub + u] = digits 0..3 of Xu for elements 8q..8q+7
//        of x-block u; in each digit dword nibble position p holds element
//        8q + q4k_sigma(p), matching the Q4_K code dwords;
//   xs [row*nsub + u] = (2^(e-15), sum of the block).
// 4 threads per x-block (8 elements each; a quad reduces max|x| and the sum).
// xq_load() fetches one round (blockDim.x items) so the caller can put the
// first round's x loads in flight ahead of its weight loads.
struct XqRound {
    float4 v0, v1;
};

__device__ __forceinline__ XqRound xq_load(const float *__restrict__ x, int items, int base) {
    const int it = base + (int)threadIdx.x;
    XqRound r;
    r.v0 = make_float4(0.f, 0.f, 0.f, 0.f);
    r.v1 = r.v0;
    if (it < items) {
        const float4 *src = reinterpret_cast<const float4 *>(x) + (int64_t)it * 2;
        r.v0 = src[0];
        r.v1 = src[1];
    }
    return r;
}

__device__ __forceinline__ void xq_process(const XqRound &r, int items, int base, int nsub,
                                           uint4 *dg, float2 *xs) {
    const int it = base + (int)threadIdx.x;
    const float4 v0 = r.v0, v1 = r.v1;
    float amax = fmaxf(fmaxf(fmaxf(fabsf(v0.x), fabsf(v0.y)), fmaxf(fabsf(v0.z), fabsf(v0.w))),
                       fmaxf(fmaxf(fabsf(v1.x), fabsf(v1.y)), fmaxf(fabsf(v1.z), fabsf(v1.w))));
    float sum = ((v0.x + v0.y) + (v0.z + v0.w)) + ((v1.x + v1.y) + (v1.z + v1.w));
    amax = fmaxf(amax, quad_perm<QP_XOR1>(amax));
    sum += quad_perm<QP_XOR1>(sum);
    amax = fmaxf(amax, quad_perm<QP_XOR2>(amax));
    sum += quad_perm<QP_XOR2>(sum);
    const int ex = (amax > 0.f) ? __builtin_amdgcn_frexp_expf(amax) : 0;
    const float vv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    uint32_t xu[8];
#pragma unroll
    for (int t = 0; t < 8; t++) {
        float q = rintf(ldexpf(vv[t], 15 - ex));
        q = fminf(fmaxf(q, -32767.f), 32767.f);
        xu[t] = (uint32_t)((int)q + 32768);
    }
    // pairs of 16-bit values, then low / high bytes of elements 0..3 and 4..7
    const uint32_t P0 = xu[0] | (xu[1] << 16), P1 = xu[2] | (xu[3] << 16);
    const uint32_t P2 = xu[4] | (xu[5] << 16), P3 = xu[6] | (xu[7] << 16);
    const uint32_t L0 = __builtin_amdgcn_perm(P1, P0, 0x06040200u);
    const uint32_t H0 = __builtin_amdgcn_perm(P1, P0, 0x07050301u);
    const uint32_t L1 = __builtin_amdgcn_perm(P3, P2, 0x06040200u);
    const uint32_t H1 = __builtin_amdgcn_perm(P3, P2, 0x07050301u);
    // byte i of each digit dword: element i (low nibble), element 4+i (high)
    const uint4 D = make_uint4((L0 & 0x0F0F0F0Fu) | ((L1 & 0x0F0F0F0Fu) << 4),
                               ((L0 >> 4) & 0x0F0F0F0Fu) | (L1 & 0xF0F0F0F0u),
                               (H0 & 0x0F0F0F0Fu) | ((H1 & 0x0F0F0F0Fu) << 4),
                               ((H0 >> 4) & 0x0F0F0F0Fu) | (H1 & 0xF0F0F0F0u));
    if (it < items) {
        const int u = it >> 2, q = it & 3;
        const int row = u / nsub, ub = u - row * nsub;
        dg[(row * 4 + q) * nsub + ub] = D;
        if (q == 0) xs[u] = make_float2(ldexpf(1.f, ex - 15), sum);
    }
}

// (d*sc_j, dmin*m_j) of sub-block j from a Q4_K header (ggml get_scale_min_k4,
// crates/arf-ml/src/weight.rs:1353-1365), branch-free for a lane-dependent j:
// two v_perm gather byte j%4 of scales[0..3], scales[4..7], scales[8..11] into
// D = [A, B, C, 0]; then
//   j < 4:  sc = A & 63,                 m = B & 63
//   j >= 4: sc = (C & 15) | (A>>6)<<4,   m = (C >> 4) | (B>>6)<<4
// are each two bit-field extracts (width 0 yields 0) and a shift-or.
struct Q4kLane {
    uint32_t sel1, sel2;          // v_perm selectors
    uint32_t o1, w1, o2, w2;      // sc = bfe(D,o1,w1) | bfe(D,o2,w2) << 4
    uint32_t o3, w3, o4, w4;      // m  = bfe(D,o3,w3) | bfe(D,o4,w4) << 4
};

__device__ __forceinline__ Q4kLane q4k_lane(int j) {
    const uint32_t i = (uint32_t)(j & 3);
    Q4kLane L;
    L.sel1 = i | ((4u + i) << 8) | (0x0Cu << 16) | (0x0Cu << 24);
    L.sel2 = 0u | (1u << 8) | ((4u + i) << 16) | (0x0Cu << 24);
    if (j < 4) {
        L.o1 = 0; L.w1 = 6; L.o2 = 0; L.w2 = 0;
        L.o3 = 8; L.w3 = 6; L.o4 = 0; L.w4 = 0;
    } else {
        L.o1 = 16; L.w1 = 4; L.o2 = 6; L.w2 = 2;
        L.o3 = 20; L.w3 = 4; L.o4 = 14; L.w4 = 2;
    }
    return L;
}

__device__ __forceinline__ void q4k_sub_scales(const uint4 h, const Q4kLane &L, float &d1,
                                               float &m1) {
    const uint32_t T = __builtin_amdgcn_perm(h.z, h.y, L.sel1);
    const uint32_t D = __builtin_amdgcn_perm(h.w, T, L.sel2);
    const uint32_t sc = __builtin_amdgcn_ubfe(D, L.o1, L.w1) | (__builtin_amdgcn_ubfe(D, L.o2, L.w2) << 4);
    const uint32_t mm = __builtin_amdgcn_ubfe(D, L.o3, L.w3) | (__builtin_amdgcn_ubfe(D, L.o4, L.w4) << 4);
    d1 = h2f(h.x) * (float)sc;
    m1 = h2f(h.x >> 16) * (float)mm;
}

// sum(q * x) / 2^(e-15) for one 32-weight sub-block: codes c (4 dwords), digits D0..D3.
__device__ __forceinline__ int q4k_subdot(const uint4 c, const uint4 D0, const uint4 D1,
                                          const uint4 D2, const uint4 D3) {
    uint32_t a0, a1, a2, a3, sq;
    a0 = __builtin_amdgcn_udot8(c.x, D0.x, 0u, false);
    a1 = __builtin_amdgcn_udot8(c.x, D0.y, 0u, false);
    a2 = __builtin_amdgcn_udot8(c.x, D0.z, 0u, false);
    a3 = __builtin_amdgcn_udot8(c.x, D0.w, 0u, false);
    sq = __builtin_amdgcn_udot8(c.x, 0x11111111u, 0u, false);
    a0 = __builtin_amdgcn_udot8(c.y, D1.x, a0, false);
    a1 = __builtin_amdgcn_udot8(c.y, D1.y, a1, false);
    a2 = __builtin_amdgcn_udot8(c.y, D1.z, a2, false);
    a3 = __builtin_amdgcn_udot8(c.y, D1.w, a3, false);
    sq = __builtin_amdgcn_udot8(c.y, 0x11111111u, sq, false);
    a0 = __builtin_amdgcn_udot8(c.z, D2.x, a0, false);
    a1 = __builtin_amdgcn_udot8(c.z, D2.y, a1, false);
    a2 = __builtin_amdgcn_udot8(c.z, D2.z, a2, false);
    a3 = __builtin_amdgcn_udot8(c.z, D2.w, a3, false);
    sq = __builtin_amdgcn_udot8(c.z, 0x11111111u, sq, false);
    a0 = __builtin_amdgcn_udot8(c.w, D3.x, a0, false);
    a1 = __builtin_amdgcn_udot8(c.w, D3.y, a1, false);
    a2 = __builtin_amdgcn_udot8(c.w, D3.z, a2, false);
    a3 = __builtin_amdgcn_udot8(c.w, D3.w, a3, false);
    sq = __builtin_amdgcn_udot8(c.w, 0x11111111u, sq, false);
    // |result| <= 32*15*32767 < 2^24: exact in int32 and in f32
    return (int)(a0 + (a1 << 4) + (a2 << 8) + (a3 << 12)) - (int)(sq << 15);
}

// header dwords 0..3 of the lane's block from the 8-lane block group
// (ds_swizzle bitmask mode: source lane = (lane & 0x18) | k within 32 lanes)
__device__ __forceinline__ uint4 q4k_gather_header(uint32_t v) {
    return make_uint4((uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x18 | (0 << 5)),
                      (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x18 | (1 << 5)),
                      (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x18 | (2 << 5)),
                      (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x18 | (3 << 5)));
}

}  // namespace

constexpr int Q4K_GEMV_THREADS = 1024;
constexpr int Q4K_GEMV_GROUPS = Q4K_GEMV_THREADS / 32;
constexpr int Q4K_GEMV_PF = 4;  // steps of loads in flight per lane

// Work split: one 1024-thread workgroup per CU (x is quantized once per CU);
// workgroup w owns rows [w*n/G, (w+1)*n/G).  Inside it, rows are handed out
// dynamically: each of the 32 half-wave groups claims whole rows from an LDS
// counter (so waves that the hardware serves faster take more rows and the
// workgroup's tail is at most one row).  A group streams a row as spr = nblk/4
// "steps" of 4 blocks; lane ll owns sub-block j = ll%8 of block 4s + ll/8, and
// the group keeps PF steps of code/header loads in flight across row
// boundaries (the next row is claimed when the load ring reaches it).  Each
// lane loads one dword of the block header (dword j%4) and gets the other
// three from its 8-lane block group with ds_swizzle.
template <int MX, int PF = Q4K_GEMV_PF>
__global__ __launch_bounds__(Q4K_GEMV_THREADS) void gemv_q4k(
    const uint4 *__restrict__ hdr, const uint4 *__restrict__ qs, const float *__restrict__ x,
    float *__restrict__ y, int n, int nblk, int m) {
    extern __shared__ uint4 smem4[];
    const int nsub = nblk * 8;
    uint4 *dg = smem4;
    float2 *xs = reinterpret_cast<float2 *>(smem4 + (size_t)MX * 4 * nsub);
    __shared__ int next_row;

    const int tid = threadIdx.x;
    const int ll = tid & 31;
    const int g = tid >> 5;
    const int j = ll & 7, bq = ll >> 3;
    const Q4kLane L = q4k_lane(j);
    const uint32_t *hdr32 = reinterpret_cast<const uint32_t *>(hdr);

    const int G = gridDim.x;
    const int r0 = (int)((int64_t)blockIdx.x * n / G);
    const int r1 = (int)((int64_t)(blockIdx.x + 1) * n / G);
    const int spr = (nblk + 3) >> 2;  // steps per row

    if (tid == 0) next_row = r0 + Q4K_GEMV_GROUPS;
    __syncthreads();
    // claim the next row of this workgroup (-1 when none is left); lane 0 of
    // the half-wave does the LDS atomic, a swizzle broadcasts it
    auto claim = [&]() -> int {
        int r = 0;
        if (ll == 0) r = atomicAdd(&next_row, 1);
        r = __builtin_amdgcn_ds_swizzle(r, 0x00);  // source lane = lane & ~31
        return r < r1 ? r : -1;
    };

    // issue pointer: row irow (absolute, -1 = done), step is.  Loads are
    // issued unconditionally (clamped addresses once the rows run out) so the
    // compiler keeps PF steps in flight with counted waits.
    int irow = r0 + g < r1 ? r0 + g : -1, is = 0;
    uint4 cbuf[PF];
    uint32_t hbuf[PF];
    int srow[PF], sstep[PF];
    auto issue = [&](int u) {
        const int b = min(4 * is + bq, nblk - 1);
        const int row = irow >= 0 ? irow : r0;
        const int64_t blk = (int64_t)row * nblk + b;
        cbuf[u] = ld_nt(qs + blk * 8 + j);
        hbuf[u] = hdr32[blk * 4 + (j & 3)];
        srow[u] = irow;
        sstep[u] = is;
        if (irow >= 0 && ++is == spr) {
            is = 0;
            irow = claim();
        }
    };

    // x first (it gates the compute), then the weight ring, then quantize
    const int xitems = m * nsub * 4;
    const XqRound xr0 = xq_load(x, xitems, 0);
#pragma unroll
    for (int u = 0; u < PF; u++) issue(u);
    xq_process(xr0, xitems, 0, nsub, dg, xs);
    for (int base = Q4K_GEMV_THREADS; base < xitems; base += Q4K_GEMV_THREADS)
        xq_process(xq_load(x, xitems, base), xitems, base, nsub, dg, xs);
    __syncthreads();

    float acc[MX];
#pragma unroll
    for (int mi = 0; mi < MX; mi++) acc[mi] = 0.f;
    bool more = srow[0] >= 0;
    while (more) {
#pragma unroll
        for (int u = 0; u < PF; u++) {
            const int row = srow[u], st = sstep[u];
            if (row < 0) {
                more = false;  // uniform within the group; later slots are empty too
                break;
            }
            const uint4 c = cbuf[u];
            const uint4 h = q4k_gather_header(hbuf[u]);
            issue(u);
            const int b = 4 * st + bq;
            float d1, m1;
            q4k_sub_scales(h, L, d1, m1);
            const int ub = min(b, nblk - 1) * 8 + j;
#pragma unroll
            for (int mi = 0; mi < MX; mi++) {
                if (mi < m) {
                    const uint4 *dp = dg + (size_t)mi * 4 * nsub + ub;
                    const float2 sx = xs[mi * nsub + ub];
                    const int S = q4k_subdot(c, dp[0], dp[nsub], dp[2 * nsub], dp[3 * nsub]);
                    const float part = d1 * (sx.x * (float)S) - m1 * sx.y;
                    acc[mi] += b < nblk ? part : 0.f;
                }
            }
            if (st == spr - 1) {
#pragma unroll
                for (int mi = 0; mi < MX; mi++) {
                    const float v = half_wave_sum_dpp(acc[mi]);
                    acc[mi] = 0.f;
                    if (ll == 0 && mi < m) y[(int64_t)mi * n + row] = v;
                }
            }
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

// LDS the Q4_K GEMV needs for the quantized x of m rows (digits + scale/sum).
static size_t q4k_gemv_lds(int64_t m, int64_t k) { return (size_t)m * (k / 32) * (16 * 4 + 8); }

bool gemv_supports(const arfq_weight *w, int64_t m) {
    if (m < 1 || m > GEMV_MAX_M) return false;
    if (w->qtype == ARFQ_Q4_K) return q4k_gemv_lds(m <= 2 ? m : 4, w->k) <= 60 * 1024;
    return w->qtype == ARFQ_Q8_0 || w->qtype == ARFQ_Q6_K;
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
        return hipErrorInvalidValue;  // handled by launch_gemv_q4k
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

template <int MX>
static hipError_t launch_gemv_q4k(const arfq_weight *w, int e, int m, const float *x, float *y,
                                  hipStream_t s) {
    const int n = (int)w->n, nblk = (int)(w->k / 256);
    const int64_t eb = (int64_t)e * w->n * nblk;
    const int64_t steps = (int64_t)n * ((nblk + 3) / 4);
    const int cus = w->ctx->cus > 0 ? w->ctx->cus : 256;
    // one workgroup per CU; small problems get fewer (>= 4 steps per group)
    int64_t grid = std::min<int64_t>(cus, (steps + 4 * Q4K_GEMV_GROUPS - 1) / (4 * Q4K_GEMV_GROUPS));
    if (grid < 1) grid = 1;
    const size_t lds = q4k_gemv_lds(MX, w->k);
    gemv_q4k<MX><<<(unsigned)grid, Q4K_GEMV_THREADS, lds, s>>>(
        (const uint4 *)w->s0 + eb, (const uint4 *)w->s1 + eb * 8, x, y, n, nblk, m);
    return hipGetLastError();
}

hipError_t launch_gemv(const arfq_weight *w, int e, int64_t m, const float *x, float *y,
                       hipStream_t s) {
    if (!gemv_supports(w, m)) return hipErrorInvalidValue;
    if (w->qtype == ARFQ_Q4_K) {
        if (m == 1) return launch_gemv_q4k<1>(w, e, 1, x, y, s);
        if (m == 2) return launch_gemv_q4k<2>(w, e, 2, x, y, s);
        return launch_gemv_q4k<4>(w, e, (int)m, x, y, s);
    }
    if (m == 1) return launch_gemv_t<4, 1>(w, e, 1, x, y, s);
    if (m == 2) return launch_gemv_t<4, 2>(w, e, 2, x, y, s);
    return launch_gemv_t<2, 4>(w, e, (int)m, x, y, s);
}

}  // namespace arfq
