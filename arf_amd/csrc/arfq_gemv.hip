// arfq_gemv.hip -- decode GEMV kernels (m = 1..4 activation rows).  HBM bound:
// every weight byte is read once, with 128-bit loads, and unpacked in
// registers.
//   * Q4_K, m = 1: gemv_q4k_f32 (f32 x times the exact codes; also the MoE
//     decode pairs and the fused SwiGLU down GEMV); m = 2..4 and the
//     ARFQ_OPT_GEMV_X16 option: gemv_q4k (x in 16-bit fixed point, integer
//     dots).  16-lane groups walk (row, 4-block column) steps handed out from
//     LDS counters.
//   * Q6_K / Q5_K / IQ4_XS: m = 1: gemv_dot_f32<Fmt> (f32 x times the exact
//     codes); m = 2..4 and ARFQ_OPT_GEMV_X16: gemv_dot<Fmt> (x in 16-bit fixed
//     point, integer dots); the same step walk; gemv_q6k is the fallback for
//     shapes neither takes.
//   * Q8_0: gemv_q80w, one wave per row, f32.
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
// output's rms).  The work split is described at gemv_q4k below.

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

// Branch-free: threads past the end re-read the last item (their results are
// not stored), so the number of loads in flight never depends on the data.
__device__ __forceinline__ XqRound xq_load(const float *__restrict__ x, int items, int base) {
    const int it = min(base + (int)threadIdx.x, items - 1);
    const float4 *src = reinterpret_cast<const float4 *>(x) + (int64_t)it * 2;
    XqRound r;
    r.v0 = src[0];
    r.v1 = src[1];
    return r;
}

// x sources of gemv_q4k: a row-major f32 x (the plain GEMV), act(g) * u of the
// FFN's gate and up outputs (XsGlu: the down GEMV with the gated activation
// applied as it reads its x), and for the MoE decode path one row per (token,
// expert) pair: the token's f32 or f16 row, or silu(g) * u of the pair's gate
// and up rows (the same expression as the grouped path's gate|up kernel).
struct XsF32 {
    const float *x;
    __device__ XqRound load(int items, int base) const { return xq_load(x, items, base); }
};
struct XsRowF32 {
    const float *x;
    int64_t stride;
    int div;  // pair p reads row p / div
    __device__ void pair(int p) { x += (int64_t)(p / div) * stride; }
    __device__ XqRound load(int items, int base) const { return xq_load(x, items, base); }
};
struct XsRowF16 {
    const _Float16 *x;
    int64_t stride;
    int div;
    __device__ void pair(int p) { x += (int64_t)(p / div) * stride; }
    __device__ XqRound load(int items, int base) const {
        const int it = min(base + (int)threadIdx.x, items - 1);
        typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
        const f16x8 h = reinterpret_cast<const f16x8 *>(x)[it];
        XqRound r;
        r.v0 = make_float4((float)h[0], (float)h[1], (float)h[2], (float)h[3]);
        r.v1 = make_float4((float)h[4], (float)h[5], (float)h[6], (float)h[7]);
        return r;
    }
};
template <int ACT>
struct XsGlu {
    const float *g, *u;
    int64_t stride;
    __device__ void pair(int p) {
        g += (int64_t)p * stride;
        u += (int64_t)p * stride;
    }
    __device__ XqRound load(int items, int base) const {
        const XqRound a = xq_load(g, items, base), b = xq_load(u, items, base);
        XqRound r;
        r.v0 = make_float4(glu<ACT>(a.v0.x, b.v0.x), glu<ACT>(a.v0.y, b.v0.y), glu<ACT>(a.v0.z, b.v0.z),
                           glu<ACT>(a.v0.w, b.v0.w));
        r.v1 = make_float4(glu<ACT>(a.v1.x, b.v1.x), glu<ACT>(a.v1.y, b.v1.y), glu<ACT>(a.v1.z, b.v1.z),
                           glu<ACT>(a.v1.w, b.v1.w));
        return r;
    }
};
using XsSwiglu = XsGlu<ACT_SILU>;

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

// (d*sc, dmin*m) of sub-blocks jj and jj+4 (jj = 0..3) of a Q4_K block from
// its header dwords h0 = d|dmin, h1 = scales[0..3], h2 = scales[4..7],
// h3 = scales[8..11] (ggml get_scale_min_k4, crates/arf-ml/src/weight.rs:
// 1353-1365): with A, B, C = byte jj of h1, h2, h3,
//   sub-block jj:    sc = A & 63,                 m = B & 63
//   sub-block jj+4:  sc = (C & 15) | (A>>6)<<4,   m = (C >> 4) | (B>>6)<<4
struct PairScales {
    float d_lo, m_lo, d_hi, m_hi;
};

__device__ __forceinline__ PairScales q4k_pair_scales(uint32_t h0, uint32_t h1, uint32_t h2,
                                                      uint32_t h3, uint32_t sh) {
    const uint32_t A = __builtin_amdgcn_ubfe(h1, sh, 8);
    const uint32_t B = __builtin_amdgcn_ubfe(h2, sh, 8);
    const uint32_t C = __builtin_amdgcn_ubfe(h3, sh, 8);
    const float d = h2f(h0), dmin = h2f(h0 >> 16);
    PairScales p;
    p.d_lo = d * (float)(A & 63u);
    p.m_lo = dmin * (float)(B & 63u);
    p.d_hi = d * (float)((C & 15u) | ((A >> 6) << 4));
    p.m_hi = dmin * (float)((C >> 4) | ((B >> 6) << 4));
    return p;
}

// DPP broadcast of lane k of each quad (quad_perm [k,k,k,k]).
template <int K>
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, K * 0x55, 0xf, 0xf, true);
}

// Sum over a 16-lane DPP row, result in every lane of the row.
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp<QP_XOR1>(v);
    v += dpp<QP_XOR2>(v);
    v += dpp<0x141>(v);  // row_half_mirror
    v += dpp<0x140>(v);  // row_mirror
    return v;
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

}  // namespace

constexpr int Q4K_GEMV_THREADS = 512;
constexpr int Q4K_GEMV_WG_PER_CU = 2;
constexpr int Q4K_GEMV_GROUPS = Q4K_GEMV_THREADS / 16;  // 16-lane groups
constexpr int Q4K_GEMV_PF = 2;                          // steps of loads in flight
constexpr int Q4K_GEMV_CHUNK = 2;                       // rows per claimed chunk (divides PF)
constexpr int Q4K_F32_THREADS = 1024;                   // the m = 1 f32 GEMV: one workgroup per CU
constexpr uint32_t Q4K_OOB = 0x80000000u;               // buffer offset past any stream

// Work split: two 512-thread workgroups per CU (x is quantized once per
// workgroup; two independent workgroups per CU measured faster than one of
// 1024 threads); workgroup w owns rows [r0, r1) = [w*n/G, (w+1)*n/G).  (The
// f32 GEMVs differ: rows w, w + G, ..., and x scaled before the first weight
// load; see gemv_q4k_f32_body.  For this kernel, whose x quantization takes
// longer, that order measured slower: C2 with the x16 option 11.6 -> 12.4 us.)
// Each row is cut into
// spr = ceil(nblk/4) "columns" of 4 blocks; a "step" is one (row, column)
// pair.  The steps are handed out in chunks of CHUNK consecutive rows of one
// column: group g starts with chunk g and then claims chunks from an LDS
// counter, so the waves the memory system serves first take more chunks (on
// this hardware the older waves of a CU are served first).  Lane l of a
// 16-lane group serves block 4*column + l/4 of the row and its sub-blocks
// jj = l%4 and jj+4: two 16-B code loads and one header dword (jj), the other
// three header dwords coming from its quad by DPP.  For one x row the x digits
// of the group's current column are held in registers (reloaded from LDS when
// the column changes); for more x rows they are read from LDS.  Each step's
// 16-lane sum is the complete contribution of that (row, column) pair; it goes
// to LDS part[mi][row][column], and at the end every row adds its columns in
// order, so the result does not depend on which group computed what.
//
// Loads are raw buffer loads with 32-bit offsets; an offset past the stream
// (blocks past the row's end, steps past the end of the work) returns zeros
// without touching memory, which contributes exactly 0 (d = 0, q = 0).  Each
// lane keeps PF steps in flight: a slot is consumed and then refilled with the
// next claimed step, in a loop unrolled by PF, so every load lands in the
// registers it is consumed from and the waits are counted ones.
//
// Start-up order matters for the first microseconds: every wave issues its x
// loads (XR rounds of the workgroup, all of them for the shapes the launcher
// sizes XR for), then all waves pass a barrier before any weight load is
// issued (the CU serves requests in issue order, and x gates all compute),
// then x is quantized into LDS and the weight ring starts.
template <int MX, int XR, int PF, class XSRC>
__device__ __forceinline__ void gemv_q4k_body(
    const uint8_t *__restrict__ hdr, uint32_t hdr_bytes, const uint8_t *__restrict__ qs,
    uint32_t qs_bytes, const XSRC &xsrc, float *__restrict__ y, int n, int nblk, int m) {
    constexpr bool XREG = MX == 1;
    constexpr int C = Q4K_GEMV_CHUNK;
    static_assert(PF % C == 0, "claims must sit at fixed slots of the unrolled loop");
    extern __shared__ uint4 smem4[];
    __shared__ int next_chunk;
    const int nsub = nblk * 8;
    uint4 *dg = smem4;
    float2 *xs = reinterpret_cast<float2 *>(smem4 + (size_t)MX * 4 * nsub);
    float *part = reinterpret_cast<float *>(xs + (size_t)MX * nsub);  // [MX][R][spr]

    const __amdgpu_buffer_rsrc_t hrs =
        __builtin_amdgcn_make_buffer_rsrc((void *)hdr, (short)0, (int)hdr_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t qrs =
        __builtin_amdgcn_make_buffer_rsrc((void *)qs, (short)0, (int)qs_bytes, 0x00020000);

    const int tid = threadIdx.x;
    const int l16 = tid & 15, grp = tid >> 4;
    const int bq = l16 >> 2, jj = l16 & 3;

    const int G = gridDim.x;
    const int r0 = (int)((int64_t)blockIdx.x * n / G);
    const int r1 = (int)((int64_t)(blockIdx.x + 1) * n / G);
    const int R = r1 - r0;
    const int spr = (nblk + 3) >> 2;
    const int cpc = (R + C - 1) / C;  // chunks per column
    const int nchunks = cpc * spr;

    // issue state: the current step's column and row.  Chunks are exactly C
    // rows (rows past the column's end are empty steps), so a new chunk starts
    // at every C-th issue and the claims sit at fixed places in the unrolled
    // loop instead of behind data-dependent branches.
    int icol = 0, irow = 0;
    auto start_chunk = [&](int k) {
        icol = k < nchunks ? k / cpc : spr;  // spr = no more work
        irow = (k - icol * cpc) * C;
    };
    u32x4 clo[PF], chi[PF];
    uint32_t hbuf[PF];
    int srow[PF], scol[PF];  // step held by each slot
    auto issue = [&](int u, bool first) {
        if (u % C == 0) {
            int k = grp;
            if (!first) {
                if (l16 == 0) k = atomicAdd(&next_chunk, 1);
                k = __builtin_amdgcn_ds_swizzle(k, 0x10);  // lane 0 of each 16-lane group
            }
            start_chunk(k);
        } else {
            irow++;
        }
        const int b = 4 * icol + bq;
        const bool live = icol < spr && irow < R && b < nblk;
        const uint32_t blk = (uint32_t)(r0 + irow) * (uint32_t)nblk + (uint32_t)b;
        const uint32_t oc = live ? blk * 128u + (uint32_t)jj * 16u : Q4K_OOB;
        const uint32_t oh = live ? blk * 16u + (uint32_t)jj * 4u : Q4K_OOB;
        clo[u] = __builtin_amdgcn_raw_buffer_load_b128(qrs, oc, 0, 2);
        chi[u] = __builtin_amdgcn_raw_buffer_load_b128(qrs, oc + 64u, 0, 2);
        hbuf[u] = __builtin_amdgcn_raw_buffer_load_b32(hrs, oh, 0, 0);
        srow[u] = irow;
        scol[u] = icol;
    };

    if (tid == 0) next_chunk = Q4K_GEMV_GROUPS;
    // x loads of every wave, then a barrier, then the first weight loads
    const int xitems = m * nsub * 4;
    XqRound xr[XR];
#pragma unroll
    for (int r = 0; r < XR; r++) xr[r] = xsrc.load(xitems, r * Q4K_GEMV_THREADS);
    __builtin_amdgcn_s_barrier();
    issue(0, true);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < XR; r++)
        if (r * Q4K_GEMV_THREADS < xitems) xq_process(xr[r], xitems, r * Q4K_GEMV_THREADS, nsub, dg, xs);
    for (int base = XR * Q4K_GEMV_THREADS; base < xitems; base += Q4K_GEMV_THREADS)
        xq_process(xsrc.load(xitems, base), xitems, base, nsub, dg, xs);
    __syncthreads();  // x digits and next_chunk are visible from here on
#pragma unroll
    for (int u = 1; u < PF; u++) {
        issue(u, u < C);
        __builtin_amdgcn_sched_barrier(0);
    }

    // x digits of the column being consumed (sub-blocks jj, jj+4)
    int xcol = -1, ub_lo = 0;
    uint4 X[2][4];
    float2 XS[2];
    auto load_x = [&](int col) {
        xcol = col;
        ub_lo = min(4 * col + bq, nblk - 1) * 8 + jj;
        if (XREG) {
#pragma unroll
            for (int h = 0; h < 2; h++) {
#pragma unroll
                for (int d = 0; d < 4; d++) X[h][d] = dg[(size_t)d * nsub + ub_lo + 4 * h];
                XS[h] = xs[ub_lo + 4 * h];
            }
        }
    };
    const uint32_t sh = 8u * (uint32_t)jj;

    auto consume = [&](int u) {
        const int col = scol[u], row = srow[u];
        const bool live = col < spr && row < R;
        if (live && col != xcol) load_x(col);
        const uint32_t hw = hbuf[u];
        const PairScales ps = q4k_pair_scales(quad_bcast<0>(hw), quad_bcast<1>(hw),
                                              quad_bcast<2>(hw), quad_bcast<3>(hw), sh);
        const uint4 cl = make_uint4(clo[u].x, clo[u].y, clo[u].z, clo[u].w);
        const uint4 ch = make_uint4(chi[u].x, chi[u].y, chi[u].z, chi[u].w);
#pragma unroll
        for (int mi = 0; mi < MX; mi++) {
            if (MX == 1 || mi < m) {
                int s_lo, s_hi;
                float2 x_lo, x_hi;
                if (XREG) {
                    s_lo = q4k_subdot(cl, X[0][0], X[0][1], X[0][2], X[0][3]);
                    s_hi = q4k_subdot(ch, X[1][0], X[1][1], X[1][2], X[1][3]);
                    x_lo = XS[0];
                    x_hi = XS[1];
                } else {
                    const uint4 *dp = dg + (size_t)mi * 4 * nsub + ub_lo;
                    s_lo = q4k_subdot(cl, dp[0], dp[nsub], dp[2 * nsub], dp[3 * nsub]);
                    s_hi = q4k_subdot(ch, dp[4], dp[nsub + 4], dp[2 * nsub + 4], dp[3 * nsub + 4]);
                    x_lo = xs[mi * nsub + ub_lo];
                    x_hi = xs[mi * nsub + ub_lo + 4];
                }
                float v = ps.d_lo * (x_lo.x * (float)s_lo) - ps.m_lo * x_lo.y;
                v += ps.d_hi * (x_hi.x * (float)s_hi) - ps.m_hi * x_hi.y;
                v = row16_sum(v);
                if (l16 == 0 && live) part[((size_t)mi * R + row) * spr + col] = v;
            }
        }
    };

    // consume a slot, then refill it (after its codes are used, so the new
    // load lands in the same registers); claims are monotonic, so once slot 0
    // holds no work, neither does any later slot
    while (scol[0] < spr) {
#pragma unroll
        for (int u = 0; u < PF; u++) {
            consume(u);
            issue(u, false);
        }
    }
    __syncthreads();

    // each row adds its columns in order
    for (int t = tid; t < MX * R; t += Q4K_GEMV_THREADS) {
        const int mi = t / R, r = t - mi * R;
        if (mi < m) {
            const float *pr = part + (size_t)t * spr;
            float v = 0.f;
            for (int c = 0; c < spr; c++) v += pr[c];
            y[(int64_t)mi * n + r0 + r] = v;
        }
    }
}

template <int MX, int XR, int PF = Q4K_GEMV_PF>
__global__ __launch_bounds__(Q4K_GEMV_THREADS) void gemv_q4k(
    const uint8_t *__restrict__ hdr, uint32_t hdr_bytes, const uint8_t *__restrict__ qs,
    uint32_t qs_bytes, const float *__restrict__ x, float *__restrict__ y, int n, int nblk,
    int m) {
    gemv_q4k_body<MX, XR, PF>(hdr, hdr_bytes, qs, qs_bytes, XsF32{x}, y, n, nblk, m);
}

// The FFN's down GEMV: x = act(g) * u over m row-major rows (g, u: [m][k]).
template <int MX, int XR, int ACT>
__global__ __launch_bounds__(Q4K_GEMV_THREADS) void gemv_q4k_glu(
    const uint8_t *__restrict__ hdr, uint32_t hdr_bytes, const uint8_t *__restrict__ qs,
    uint32_t qs_bytes, const float *__restrict__ g, const float *__restrict__ u,
    float *__restrict__ y, int n, int nblk, int m) {
    gemv_q4k_body<MX, XR, Q4K_GEMV_PF>(hdr, hdr_bytes, qs, qs_bytes, XsGlu<ACT>{g, u, 0}, y, n, nblk, m);
}

// ------------------------------------------------- Q4_K, f32 activations ----
// The decode GEMV at the reference's arithmetic (one x row): f32 x times the
// exact 4-bit codes, accumulated in f32 per 32-weight sub-block, then
//     (d*sc) * code_sum - (dmin*m) * x_sum
// as dot_q4ks (crates/arf-ml/src/matmul.rs:327-358) and the reference GEMV
// (shaders/metal/matmul_vec_q4ks_msl.metal:46-165) compute it.  Nothing about
// x is rounded; only the order of the f32 sums differs from the reference.
//
// The product x*q is one v_fma_mix_f32 per weight, its f16 operand taken
// straight from the code dword: masking a dword with 0x000F000F leaves two
// nibbles q as the mantissas of two f16 subnormals, i.e. the exact values
// q * 2^-24 (0x00F000F0 gives 16q * 2^-24).  x is held pre-multiplied by
// 2^24 (2^20 for the high-nibble elements), so each product is exactly x * q.
// Five bit operations unpack eight weights.  A sub-block whose max |x| is
// 2^76 or more is held at 2^s with s < 24 instead, so that x * 2^s stays
// below 2^100, and its code sum is multiplied back by 2^(24 - s).
//
// LDS per x row: the scaled x (k floats, element order) and per sub-block the
// pair (sum of x, 2^(24 - s)).  Work split, loads and the load ring are those
// of gemv_q4k (above); for m = 1 the lane keeps the 64 scaled x of its column's
// two sub-blocks in registers.
namespace {

// One round of x items (8 elements each, a quad per 32-element sub-block) into
// the scaled copy xf (as float4 pairs) and the sub-block pairs xs.
__device__ __forceinline__ void xf_process(const XqRound &r, int items, int base, float4 *xf,
                                           float2 *xs) {
    const int it = base + (int)threadIdx.x;
    const float4 v0 = r.v0, v1 = r.v1;
    float amax = fmaxf(fmaxf(fmaxf(fabsf(v0.x), fabsf(v0.y)), fmaxf(fabsf(v0.z), fabsf(v0.w))),
                       fmaxf(fmaxf(fabsf(v1.x), fabsf(v1.y)), fmaxf(fabsf(v1.z), fabsf(v1.w))));
    float sum = ((v0.x + v0.y) + (v0.z + v0.w)) + ((v1.x + v1.y) + (v1.z + v1.w));
    amax = fmaxf(amax, quad_perm<QP_XOR1>(amax));
    sum += quad_perm<QP_XOR1>(sum);
    amax = fmaxf(amax, quad_perm<QP_XOR2>(amax));
    sum += quad_perm<QP_XOR2>(sum);
    // amax < 2^ex; keep max |x| * 2^s below 2^100
    const int ex = (amax > 0.f) ? __builtin_amdgcn_frexp_expf(amax) : 0;
    const int s = min(24, 100 - ex);
    if (it < items) {
        xf[2 * it] = make_float4(ldexpf(v0.x, s), ldexpf(v0.y, s), ldexpf(v0.z, s), ldexpf(v0.w, s));
        xf[2 * it + 1] = make_float4(ldexpf(v1.x, s - 4), ldexpf(v1.y, s - 4), ldexpf(v1.z, s - 4),
                                     ldexpf(v1.w, s - 4));
        if ((it & 3) == 0) xs[it >> 2] = make_float2(sum, ldexpf(1.f, 24 - s));
    }
}

typedef _Float16 f16x2v __attribute__((ext_vector_type(2)));

// acc + x * h, h the low (H = 0) or high (H = 1) f16 half of w: v_fma_mix_f32
template <int H>
__device__ __forceinline__ float fmix(float x, uint32_t w, float acc) {
    const f16x2v h = __builtin_bit_cast(f16x2v, w);
    return __builtin_fmaf(x, H ? (float)h.y : (float)h.x, acc);
}

// sum_i x_i * q_i over one 32-weight sub-block: code dwords c, scaled x X[32]
// (element order; X[8w + 4..7] carry the extra 2^-4)
__device__ __forceinline__ float q4k_fdot(const uint4 c, const float *X) {
    const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
    float acc = 0.f;
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const uint32_t v = cw[w], t = v >> 8;
        const uint32_t A = v & 0x000F000Fu, B = v & 0x00F000F0u;
        const uint32_t C = t & 0x000F000Fu, D = t & 0x00F000F0u;
        const float *xw = X + 8 * w;
        acc = fmix<0>(xw[0], A, acc);
        acc = fmix<1>(xw[2], A, acc);
        acc = fmix<0>(xw[1], C, acc);
        acc = fmix<1>(xw[3], C, acc);
        acc = fmix<0>(xw[4], B, acc);
        acc = fmix<1>(xw[6], B, acc);
        acc = fmix<0>(xw[5], D, acc);
        acc = fmix<1>(xw[7], D, acc);
    }
    return acc;
}

}  // namespace

// NT threads per workgroup.  x is scaled into LDS before any weight load is
// issued, and workgroup w owns rows w, w + G, w + 2G, ... (G workgroups): the
// whole chip reads a narrow window of the weight stream at a time.
template <int XR, int PF, int NT, class XSRC, bool MASKED = false>
__device__ __forceinline__ void gemv_q4k_f32_body(
    const uint8_t *__restrict__ hdr, uint32_t hdr_bytes, const uint8_t *__restrict__ qs,
    uint32_t qs_bytes, const XSRC &xsrc, float *__restrict__ y, int n, int nblk) {
    constexpr int C = Q4K_GEMV_CHUNK;
    constexpr int GROUPS = NT / 16;
    static_assert(PF % C == 0, "claims must sit at fixed slots of the unrolled loop");
    extern __shared__ uint4 smem4[];
    __shared__ unsigned long long exm;  // columns seen exhausted (spr <= 64)
    const int nsub = nblk * 8;
    const int spr = (nblk + 3) >> 2;
    float4 *xf = reinterpret_cast<float4 *>(smem4);                 // [k / 4]
    float2 *xs = reinterpret_cast<float2 *>(xf + (size_t)nsub * 8);  // [nsub]
    int *cnt = reinterpret_cast<int *>(xs + nsub);                   // [spr] chunk counters
    float *part = reinterpret_cast<float *>(cnt + ((spr + 3) & ~3));  // [R][spr]

    const __amdgpu_buffer_rsrc_t hrs =
        __builtin_amdgcn_make_buffer_rsrc((void *)hdr, (short)0, (int)hdr_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t qrs =
        __builtin_amdgcn_make_buffer_rsrc((void *)qs, (short)0, (int)qs_bytes, 0x00020000);

    const int tid = threadIdx.x;
    const int l16 = tid & 15, grp = tid >> 4;
    const int bq = l16 >> 2, jj = l16 & 3;

    const int G = gridDim.x;
    // rows of this workgroup: r0 + i * G for i < R
    const int r0 = blockIdx.x;
    const int R = (n - r0 + G - 1) / G;
    const int cpc = (R + C - 1) / C;  // chunks (of C rows) per column

    // Each 16-lane group has a home column (group % spr) and starts on chunk
    // group / spr of it; further chunks are claimed from that column's counter,
    // and only when it runs out from the next columns, so a group keeps the x
    // of one column in registers for most of its work.
    int icol = grp % spr, irow = (grp / spr) * C;
    // MASKED (taken past 8 columns, i.e. with more than one round of x at
    // 1024 threads): a group whose column ran out takes the
    // next column not yet seen exhausted (a bit mask; lane 0 decides and
    // claims, the group follows by broadcast).  Trying the next columns one by
    // one costs an LDS atomic round trip per exhausted column: at the FFN's
    // down GEMV (17 columns) 40.2 -> 37.2 us per FFN with the mask (same box);
    // at C2's 5 columns the scan stays (the mask's code there cost 0.3 us).
    auto claim = [&]() {
        int col = icol;
        for (int t = 0; t < spr; t++) {
            int k = 0;
            if constexpr (MASKED) {
                if (l16 == 0) {
                    if (t > 0) {
                        const uint64_t all = spr == 64 ? ~0ull : ((1ull << spr) - 1);
                        const uint64_t av =
                            ~__hip_atomic_load(&exm, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) & all;
                        const uint64_t r = col == 0 ? av : ((av >> col) | (av << (spr - col))) & all;
                        if (r == 0) {
                            col = -1;  // none left
                        } else {
                            col += __builtin_ctzll(r);
                            if (col >= spr) col -= spr;
                        }
                    }
                    if (col >= 0) {
                        k = atomicAdd(&cnt[col], 1);
                        if (k >= cpc) atomicOr(&exm, 1ull << col);
                    }
                }
                col = __builtin_amdgcn_ds_swizzle(col, 0x10);  // lane 0 of each 16-lane group
                k = __builtin_amdgcn_ds_swizzle(k, 0x10);
                if (col < 0) break;
            } else {
                if (l16 == 0) k = atomicAdd(&cnt[col], 1);
                k = __builtin_amdgcn_ds_swizzle(k, 0x10);  // lane 0 of each 16-lane group
            }
            if (k < cpc) {
                icol = col;
                irow = k * C;
                return;
            }
            if constexpr (!MASKED) col = col + 1 == spr ? 0 : col + 1;
        }
        icol = spr;  // no work left
    };
    u32x4 clo[PF], chi[PF];
    uint32_t hbuf[PF];
    int srow[PF], scol[PF];
    auto issue = [&](int u, bool first) {
        if (!first) {
            if (u % C == 0) claim();
            else irow++;
        } else if (u > 0) {
            irow++;
        }
        const int b = 4 * icol + bq;
        const bool live = icol < spr && irow < R && b < nblk;
        const uint32_t blk = (uint32_t)(r0 + irow * G) * (uint32_t)nblk + (uint32_t)b;
        const uint32_t oc = live ? blk * 128u + (uint32_t)jj * 16u : Q4K_OOB;
        const uint32_t oh = live ? blk * 16u + (uint32_t)jj * 4u : Q4K_OOB;
        clo[u] = __builtin_amdgcn_raw_buffer_load_b128(qrs, oc, 0, 2);
        chi[u] = __builtin_amdgcn_raw_buffer_load_b128(qrs, oc + 64u, 0, 2);
        hbuf[u] = __builtin_amdgcn_raw_buffer_load_b32(hrs, oh, 0, 0);
        srow[u] = irow;
        scol[u] = icol;
    };

    // counters start past the chunks the groups begin on
    for (int c = tid; c < spr; c += NT)
        cnt[c] = (GROUPS - c + spr - 1) / spr;
    if (MASKED && tid == 0) exm = 0;
    // x loads, x scaled into LDS, the barrier, then the weights: a wave's
    // loads issue in order and stall once the CU's memory queue is full, and
    // every CU's weight requests delay the x requests, so x issued alone
    // arrives 2-3 us earlier at C2's shape than behind the first weights.
    const int xitems = nsub * 4;
    XqRound xr[XR];
#pragma unroll
    for (int r = 0; r < XR; r++) xr[r] = xsrc.load(xitems, r * NT);
    asm volatile("" ::: "memory");  // keep the x loads ahead of everything after them
    // (every round is processed: items past the end load a clamped index and
    // store nothing, and an unconditional use keeps the loads where they are)
#pragma unroll
    for (int r = 0; r < XR; r++) xf_process(xr[r], xitems, r * NT, xf, xs);
    for (int base = XR * NT; base < xitems; base += NT)
        xf_process(xsrc.load(xitems, base), xitems, base, xf, xs);
    lds_barrier();  // scaled x and the counters are visible from here on
#pragma unroll
    for (int u = 0; u < PF; u++) issue(u, true);

    // scaled x of the column being consumed (sub-blocks jj, jj + 4)
    int xcol = -1;
    float X[2][32];
    float2 XS[2];
    auto load_x = [&](int col) {
        xcol = col;
        const int ub = min(4 * col + bq, nblk - 1) * 8 + jj;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const float4 *src = xf + (size_t)(ub + 4 * h) * 8;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float4 t = src[i];
                X[h][4 * i] = t.x;
                X[h][4 * i + 1] = t.y;
                X[h][4 * i + 2] = t.z;
                X[h][4 * i + 3] = t.w;
            }
            XS[h] = xs[ub + 4 * h];
        }
    };
    const uint32_t sh = 8u * (uint32_t)jj;

    auto consume = [&](int u) {
        const int col = scol[u], row = srow[u];
        const bool live = col < spr && row < R;
        if (live && col != xcol) load_x(col);
        const uint32_t hw = hbuf[u];
        const PairScales ps = q4k_pair_scales(quad_bcast<0>(hw), quad_bcast<1>(hw),
                                              quad_bcast<2>(hw), quad_bcast<3>(hw), sh);
        const uint4 cl = make_uint4(clo[u].x, clo[u].y, clo[u].z, clo[u].w);
        const uint4 ch = make_uint4(chi[u].x, chi[u].y, chi[u].z, chi[u].w);
        const float s_lo = q4k_fdot(cl, X[0]) * XS[0].y;
        const float s_hi = q4k_fdot(ch, X[1]) * XS[1].y;
        float v = ps.d_lo * s_lo - ps.m_lo * XS[0].x;
        v += ps.d_hi * s_hi - ps.m_hi * XS[1].x;
        v = row16_sum(v);
        if (l16 == 0 && live) part[(size_t)row * spr + col] = v;
    };

    // consume a slot, then refill it; a group that has run out of work (icol ==
    // spr) stays out, so once slot 0 holds no work neither does any later slot
    while (scol[0] < spr) {
#pragma unroll
        for (int u = 0; u < PF; u++) {
            consume(u);
            issue(u, false);
        }
    }
    lds_barrier();

    for (int t = tid; t < R; t += NT) {
        const float *pr = part + (size_t)t * spr;
        float v = 0.f;
        for (int c = 0; c < spr; c++) v += pr[c];
        y[r0 + t * G] = v;
    }
}

template <int XR>
__global__ __launch_bounds__(Q4K_F32_THREADS) void gemv_q4k_f32(
    const uint8_t *__restrict__ hdr, uint32_t hdr_bytes, const uint8_t *__restrict__ qs,
    uint32_t qs_bytes, const float *__restrict__ x, float *__restrict__ y, int n, int nblk) {
    gemv_q4k_f32_body<XR, Q4K_GEMV_PF, Q4K_F32_THREADS, XsF32, (XR > 1)>(hdr, hdr_bytes, qs, qs_bytes, XsF32{x}, y, n,
                                                        nblk);
}

// The FFN's down GEMV at one x row: x = act(g) * u, f32 arithmetic.
template <int XR, int ACT>
__global__ __launch_bounds__(Q4K_F32_THREADS) void gemv_q4k_f32_glu(
    const uint8_t *__restrict__ hdr, uint32_t hdr_bytes, const uint8_t *__restrict__ qs,
    uint32_t qs_bytes, const float *__restrict__ g, const float *__restrict__ u,
    float *__restrict__ y, int n, int nblk) {
    gemv_q4k_f32_body<XR, Q4K_GEMV_PF, Q4K_F32_THREADS>(hdr, hdr_bytes, qs, qs_bytes, XsGlu<ACT>{g, u, 0}, y,
                                                        n, nblk);
}

// The FFN's gate and up GEMVs in one launch: blockIdx.y = 0 multiplies x by
// the first weight into y0, 1 by the second into y1 (same shape), each
// weight's rows split over gridDim.x workgroups; f32 arithmetic.
template <int XR>
__global__ __launch_bounds__(Q4K_F32_THREADS) void gemv_q4k_f32_dual(
    const uint8_t *__restrict__ hdr0, const uint8_t *__restrict__ qs0, const uint8_t *__restrict__ hdr1,
    const uint8_t *__restrict__ qs1, uint32_t hdr_bytes, uint32_t qs_bytes, const float *__restrict__ x,
    float *__restrict__ y0, float *__restrict__ y1, int n, int nblk) {
    const bool second = blockIdx.y != 0;  // uniform over the workgroup
    gemv_q4k_f32_body<XR, Q4K_GEMV_PF, Q4K_F32_THREADS, XsF32, (XR > 1)>(second ? hdr1 : hdr0, hdr_bytes, second ? qs1 : qs0,
                                                        qs_bytes, XsF32{x}, second ? y1 : y0, n, nblk);
}

// MoE decode: blockIdx.y = pair p, one x row each, the weight of expert ids[p]
// (its n rows split over gridDim.x workgroups) into y row p, at f32
// arithmetic.  A pair whose id is out of range is dropped (its row is not
// written; the combine skips it).
// Reference: the indirect GEMVs gemv_q4ks_id / gemv_q4ks_id_down
// (shaders/metal/gemv_q4ks_id_msl.metal:40-153, gemv_q4ks_id_down_msl.metal:186-275).
template <int XR, class XSRC>
__global__ __launch_bounds__(Q4K_GEMV_THREADS) void gemv_q4k_pairs(
    const uint8_t *__restrict__ hdr, const uint8_t *__restrict__ qs, uint32_t e_hdr_bytes,
    uint32_t e_qs_bytes, XSRC xsrc, float *__restrict__ y, int n, int nblk,
    const int32_t *__restrict__ ids, int E) {
    const int p = blockIdx.y;
    const int e = ids[p];
    if (e < 0 || e >= E) return;  // uniform over the workgroup
    xsrc.pair(p);
    gemv_q4k_f32_body<XR, Q4K_GEMV_PF, Q4K_GEMV_THREADS>(hdr + (int64_t)e * e_hdr_bytes, e_hdr_bytes,
                                       qs + (int64_t)e * e_qs_bytes, e_qs_bytes, xsrc,
                                       y + (int64_t)p * n, n, nblk);
}

// MoE decode, gate and up in one launch: blockIdx.z = 0 multiplies pair p's x
// by expert ids[p]'s first weight into y0 row p, 1 by its second weight (same
// shape) into y1.
template <int XR, class XSRC>
__global__ __launch_bounds__(Q4K_GEMV_THREADS) void gemv_q4k_pairs_dual(
    const uint8_t *__restrict__ hdr0, const uint8_t *__restrict__ qs0, const uint8_t *__restrict__ hdr1,
    const uint8_t *__restrict__ qs1, uint32_t e_hdr_bytes, uint32_t e_qs_bytes, XSRC xsrc,
    float *__restrict__ y0, float *__restrict__ y1, int n, int nblk, const int32_t *__restrict__ ids,
    int E) {
    const int p = blockIdx.y;
    const int e = ids[p];
    if (e < 0 || e >= E) return;  // uniform over the workgroup
    const bool second = blockIdx.z != 0;
    xsrc.pair(p);
    gemv_q4k_f32_body<XR, Q4K_GEMV_PF, Q4K_GEMV_THREADS>((second ? hdr1 : hdr0) + (int64_t)e * e_hdr_bytes, e_hdr_bytes,
                                       (second ? qs1 : qs0) + (int64_t)e * e_qs_bytes, e_qs_bytes, xsrc,
                                       (second ? y1 : y0) + (int64_t)p * n, n, nblk);
}

// --------------------------------------------- Q6_K / Q5_K / IQ4_XS (dot) ----
// Integer-dot GEMV for up to four x rows (gemv_dot<Format, MX, XR>; the
// formats are below).  x is quantized per 32-element
// block to 16-bit fixed point X = rint(x * 2^(15-e)) (as for Q4_K) and held in
// LDS as a low-byte plane (u8) and a high-byte plane (i8, X >> 8), both in
// element order, with the sum of every 16 elements and 2^(e-15) per 32.  A
// 16-element Q6_K sub-block then gives
//     sum(q * X) = 256 * sdot4(q, hi) + udot4(q, lo)    (4 + 4 dots, exact int32)
// and contributes (d*sc) * (2^(e-15) * sum(q*X) - 32 * sum(x)): the oracle's
// (d*sc)*(q-32) per weight (gguf.rs:2120-2123), factorised.
// Work split as gemv_q4k: two 512-thread workgroups per CU, steps = (row,
// column of 4 blocks) claimed in chunks of 2 rows of one column.  Lane l of a
// 16-lane group serves block 4*column + l/4 and its 64 codes c = l%4 (four
// 16-code quadrants); for Q6_K that is its 48-byte chunk c, one scale dword (c)
// whose neighbours come from its quad by DPP, and the block's d.
constexpr int Q6K_GEMV_THREADS = 512;
constexpr int Q6K_GEMV_GROUPS = Q6K_GEMV_THREADS / 16;
constexpr int Q6K_GEMV_PF = 2;
constexpr int Q6K_GEMV_CHUNK = 2;

namespace {

// Quantize one round of x items (8 elements each, 4 per 32-element block) into
// the byte planes: lo/hi [row*k + e], s16 [row*k/16 + e/16], xe [row*k/32 + e/32].
__device__ __forceinline__ void xq6_process(const XqRound &r, int items, int base, int k,
                                            uint8_t *lo, uint8_t *hi, float *s16, float *xe) {
    const int it = base + (int)threadIdx.x;
    const float4 v0 = r.v0, v1 = r.v1;
    float amax = fmaxf(fmaxf(fmaxf(fabsf(v0.x), fabsf(v0.y)), fmaxf(fabsf(v0.z), fabsf(v0.w))),
                       fmaxf(fmaxf(fabsf(v1.x), fabsf(v1.y)), fmaxf(fabsf(v1.z), fabsf(v1.w))));
    float sum = ((v0.x + v0.y) + (v0.z + v0.w)) + ((v1.x + v1.y) + (v1.z + v1.w));
    amax = fmaxf(amax, quad_perm<QP_XOR1>(amax));
    sum += quad_perm<QP_XOR1>(sum);  // 16 elements (items 2i, 2i+1)
    amax = fmaxf(amax, quad_perm<QP_XOR2>(amax));
    const int ex = (amax > 0.f) ? __builtin_amdgcn_frexp_expf(amax) : 0;
    const float vv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    uint32_t L[2] = {0u, 0u}, H[2] = {0u, 0u};
#pragma unroll
    for (int t = 0; t < 8; t++) {
        float q = rintf(ldexpf(vv[t], 15 - ex));
        q = fminf(fmaxf(q, -32767.f), 32767.f);
        const uint32_t xi = (uint32_t)(int)q;
        L[t >> 2] |= (xi & 0xFFu) << (8 * (t & 3));
        H[t >> 2] |= ((xi >> 8) & 0xFFu) << (8 * (t & 3));
    }
    if (it < items) {
        const int e = it * 8;  // element of the flattened [m][k] x
        *reinterpret_cast<u32x2 *>(lo + e) = u32x2{L[0], L[1]};
        *reinterpret_cast<u32x2 *>(hi + e) = u32x2{H[0], H[1]};
        if ((it & 1) == 0) s16[e >> 4] = sum;
        if ((it & 3) == 0) xe[e >> 5] = ldexpf(1.f, ex - 15);
    }
}

// sum(q * X) of one 16-code quadrant: codes cw[4] (one byte each, q < 64),
// planes lo/hi.
__device__ __forceinline__ int q6k_subdot(const uint32_t *cw, const u32x4 lo, const u32x4 hi) {
    uint32_t a = __builtin_amdgcn_udot4(cw[0], lo.x, 0u, false);
    int b = __builtin_amdgcn_sdot4((int)cw[0], (int)hi.x, 0, false);
    a = __builtin_amdgcn_udot4(cw[1], lo.y, a, false);
    b = __builtin_amdgcn_sdot4((int)cw[1], (int)hi.y, b, false);
    a = __builtin_amdgcn_udot4(cw[2], lo.z, a, false);
    b = __builtin_amdgcn_sdot4((int)cw[2], (int)hi.z, b, false);
    a = __builtin_amdgcn_udot4(cw[3], lo.w, a, false);
    b = __builtin_amdgcn_sdot4((int)cw[3], (int)hi.w, b, false);
    // |256 b + a| <= 16 * 63 * 32767 < 2^25: exact in int32 and in f32
    return b * 256 + (int)a;
}

}  // namespace

// Formats of the byte-code dot GEMV.  Lane c (0..3) of a block's quad holds
// 64 codes as four 16-code quadrants t; quadrant t's x elements start at
// xbase(b, c) + XSTEP * t.  codes() builds the quadrant's code bytes, scales()
// the per-quadrant factors, term() the quadrant's contribution from
// sdot = sum(q * X) (X: x in 16-bit fixed point, scale xsc) and xsum = sum(x).
//
// Q6_K: lane c = 48-byte chunk c of the repacked block (ql_a | ql_b | qh, see
// repack_q6k); q = ql nibble | qh bits << 4 (0..63); weight (d * sc) * (q - 32).
struct DotQ6K {
    const uint8_t *qb, *scb, *db;
    uint32_t qb_bytes, sc_bytes, d_bytes;
    struct Res {
        __amdgpu_buffer_rsrc_t q, s, d;
    };
    struct Lane {
        u32x4 q0, q1, q2;
        uint32_t sw, dw;
    };
    static constexpr int XSTEP = 32, PF = Q6K_GEMV_PF;
    __device__ Res res() const {
        return {__builtin_amdgcn_make_buffer_rsrc((void *)qb, (short)0, (int)qb_bytes, 0x00020000),
                __builtin_amdgcn_make_buffer_rsrc((void *)scb, (short)0, (int)sc_bytes, 0x00020000),
                __builtin_amdgcn_make_buffer_rsrc((void *)db, (short)0, (int)d_bytes, 0x00020000)};
    }
    __device__ static void load(const Res &r, Lane &l, uint32_t blk, bool live, int c) {
        const uint32_t oq = live ? blk * 192u + (uint32_t)c * 48u : Q4K_OOB;
        l.q0 = __builtin_amdgcn_raw_buffer_load_b128(r.q, oq, 0, 2);
        l.q1 = __builtin_amdgcn_raw_buffer_load_b128(r.q, oq + 16u, 0, 2);
        l.q2 = __builtin_amdgcn_raw_buffer_load_b128(r.q, oq + 32u, 0, 2);
        l.sw = __builtin_amdgcn_raw_buffer_load_b32(r.s, live ? blk * 16u + (uint32_t)c * 4u : Q4K_OOB, 0, 0);
        l.dw = __builtin_amdgcn_raw_buffer_load_b16(r.d, live ? blk * 2u : Q4K_OOB, 0, 0);
    }
    __device__ static void expand(Lane &) {}
    __device__ static int xbase(int b, int c) { return 256 * b + 128 * (c >> 1) + 16 * (c & 1); }
    // scales 8 n2 + isub + 2t: bytes isub, isub + 2 of dwords 2 n2 and 2 n2 + 1 of
    // the quad's scale dwords (all lanes take part in the DPP broadcasts)
    __device__ static void scales(const Lane &l, int c, float A[4], float B[4]) {
        // lanes 0, 1 of the quad take its scale dwords 0, 1 and lanes 2, 3
        // dwords 2, 3 (DPP quad_perm [0,0,2,2] and [1,1,3,3]); v_perm then
        // gathers bytes isub, isub + 2 of both into one dword
        const uint32_t sa = (uint32_t)__builtin_amdgcn_mov_dpp((int)l.sw, 0xA0, 0xf, 0xf, true);
        const uint32_t sb = (uint32_t)__builtin_amdgcn_mov_dpp((int)l.sw, 0xF5, 0xf, 0xf, true);
        const uint32_t sc = __builtin_amdgcn_perm(sb, sa, (c & 1) ? 0x07050301u : 0x06040200u);
        const float d = h2f(l.dw);
#pragma unroll
        for (int t = 0; t < 4; t++) A[t] = d * (float)(int8_t)(sc >> (8 * t));
        (void)B;
    }
    // quadrant t: ql_a / ql_b (t odd), low / high nibble (t >= 2), qh bits 2t..2t+1
    template <uint32_t X = 0u>
    __device__ static void codes(const Lane &l, int c, int t, uint32_t cw[4]) {
        (void)c;
        const uint32_t w[12] = {l.q0.x, l.q0.y, l.q0.z, l.q0.w, l.q1.x, l.q1.y,
                                l.q1.z, l.q1.w, l.q2.x, l.q2.y, l.q2.z, l.q2.w};
#pragma unroll
        for (int j = 0; j < 4; j++)
            cw[j] = (((w[4 * (t & 1) + j] >> (4 * (t >> 1))) & 0x0F0F0F0Fu) |
                     (((w[8 + j] >> (2 * t)) << 4) & 0x30303030u)) ^ X;
    }
    __device__ static int subdot(const uint32_t cw[4], const u32x4 lo, const u32x4 hi) {
        return q6k_subdot(cw, lo, hi);
    }
    __device__ static float term(float A, float B, float xsc, int sdot, float xsum) {
        (void)B;
        return A * (xsc * (float)sdot - 32.f * xsum);
    }
    // the f32-x kernel's codes are the bytes xor FXOR (unsigned), its quadrant
    // term; its xsum arrives as XSUM_MUL * sum(x), scaled where x is read from LDS
    static constexpr uint32_t FXOR = 0u;
    static constexpr float XSUM_MUL = -32.f;
    __device__ static float fterm(float A, float B, float xsc, float dot, float xsum) {
        (void)B;
        return A * __builtin_fmaf(xsc, dot, xsum);
    }
};

// Q5_K: streams hdr (d, dmin, the 12 scale bytes: 16 B per block) and q
// (ggml's qh[32] then qs[128]: 160 B).  Lane c takes sub-blocks 2c (low
// nibbles of qs[32c + l]) and 2c + 1 (high nibbles), the 5th bits in qh[l] bits
// 2c and 2c + 1; quadrant t = sub-block 2c + t / 2, elements 16 (t % 2) ..+15.
// Each lane loads its own 32 qs bytes, a quarter of qh (bytes 8c..8c+7) and
// header dword c; expand() gathers the whole qh and header of the block from
// the quad by DPP, so no byte is loaded twice.  q = nibble | bit << 4 (0..31);
// weight (d * sc) * q - dmin * m (crates/arf-core/src/model/gguf.rs:2053-2090).
struct DotQ5K {
    const uint8_t *hdr, *q;
    uint32_t hdr_bytes, q_bytes;
    struct Res {
        __amdgpu_buffer_rsrc_t h, q;
    };
    struct Lane {
        u32x4 qs0, qs1;
        u32x2 qh;
        uint32_t hw;
        uint32_t qhd[8], hd[4];  // filled by expand()
    };
    static constexpr int XSTEP = 16, PF = Q6K_GEMV_PF;
    __device__ Res res() const {
        return {__builtin_amdgcn_make_buffer_rsrc((void *)hdr, (short)0, (int)hdr_bytes, 0x00020000),
                __builtin_amdgcn_make_buffer_rsrc((void *)q, (short)0, (int)q_bytes, 0x00020000)};
    }
    __device__ static void load(const Res &r, Lane &l, uint32_t blk, bool live, int c) {
        const uint32_t oq = live ? blk * 160u : Q4K_OOB;
        l.qs0 = __builtin_amdgcn_raw_buffer_load_b128(r.q, oq + 32u + 32u * (uint32_t)c, 0, 2);
        l.qs1 = __builtin_amdgcn_raw_buffer_load_b128(r.q, oq + 48u + 32u * (uint32_t)c, 0, 2);
        l.qh = __builtin_amdgcn_raw_buffer_load_b64(r.q, oq + 8u * (uint32_t)c, 0, 2);
        l.hw = __builtin_amdgcn_raw_buffer_load_b32(r.h, live ? blk * 16u + 4u * (uint32_t)c : Q4K_OOB, 0, 0);
    }
    __device__ static void expand(Lane &l) {
        l.qhd[0] = quad_bcast<0>(l.qh.x), l.qhd[1] = quad_bcast<0>(l.qh.y);
        l.qhd[2] = quad_bcast<1>(l.qh.x), l.qhd[3] = quad_bcast<1>(l.qh.y);
        l.qhd[4] = quad_bcast<2>(l.qh.x), l.qhd[5] = quad_bcast<2>(l.qh.y);
        l.qhd[6] = quad_bcast<3>(l.qh.x), l.qhd[7] = quad_bcast<3>(l.qh.y);
        l.hd[0] = quad_bcast<0>(l.hw), l.hd[1] = quad_bcast<1>(l.hw);
        l.hd[2] = quad_bcast<2>(l.hw), l.hd[3] = quad_bcast<3>(l.hw);
    }
    __device__ static int xbase(int b, int c) { return 256 * b + 64 * c; }
    // the 6-bit (sc, m) of sub-blocks 2c and 2c + 1 (q4k_scale_min without a
    // per-lane branch)
    __device__ static void scales(const Lane &l, int c, float A[4], float B[4]) {
        const float d = h2f(l.hd[0]), dmin = h2f(l.hd[0] >> 16);
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int j = 2 * c + u, i = j & 3;
            const uint32_t a = byte_of(l.hd[1], i), bb = byte_of(l.hd[2], i), cc = byte_of(l.hd[3], i);
            const uint32_t sc = j < 4 ? (a & 63u) : ((cc & 0xFu) | ((a >> 6) << 4));
            const uint32_t m = j < 4 ? (bb & 63u) : ((cc >> 4) | ((bb >> 6) << 4));
            A[2 * u] = A[2 * u + 1] = d * (float)sc;
            B[2 * u] = B[2 * u + 1] = dmin * (float)m;
        }
    }
    // quadrant t: qs bytes 16 (t % 2) + 4j ..+3 and qh dword 4 (t % 2) + j
    template <uint32_t X = 0u>
    __device__ static void codes(const Lane &l, int c, int t, uint32_t cw[4]) {
        const int nib = t >> 1;
        const u32x4 qs = (t & 1) ? l.qs1 : l.qs0;
#pragma unroll
        for (int j = 0; j < 4; j++)
            cw[j] = (((qs[j] >> (4 * nib)) & 0x0F0F0F0Fu) | bit_to4(l.qhd[4 * (t & 1) + j], 2 * c + nib)) ^ X;
    }
    __device__ static int subdot(const uint32_t cw[4], const u32x4 lo, const u32x4 hi) {
        return q6k_subdot(cw, lo, hi);
    }
    __device__ static float term(float A, float B, float xsc, int sdot, float xsum) {
        return A * (xsc * (float)sdot) - B * xsum;
    }
    static constexpr uint32_t FXOR = 0u;
    static constexpr float XSUM_MUL = 1.f;
    __device__ static float fterm(float A, float B, float xsc, float dot, float xsum) {
        return A * (xsc * dot) - B * xsum;
    }
};

// IQ4_XS: streams hdr (d, scales_h, scales_l[4]: 8 B per block) and qs (128 B).
// Lane c takes sub-blocks 2c and 2c + 1 (qs bytes 32c .. 32c + 31); quadrant
// t = sub-block 2c + t / 2, low (t even) or high nibbles: elements 16 t ..+15
// of the lane's 64.  Lanes 0 and 1 load the header's two dwords and expand()
// shares them over the quad.  A code is the non-linear codebook's int8 value
// (kvalues_iq4nl), looked up with two v_perm over the 16 entries; weight
// (d * (ls - 32)) * kv (crates/arf-core/src/model/gguf.rs:1908-1976).
struct DotIQ4XS {
    const uint8_t *hdr, *qs;
    uint32_t hdr_bytes, qs_bytes;
    struct Res {
        __amdgpu_buffer_rsrc_t h, q;
    };
    struct Lane {
        u32x4 q0, q1;
        uint32_t hw;
        uint32_t hd[2];  // filled by expand()
    };
    static constexpr int XSTEP = 16, PF = Q6K_GEMV_PF;
    __device__ Res res() const {
        return {__builtin_amdgcn_make_buffer_rsrc((void *)hdr, (short)0, (int)hdr_bytes, 0x00020000),
                __builtin_amdgcn_make_buffer_rsrc((void *)qs, (short)0, (int)qs_bytes, 0x00020000)};
    }
    __device__ static void load(const Res &r, Lane &l, uint32_t blk, bool live, int c) {
        const uint32_t oq = live ? blk * 128u + 32u * (uint32_t)c : Q4K_OOB;
        l.q0 = __builtin_amdgcn_raw_buffer_load_b128(r.q, oq, 0, 2);
        l.q1 = __builtin_amdgcn_raw_buffer_load_b128(r.q, oq + 16u, 0, 2);
        l.hw = __builtin_amdgcn_raw_buffer_load_b32(r.h, live && c < 2 ? blk * 8u + 4u * (uint32_t)c : Q4K_OOB,
                                                     0, 0);
    }
    __device__ static void expand(Lane &l) {
        l.hd[0] = quad_bcast<0>(l.hw), l.hd[1] = quad_bcast<1>(l.hw);
    }
    __device__ static int xbase(int b, int c) { return 256 * b + 64 * c; }
    __device__ static void scales(const Lane &l, int c, float A[4], float B[4]) {
        const float d = h2f(l.hd[0]);
        const uint32_t sh = l.hd[0] >> 16, sl = byte_of(l.hd[1], c);
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int j = 2 * c + u;
            const int ls = (int)(((sl >> (4 * u)) & 0xFu) | (((sh >> (2 * j)) & 3u) << 4));
            A[2 * u] = A[2 * u + 1] = d * (float)(ls - 32);
            B[2 * u] = B[2 * u + 1] = 0.f;
        }
    }
    template <uint32_t X = 0u>
    __device__ static void codes(const Lane &l, int c, int t, uint32_t cw[4]) {
        (void)c;
        const u32x4 q = (t >> 1) ? l.q1 : l.q0;
#pragma unroll
        for (int j = 0; j < 4; j++) cw[j] = iq4nl_lookup<X>((q[j] >> (4 * (t & 1))) & 0x0F0F0F0Fu);
    }
    // sum(kv * X) with signed kv: the high plane by sdot4; the low (unsigned)
    // plane by udot4 of kv + 128 (kv xor 0x80), less 128 * sum(X_lo)
    __device__ static int subdot(const uint32_t cw[4], const u32x4 lo, const u32x4 hi) {
        uint32_t a = 0u, sl = 0u;
        int b = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            a = __builtin_amdgcn_udot4(cw[j] ^ 0x80808080u, lo[j], a, false);
            sl = __builtin_amdgcn_udot4(0x01010101u, lo[j], sl, false);
            b = __builtin_amdgcn_sdot4((int)cw[j], (int)hi[j], b, false);
        }
        // |sum| <= 16 * 127 * 32767 < 2^26: exact in int32 and in f32
        return b * 256 + (int)a - 128 * (int)sl;
    }
    __device__ static float term(float A, float B, float xsc, int sdot, float xsum) {
        (void)B, (void)xsum;
        return A * (xsc * (float)sdot);
    }
    // f32 x: the unsigned codes kv + 128 (kv xor 0x80), less 128 * sum(x)
    static constexpr uint32_t FXOR = 0x80808080u;
    static constexpr float XSUM_MUL = -128.f;
    __device__ static float fterm(float A, float B, float xsc, float dot, float xsum) {
        (void)B;
        return A * __builtin_fmaf(xsc, dot, xsum);
    }
};

template <class F, int MX, int XR>
__global__ __launch_bounds__(Q6K_GEMV_THREADS) void gemv_dot(F fmt, const float *__restrict__ x,
                                                            float *__restrict__ y, int n, int nblk,
                                                            int m) {
    constexpr bool XREG = MX == 1;
    constexpr int C = Q6K_GEMV_CHUNK, PF = F::PF;
    static_assert(PF % C == 0, "claims must sit at fixed slots of the unrolled loop");
    extern __shared__ uint4 smem4[];
    __shared__ int next_chunk;
    const int k = nblk * 256;
    uint8_t *xlo = reinterpret_cast<uint8_t *>(smem4);
    uint8_t *xhi = xlo + (size_t)MX * k;
    float *s16 = reinterpret_cast<float *>(xhi + (size_t)MX * k);
    float *xe = s16 + (size_t)MX * (k / 16);
    float *part = xe + (size_t)MX * (k / 32);  // [MX][R][spr]

    const typename F::Res res = fmt.res();

    const int tid = threadIdx.x;
    const int l16 = tid & 15, grp = tid >> 4;
    const int bq = l16 >> 2, c = l16 & 3;

    const int G = gridDim.x;
    const int r0 = (int)((int64_t)blockIdx.x * n / G);
    const int r1 = (int)((int64_t)(blockIdx.x + 1) * n / G);
    const int R = r1 - r0;
    const int spr = (nblk + 3) >> 2;
    const int cpc = (R + C - 1) / C;
    const int nchunks = cpc * spr;

    int icol = 0, irow = 0;
    auto start_chunk = [&](int kc) {
        icol = kc < nchunks ? kc / cpc : spr;
        irow = (kc - icol * cpc) * C;
    };
    typename F::Lane ld[PF];
    int srow[PF], scol[PF];
    auto issue = [&](int u, bool first) {
        if (u % C == 0) {
            int kc = grp;
            if (!first) {
                if (l16 == 0) kc = atomicAdd(&next_chunk, 1);
                kc = __builtin_amdgcn_ds_swizzle(kc, 0x10);  // lane 0 of each 16-lane group
            }
            start_chunk(kc);
        } else {
            irow++;
        }
        const int b = 4 * icol + bq;
        const bool live = icol < spr && irow < R && b < nblk;
        const uint32_t blk = (uint32_t)(r0 + irow) * (uint32_t)nblk + (uint32_t)b;
        F::load(res, ld[u], blk, live, c);
        srow[u] = irow;
        scol[u] = icol;
    };

    if (tid == 0) next_chunk = Q6K_GEMV_GROUPS;
    const int xitems = m * k / 8;
    XqRound xr[XR];
#pragma unroll
    for (int r = 0; r < XR; r++) xr[r] = xq_load(x, xitems, r * Q6K_GEMV_THREADS);
    __builtin_amdgcn_s_barrier();
    issue(0, true);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < XR; r++)
        if (r * Q6K_GEMV_THREADS < xitems) xq6_process(xr[r], xitems, r * Q6K_GEMV_THREADS, k, xlo, xhi, s16, xe);
    for (int base = XR * Q6K_GEMV_THREADS; base < xitems; base += Q6K_GEMV_THREADS)
        xq6_process(xq_load(x, xitems, base), xitems, base, k, xlo, xhi, s16, xe);
    __syncthreads();
#pragma unroll
    for (int u = 1; u < PF; u++) {
        issue(u, u < C);
        __builtin_amdgcn_sched_barrier(0);
    }

    // x of the column being consumed: the lane's 4 quadrants (elements
    // xbase + XSTEP t .. + 15)
    int xcol = -1, xbase = 0;
    u32x4 XL[4], XH[4];
    float XS[4], XE[4];
    auto load_x = [&](int col) {
        xcol = col;
        xbase = F::xbase(min(4 * col + bq, nblk - 1), c);
        if (XREG) {
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int eo = xbase + F::XSTEP * t;
                XL[t] = *reinterpret_cast<const u32x4 *>(xlo + eo);
                XH[t] = *reinterpret_cast<const u32x4 *>(xhi + eo);
                XS[t] = s16[eo >> 4];
                XE[t] = xe[eo >> 5];
            }
        }
    };

    auto consume = [&](int u) {
        const int col = scol[u], row = srow[u];
        const bool live = col < spr && row < R;
        if (live && col != xcol) load_x(col);
        F::expand(ld[u]);  // DPP: every lane, live or not
        float A[4], B[4];
        F::scales(ld[u], c, A, B);
#pragma unroll
        for (int mi = 0; mi < MX; mi++) {
            if (MX == 1 || mi < m) {
                float v = 0.f;
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    uint32_t cw[4];
                    F::codes(ld[u], c, t, cw);
                    int sdot;
                    float xsum, xsc;
                    if (XREG) {
                        sdot = F::subdot(cw, XL[t], XH[t]);
                        xsum = XS[t];
                        xsc = XE[t];
                    } else {
                        const size_t eo = (size_t)mi * k + xbase + F::XSTEP * t;
                        sdot = F::subdot(cw, *reinterpret_cast<const u32x4 *>(xlo + eo),
                                         *reinterpret_cast<const u32x4 *>(xhi + eo));
                        xsum = s16[eo >> 4];
                        xsc = xe[eo >> 5];
                    }
                    v += F::term(A[t], B[t], xsc, sdot, xsum);
                }
                v = row16_sum(v);
                if (l16 == 0 && live) part[((size_t)mi * R + row) * spr + col] = v;
            }
        }
    };

    while (scol[0] < spr) {
#pragma unroll
        for (int u = 0; u < PF; u++) {
            consume(u);
            issue(u, false);
        }
    }
    __syncthreads();

    for (int t = tid; t < MX * R; t += Q6K_GEMV_THREADS) {
        const int mi = t / R, r = t - mi * R;
        if (mi < m) {
            const float *pr = part + (size_t)t * spr;
            float v = 0.f;
            for (int cc = 0; cc < spr; cc++) v += pr[cc];
            y[(int64_t)mi * n + r0 + r] = v;
        }
    }
}

// ----------------------------------------------- Q6_K / Q5_K at f32 x (m = 1) ----
// The dot GEMV's work split and lane map with f32 arithmetic: x is kept in LDS
// as f32, each 32 elements scaled by 2^s (s = min(24, 100 - e), |x| < 2^e, so
// no product overflows), with the true-unit sum of every 16 elements and
// 2^(24 - s) per 32.  A quadrant's 16 codes (unsigned bytes: Q6_K q < 64,
// Q5_K q < 32, IQ4_XS kv + 128) go into v_fma_mix_f32 as the f16 subnormals
// q * 2^-24, so each product x * 2^s * q * 2^-24 is exact in f32 and the
// quadrant adds F::fterm(A, B, 2^(24 - s), sum(x * q), XSUM_MUL * sum(x)): for Q6_K
// (d * sc) * (sum(x * q) - 32 * sum(x)), the oracle's (d * sc) * (q - 32) per
// weight (gguf.rs:2120-2123) times f32 x, factorised.
namespace {

__device__ __forceinline__ void xf16_process(const XqRound &r, int items, int base, float4 *xf,
                                             float *s16, float *xe) {
    const int it = base + (int)threadIdx.x;
    const float4 v0 = r.v0, v1 = r.v1;
    float amax = fmaxf(fmaxf(fmaxf(fabsf(v0.x), fabsf(v0.y)), fmaxf(fabsf(v0.z), fabsf(v0.w))),
                       fmaxf(fmaxf(fabsf(v1.x), fabsf(v1.y)), fmaxf(fabsf(v1.z), fabsf(v1.w))));
    float sum = ((v0.x + v0.y) + (v0.z + v0.w)) + ((v1.x + v1.y) + (v1.z + v1.w));
    amax = fmaxf(amax, quad_perm<QP_XOR1>(amax));
    sum += quad_perm<QP_XOR1>(sum);  // 16 elements (items 2i, 2i + 1)
    amax = fmaxf(amax, quad_perm<QP_XOR2>(amax));
    const int ex = (amax > 0.f) ? __builtin_amdgcn_frexp_expf(amax) : 0;
    const int sh = min(24, 100 - ex);
    if (it < items) {
        xf[2 * it] = make_float4(ldexpf(v0.x, sh), ldexpf(v0.y, sh), ldexpf(v0.z, sh), ldexpf(v0.w, sh));
        xf[2 * it + 1] = make_float4(ldexpf(v1.x, sh), ldexpf(v1.y, sh), ldexpf(v1.z, sh), ldexpf(v1.w, sh));
        if ((it & 1) == 0) s16[it >> 1] = sum;
        if ((it & 3) == 0) xe[it >> 2] = ldexpf(1.f, 24 - sh);
    }
}

// sum of x * q over 16 codes (one byte each in cw[4], element order), x scaled
__device__ __forceinline__ float codes16_fdot(const uint32_t cw[4], const float *X) {
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        // bytes 0, 2 and bytes 1, 3 into 16-bit halves (v_perm_b32, selector 0x0C = 0)
        const uint32_t A = __builtin_amdgcn_perm(cw[j], cw[j], 0x0C020C00u),
                       B = __builtin_amdgcn_perm(cw[j], cw[j], 0x0C030C01u);
        acc = fmix<0>(X[4 * j], A, acc);
        acc = fmix<1>(X[4 * j + 2], A, acc);
        acc = fmix<0>(X[4 * j + 1], B, acc);
        acc = fmix<1>(X[4 * j + 3], B, acc);
    }
    return acc;
}

}  // namespace

// Rows: workgroup w of G owns rows w, w + G, w + 2G, ... (the whole chip reads a
// narrow window of the weight stream at a time), and x is scaled into LDS
// before the first weight load is issued (every weight request in flight
// delays the x requests); as the Q4_K f32 GEMV (gemv_q4k_f32_body).
template <class F, int XR>
__global__ __launch_bounds__(Q6K_GEMV_THREADS) void gemv_dot_f32(F fmt, const float *__restrict__ x,
                                                                float *__restrict__ y, int n, int nblk) {
    constexpr int C = Q6K_GEMV_CHUNK, PF = F::PF;
    static_assert(PF % C == 0, "claims must sit at fixed slots of the unrolled loop");
    extern __shared__ uint4 smem4[];
    __shared__ int cnt[64];             // chunk counters per column (spr <= 64)
    __shared__ unsigned long long exm;  // columns seen exhausted
    const int k = nblk * 256;
    float *xfl = reinterpret_cast<float *>(smem4);  // [k], scaled
    float *s16 = xfl + k;                           // [k / 16]
    float *xe = s16 + k / 16;                       // [k / 32]
    float *part = xe + k / 32;                      // [R][spr]

    const typename F::Res res = fmt.res();
    const int tid = threadIdx.x;
    const int l16 = tid & 15, grp = tid >> 4;
    const int bq = l16 >> 2, c = l16 & 3;

    const int G = gridDim.x;
    const int r0 = blockIdx.x;             // rows r0 + i * G, i < R
    const int R = (n - r0 + G - 1) / G;
    const int spr = (nblk + 3) >> 2;
    const int cpc = (R + C - 1) / C;

    // A home column per group (group % spr), its chunks claimed from that
    // column's counter, so a group keeps the x of one column in registers for
    // most of its work; when it runs out, the next column not yet seen
    // exhausted (a bit mask of them).  Lane 0 of the group decides and claims,
    // the group takes column and chunk by broadcast, so its lanes stay in step.
    // (One counter over all chunks, column by column, had a group's chunks ~32
    // apart, in another column each time, its x reloaded from LDS per chunk:
    // Q5_K at C2's shape 24.1 -> 19.5 us, C3 m = 1 21.9 -> 20.7 us with home
    // columns and the mask; home columns that tried the next columns one by
    // one were slower at C3's 17 columns, 24.2 us: every failed try is an LDS
    // atomic round trip.)
    int icol = grp % spr, irow = (grp / spr) * C;
    auto claim = [&]() {
        int col = icol;
        for (int t = 0; t < spr; t++) {
            int kk = 0;
            if (l16 == 0) {
                if (t > 0) {
                    const uint64_t all = spr == 64 ? ~0ull : ((1ull << spr) - 1);
                    const uint64_t av = ~__hip_atomic_load(&exm, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) & all;
                    const uint64_t r = col == 0 ? av : ((av >> col) | (av << (spr - col))) & all;
                    if (r == 0) {
                        col = -1;  // none left
                    } else {
                        col += __builtin_ctzll(r);
                        if (col >= spr) col -= spr;
                    }
                }
                if (col >= 0) {
                    kk = atomicAdd(&cnt[col], 1);
                    if (kk >= cpc) atomicOr(&exm, 1ull << col);
                }
            }
            col = __builtin_amdgcn_ds_swizzle(col, 0x10);  // lane 0 of each 16-lane group
            kk = __builtin_amdgcn_ds_swizzle(kk, 0x10);
            if (col < 0) break;
            if (kk < cpc) {
                icol = col;
                irow = kk * C;
                return;
            }
        }
        icol = spr;  // no work left
    };
    typename F::Lane ld[PF];
    int srow[PF], scol[PF];
    auto issue = [&](int u, bool first) {
        if (!first) {
            if (u % C == 0) claim();
            else irow++;
        } else if (u > 0) {
            irow++;
        }
        const int b = 4 * icol + bq;
        const bool live = icol < spr && irow < R && b < nblk;
        const uint32_t blk = (uint32_t)(r0 + irow * G) * (uint32_t)nblk + (uint32_t)b;
        F::load(res, ld[u], blk, live, c);
        srow[u] = irow;
        scol[u] = icol;
    };

    // counters start past the chunks the groups begin on
    for (int cc = tid; cc < spr; cc += Q6K_GEMV_THREADS) cnt[cc] = (Q6K_GEMV_GROUPS - cc + spr - 1) / spr;
    if (tid == 0) exm = 0;
    // x loads, x scaled into LDS, the barrier (which orders LDS only), then the
    // first weight loads
    const int xitems = k / 8;
    XqRound xr[XR];
#pragma unroll
    for (int r = 0; r < XR; r++) xr[r] = xq_load(x, xitems, r * Q6K_GEMV_THREADS);
    asm volatile("" ::: "memory");
#pragma unroll
    for (int r = 0; r < XR; r++)
        xf16_process(xr[r], xitems, r * Q6K_GEMV_THREADS, reinterpret_cast<float4 *>(xfl), s16, xe);
    for (int base = XR * Q6K_GEMV_THREADS; base < xitems; base += Q6K_GEMV_THREADS)
        xf16_process(xq_load(x, xitems, base), xitems, base, reinterpret_cast<float4 *>(xfl), s16, xe);
    lds_barrier();
#pragma unroll
    for (int u = 0; u < PF; u++) issue(u, u < C);

    // scaled x of the column being consumed: the lane's 4 quadrants
    int xcol = -1;
    float X[4][16], XS[4], XE[4];
    auto load_x = [&](int col) {
        xcol = col;
        const int xb = F::xbase(min(4 * col + bq, nblk - 1), c);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int eo = xb + F::XSTEP * t;
            const float4 *src = reinterpret_cast<const float4 *>(xfl + eo);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 v = src[i];
                X[t][4 * i] = v.x;
                X[t][4 * i + 1] = v.y;
                X[t][4 * i + 2] = v.z;
                X[t][4 * i + 3] = v.w;
            }
            XS[t] = F::XSUM_MUL * s16[eo >> 4];
            XE[t] = xe[eo >> 5];
        }
    };

    auto consume = [&](int u) {
        const int col = scol[u], row = srow[u];
        const bool live = col < spr && row < R;
        if (live && col != xcol) load_x(col);
        F::expand(ld[u]);  // DPP: every lane, live or not
        float A[4], B[4];
        F::scales(ld[u], c, A, B);
        float v = 0.f;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            uint32_t cw[4];
            F::template codes<F::FXOR>(ld[u], c, t, cw);
            v += F::fterm(A[t], B[t], XE[t], codes16_fdot(cw, X[t]), XS[t]);
        }
        v = row16_sum(v);
        if (l16 == 0 && live) part[(size_t)row * spr + col] = v;
    };

    while (scol[0] < spr) {
#pragma unroll
        for (int u = 0; u < PF; u++) {
            consume(u);
            issue(u, false);
        }
    }
    lds_barrier();

    for (int t = tid; t < R; t += Q6K_GEMV_THREADS) {
        const float *pr = part + (size_t)t * spr;
        float v = 0.f;
        for (int cc = 0; cc < spr; cc++) v += pr[cc];
        y[r0 + t * G] = v;
    }
}

// ------------------------------------------------------------------ Q8_0 ----
// One wave per Q80_ROWS weight rows; lane l takes blocks l, l + 64, ... of
// each: two 16-byte code loads and the block's f16 d per row, all the loads
// of a 128-block round issued before the first use, so a row of up to 128
// blocks costs one memory round trip.  Per block the lane forms
// d * (sum of x * q over its 32 codes) in f32; the wave then adds its lanes.
// x rows (f32, <= 4) are read per block from the L1/L2-resident vector, once
// for the wave's rows.
// Reference arithmetic: matmul_nt_q8_0 (crates/arf-ml/src/matmul.rs:174-204).
// two waves per workgroup (twice as many workgroups as four): C1 3.91 -> 3.73 us
// per launch; one row per wave or four rows per wave measured 4.5-4.7 us
constexpr int Q80_WAVES = 2, Q80_ROWS = 2;
template <int MX>
__global__ __launch_bounds__(64 * Q80_WAVES) void gemv_q80w(const uint4 *__restrict__ qs,
                                                           const uint16_t *__restrict__ dd,
                                                           const float *__restrict__ x,
                                                           float *__restrict__ y, int n, int nblk,
                                                           int m) {
    constexpr int R = Q80_ROWS;
    const int lane = threadIdx.x & 63;
    const int64_t row0 = ((int64_t)blockIdx.x * Q80_WAVES + (threadIdx.x >> 6)) * R;
    if (row0 >= n) return;  // the whole wave
    const int64_t k = (int64_t)nblk * 32;
    const uint4 *qr[R];
    const uint16_t *dr[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int64_t row = min(row0 + r, (int64_t)n - 1);  // rows past n: computed, not stored
        qr[r] = qs + row * nblk * 2;
        dr[r] = dd + row * nblk;
    }
    float acc[MX][R];
#pragma unroll
    for (int mi = 0; mi < MX; mi++)
#pragma unroll
        for (int r = 0; r < R; r++) acc[mi][r] = 0.f;
    for (int b0 = 0; b0 < nblk; b0 += 128) {
        const int nu = nblk - b0 > 64 ? 2 : 1;  // 64-block rounds in this pass (uniform)
        uint4 q[2][R][2];
        float dv[2][R];
        int bc[2];
        bool ok[2];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int b = b0 + 64 * u + lane;
            ok[u] = b < nblk;
            bc[u] = ok[u] ? b : nblk - 1;  // past the row: a valid block, its term dropped
            if (u < nu) {
#pragma unroll
                for (int r = 0; r < R; r++) {
                    q[u][r][0] = ld_nt(qr[r] + 2 * bc[u]);
                    q[u][r][1] = ld_nt(qr[r] + 2 * bc[u] + 1);
                    dv[u][r] = h2f(dr[r][bc[u]]);
                }
            }
        }
#pragma unroll
        for (int mi = 0; mi < MX; mi++) {
            if (mi < m) {
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    if (u < nu) {
                        float xv[32];
                        load16(x + mi * k + (int64_t)bc[u] * 32, xv);
                        load16(x + mi * k + (int64_t)bc[u] * 32 + 16, xv + 16);
#pragma unroll
                        for (int r = 0; r < R; r++) {
                            const float t = dv[u][r] * (dot16_i8(xv, q[u][r][0]) + dot16_i8(xv + 16, q[u][r][1]));
                            acc[mi][r] += ok[u] ? t : 0.f;
                        }
                    }
                }
            }
        }
    }
#pragma unroll
    for (int mi = 0; mi < MX; mi++)
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float hv = half_wave_sum_dpp(acc[mi][r]);
            // every lane: .x = lane half 0's sum, .y = half 1's
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(hv), __float_as_uint(hv), false, false);
            const float v = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
            if (lane == 0 && mi < m && row0 + r < n) y[(int64_t)mi * n + row0 + r] = v;
        }
}

template <int MX>
static hipError_t launch_q80(const arfq_weight *w, int e, int m, const float *x, float *y, hipStream_t s) {
    const int nblk = (int)(w->k / 32);
    const int64_t eb = (int64_t)e * w->n * nblk;  // first block of expert e
    const int64_t rows_per_wg = (int64_t)Q80_WAVES * Q80_ROWS;
    const unsigned grid = (unsigned)((w->n + rows_per_wg - 1) / rows_per_wg);
    gemv_q80w<MX><<<grid, 64 * Q80_WAVES, 0, s>>>((const uint4 *)w->s0 + eb * 2, (const uint16_t *)w->s1 + eb,
                                                  x, y, (int)w->n, nblk, m);
    return hipGetLastError();
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

static size_t q4k_gemv_lds(const arfq_weight *w, int mx);
static bool q4k_f32s_ok(const arfq_weight *w);
static size_t dot_lds(const arfq_weight *w, int mx);
static bool dot_f32_ok(const arfq_weight *w);
// the byte-code dot GEMV: Q6_K at m <= 2, Q5_K at m <= 4, while x fits in LDS and
// one expert's streams fit 31-bit buffer offsets
static int dot_mx(int64_t m) { return m <= 2 ? (int)m : 4; }
static bool dot_ok(const arfq_weight *w, int64_t m) {
    const int64_t nb = w->n * (w->k / 256);
    if (w->qtype == ARFQ_Q6_K)
        return m <= 2 && dot_lds(w, (int)m) <= 64 * 1024 && nb * 192 < (int64_t)Q4K_OOB;
    if (w->qtype == ARFQ_Q5_K)
        return m <= 4 && dot_lds(w, dot_mx(m)) <= 64 * 1024 && nb * 160 < (int64_t)Q4K_OOB;
    if (w->qtype == ARFQ_IQ4_XS)
        return m <= 4 && dot_lds(w, dot_mx(m)) <= 64 * 1024 && nb * 128 < (int64_t)Q4K_OOB;
    return false;
}

// The 16-bit fixed-point x kernels (gemv_q4k / gemv_dot): only under
// ARFQ_OPT_GEMV_X16, and only where their LDS fits the default 64 KiB (they are
// launched without raising the limit) and one expert's code stream fits the
// 31-bit buffer offsets.
static bool q4k_x16_ok(const arfq_weight *w, int64_t m) {
    return w->qtype == ARFQ_Q4_K && m >= 1 && m <= GEMV_MAX_M && q4k_gemv_lds(w, m <= 2 ? (int)m : 4) <= 64 * 1024 &&
           w->n * (w->k / 256) * 128 < (int64_t)Q4K_OOB;
}

// Which (qtype, m) the GEMV family takes.  Without x16 every path multiplies
// f32 x in f32: Q4_K / Q5_K / IQ4_XS / Q6_K at m = 1 (the exact-code f32
// kernels, while their LDS fits), Q6_K at m = 2..4 (gemv_q6k) and Q8_0 at
// m <= 4 (gemv_q80w).  Q4_K / Q5_K / IQ4_XS at m = 2..4, and m = 1 shapes too
// long for the f32 kernels' LDS, go to the skinny MFMA GEMM (x as f16 hi + lo).
// With x16 the 16-bit kernels take the shapes they fit; the rest keep the
// f32 path.
bool gemv_supports(const arfq_weight *w, int64_t m, bool x16) {
    if (m < 1 || m > GEMV_MAX_M) return false;
    switch (w->qtype) {
    case ARFQ_Q4_K:
        if (x16 && q4k_x16_ok(w, m)) return true;
        return m == 1 && q4k_f32s_ok(w);
    case ARFQ_Q5_K:
    case ARFQ_IQ4_XS:
        if (x16 && dot_ok(w, m)) return true;
        return m == 1 && dot_f32_ok(w);
    case ARFQ_Q6_K:  // gemv_q6k takes what the dot kernels do not
    case ARFQ_Q8_0:
        return true;
    default:
        return false;
    }
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

static int64_t q4k_gemv_grid(const arfq_weight *w) {
    const int nblk = (int)(w->k / 256);
    const int64_t steps = w->n * ((nblk + 3) / 4);
    const int cus = w->ctx->cus > 0 ? w->ctx->cus : 256;
    // two workgroups per CU; small problems get fewer (>= 2 steps per group)
    int64_t grid = std::min<int64_t>((int64_t)Q4K_GEMV_WG_PER_CU * cus,
                                     (steps + 2 * Q4K_GEMV_GROUPS - 1) / (2 * Q4K_GEMV_GROUPS));
    grid = std::min<int64_t>(grid, w->n);  // every workgroup owns at least one row
    return grid < 1 ? 1 : grid;
}

// LDS of the Q4_K GEMV: quantized x of mx rows (digits + scale/sum) and the
// per-(row, column) sums of the workgroup's rows.
// steps = (row, column of 4 blocks); two workgroups per CU (one when x is
// long: every workgroup quantizes all of x, and at C3's k = 17408 one per CU
// measured 3 % faster), >= 2 steps per group
static int64_t gemv_grid(const arfq_weight *w, int groups) {
    const int nblk = (int)(w->k / 256);
    const int64_t steps = w->n * ((nblk + 3) / 4);
    const int cus = w->ctx->cus > 0 ? w->ctx->cus : 256;
    const int per_cu = w->k > 8192 ? 1 : 2;
    int64_t grid = std::min<int64_t>(per_cu * (int64_t)cus, (steps + 2 * groups - 1) / (2 * groups));
    grid = std::min<int64_t>(grid, w->n);
    return grid < 1 ? 1 : grid;
}
static size_t dot_lds(const arfq_weight *w, int mx) {
    const int64_t nblk = w->k / 256, spr = (nblk + 3) / 4;
    const int64_t grid = gemv_grid(w, Q6K_GEMV_GROUPS);
    const int64_t rows = (w->n + grid - 1) / grid;
    return (size_t)mx * w->k * 2 + (size_t)mx * (w->k / 16) * 4 + (size_t)mx * (w->k / 32) * 4 +
           (size_t)mx * rows * spr * 4;
}
// the streams of expert e
static DotQ6K dot_q6k(const arfq_weight *w, int e) {
    const int64_t nb = w->n * (w->k / 256), eb = (int64_t)e * nb;
    return {(const uint8_t *)w->s0 + eb * 192, (const uint8_t *)w->s1 + eb * 16,
            (const uint8_t *)w->s2 + eb * 2, (uint32_t)(nb * 192), (uint32_t)(nb * 16),
            (uint32_t)(nb * 2)};
}
static DotQ5K dot_q5k(const arfq_weight *w, int e) {
    const int64_t nb = w->n * (w->k / 256), eb = (int64_t)e * nb;
    return {(const uint8_t *)w->s0 + eb * 16, (const uint8_t *)w->s1 + eb * 160, (uint32_t)(nb * 16),
            (uint32_t)(nb * 160)};
}
static DotIQ4XS dot_iq4xs(const arfq_weight *w, int e) {
    const int64_t nb = w->n * (w->k / 256), eb = (int64_t)e * nb;
    return {(const uint8_t *)w->s0 + eb * 8, (const uint8_t *)w->s1 + eb * 128, (uint32_t)(nb * 8),
            (uint32_t)(nb * 128)};
}
template <class F, int MX, int XR>
static hipError_t launch_dot_t(const F &fmt, const arfq_weight *w, int m, const float *x, float *y,
                               hipStream_t s) {
    const int64_t grid = gemv_grid(w, Q6K_GEMV_GROUPS);
    gemv_dot<F, MX, XR><<<(unsigned)grid, Q6K_GEMV_THREADS, dot_lds(w, MX), s>>>(
        fmt, x, y, (int)w->n, (int)(w->k / 256), m);
    return hipGetLastError();
}
// f32-x dot GEMV (m = 1): one workgroup per CU (its 137 VGPRs leave room for
// one; held to 128 for two, it spilled and ran 31.7 us instead of 23.9 at C3)
constexpr size_t DOT_F32_LDS_MAX = 159 * 1024;
static size_t dot_f32_lds_rows(const arfq_weight *w, int64_t rows) {
    const int64_t nblk = w->k / 256, spr = (nblk + 3) / 4;
    return (size_t)w->k * 4 + (size_t)(w->k / 16) * 4 + (size_t)(w->k / 32) * 4 + (size_t)rows * spr * 4;
}
static int64_t dot_f32_grid(const arfq_weight *w) {
    const int nblk = (int)(w->k / 256);
    const int64_t steps = w->n * ((nblk + 3) / 4);
    const int cus = w->ctx->cus > 0 ? w->ctx->cus : 256;
    return std::max<int64_t>(1, std::min<int64_t>({(int64_t)cus, w->n,
                                                   (steps + 2 * Q6K_GEMV_GROUPS - 1) / (2 * Q6K_GEMV_GROUPS)}));
}
static size_t dot_f32_lds(const arfq_weight *w) {
    const int64_t g = dot_f32_grid(w);
    return dot_f32_lds_rows(w, (w->n + g - 1) / g);
}
static bool dot_f32_ok(const arfq_weight *w) {
    const int64_t nb = w->n * (w->k / 256);
    const int64_t bpb = w->qtype == ARFQ_Q6_K ? 192 : w->qtype == ARFQ_Q5_K ? 160 : w->qtype == ARFQ_IQ4_XS ? 128 : 0;
    return bpb && w->k % 256 == 0 && dot_f32_lds(w) <= DOT_F32_LDS_MAX && nb * bpb < (int64_t)Q4K_OOB &&
           (w->k / 256 + 3) / 4 <= 64;  // the kernel's column counters
}
template <class F, int XR>
static hipError_t launch_dot_f32_t(const F &fmt, const arfq_weight *w, const float *x, float *y, hipStream_t s) {
    static std::atomic<uint64_t> lds_set{0};  // the attribute belongs to the kernel, per device
    if (hipError_t err = set_max_lds_once((const void *)gemv_dot_f32<F, XR>, DOT_F32_LDS_MAX, lds_set))
        return err;
    gemv_dot_f32<F, XR><<<(unsigned)dot_f32_grid(w), Q6K_GEMV_THREADS, dot_f32_lds(w), s>>>(
        fmt, x, y, (int)w->n, (int)(w->k / 256));
    return hipGetLastError();
}
template <class F>
static hipError_t launch_dot_f32(const F &fmt, const arfq_weight *w, const float *x, float *y, hipStream_t s) {
    const int64_t rounds = (w->k / 8 + Q6K_GEMV_THREADS - 1) / Q6K_GEMV_THREADS;
    if (rounds <= 1) return launch_dot_f32_t<F, 1>(fmt, w, x, y, s);
    if (rounds <= 2) return launch_dot_f32_t<F, 2>(fmt, w, x, y, s);
    return launch_dot_f32_t<F, 4>(fmt, w, x, y, s);
}

template <class F, int MX>
static hipError_t launch_dot(const F &fmt, const arfq_weight *w, int m, const float *x, float *y,
                             hipStream_t s) {
    const int64_t rounds = ((int64_t)m * (w->k / 8) + Q6K_GEMV_THREADS - 1) / Q6K_GEMV_THREADS;
    if (rounds <= 1) return launch_dot_t<F, MX, 1>(fmt, w, m, x, y, s);
    if (rounds <= 2) return launch_dot_t<F, MX, 2>(fmt, w, m, x, y, s);
    return launch_dot_t<F, MX, 4>(fmt, w, m, x, y, s);
}
static size_t q4k_gemv_lds(const arfq_weight *w, int mx) {
    const int64_t nblk = w->k / 256, spr = (nblk + 3) / 4;
    const int64_t grid = q4k_gemv_grid(w);
    const int64_t rows = (w->n + grid - 1) / grid;
    return (size_t)mx * (w->k / 32) * (16 * 4 + 8) + (size_t)mx * rows * spr * 4;
}

template <int MX, int XR>
static hipError_t launch_gemv_q4k_t(const arfq_weight *w, int e, int m, const float *x, float *y,
                                    hipStream_t s) {
    const int n = (int)w->n, nblk = (int)(w->k / 256);
    const int64_t nb = w->n * nblk;  // blocks of one expert
    const int64_t eb = (int64_t)e * nb;
    const int64_t grid = q4k_gemv_grid(w);
    const size_t lds = q4k_gemv_lds(w, MX);
    gemv_q4k<MX, XR><<<(unsigned)grid, Q4K_GEMV_THREADS, lds, s>>>(
        (const uint8_t *)w->s0 + eb * 16, (uint32_t)(nb * 16), (const uint8_t *)w->s1 + eb * 128,
        (uint32_t)(nb * 128), x, y, n, nblk, m);
    return hipGetLastError();
}

// XR: rounds of x loads issued ahead of the weight ring (the rest, if any,
// are loaded after it)
template <int MX>
static hipError_t launch_gemv_q4k(const arfq_weight *w, int e, int m, const float *x, float *y,
                                  hipStream_t s) {
    const int64_t rounds = ((int64_t)m * (w->k / 8) + Q4K_GEMV_THREADS - 1) / Q4K_GEMV_THREADS;
    if (rounds <= 1) return launch_gemv_q4k_t<MX, 1>(w, e, m, x, y, s);
    if (rounds <= 2) return launch_gemv_q4k_t<MX, 2>(w, e, m, x, y, s);
    return launch_gemv_q4k_t<MX, 4>(w, e, m, x, y, s);
}

// ---- the f32-x Q4_K GEMV (one x row) ----
// LDS: the scaled x (4 B per element), a (sum, factor) pair per sub-block and
// the column sums of the workgroup's `rows` rows.  The single GEMV, the FFN's
// gate|up pair and its down GEMV run one 1024-thread workgroup per CU (up to
// 159 KB each); the MoE decode pairs kernels run 512-thread workgroups, two per
// CU where the LDS allows.  (The static LDS of the kernel -- the chunk counter --
// sits beside the dynamic part, so the dynamic part stays 1 KB short of 160 KB.)
constexpr size_t Q4K_F32_LDS_MAX = 159 * 1024;
static size_t q4k_f32_lds_rows(const arfq_weight *w, int64_t rows) {
    const int64_t nblk = w->k / 256, spr = (nblk + 3) / 4;
    return (size_t)w->k * 4 + (size_t)(w->k / 32) * 8 + (size_t)((spr + 3) & ~3) * 4 +
           (size_t)rows * spr * 4;
}
// rounds of x loads issued ahead of the weight ring (8 elements per thread and round)
static int q4k_f32_xr(const arfq_weight *w, int threads = Q4K_GEMV_THREADS) {
    const int64_t rounds = (w->k / 8 + threads - 1) / threads;
    return rounds <= 1 ? 1 : rounds <= 2 ? 2 : rounds <= 3 ? 3 : 4;
}
// The single m = 1 GEMV (gemv_q4k_f32): one 1024-thread workgroup per CU, rows
// interleaved over the workgroups, x scaled before the first weight load.  At C2
// (k = 5120, n = 17408) this measured 13.2-13.5 us per launch against 14.6-14.8
// for two 512-thread workgroups per CU with contiguous row ranges and the
// weight loads issued ahead of x (same driver loop, rotating weight copies).
// Small problems get fewer workgroups (>= 2 steps per 16-lane group).
static int64_t q4k_f32s_grid(const arfq_weight *w) {
    const int64_t steps = w->n * ((w->k / 256 + 3) / 4);
    const int cus = w->ctx->cus > 0 ? w->ctx->cus : 256;
    int64_t grid = std::min<int64_t>(cus, (steps + 2 * (Q4K_F32_THREADS / 16) - 1) / (2 * (Q4K_F32_THREADS / 16)));
    grid = std::min<int64_t>(grid, w->n);
    return grid < 1 ? 1 : grid;
}
static size_t q4k_f32s_lds(const arfq_weight *w) {
    const int64_t grid = q4k_f32s_grid(w);
    return q4k_f32_lds_rows(w, (w->n + grid - 1) / grid);
}
static bool q4k_f32s_ok(const arfq_weight *w) {
    return w->qtype == ARFQ_Q4_K && q4k_f32s_lds(w) <= Q4K_F32_LDS_MAX &&
           w->n * (w->k / 256) * 128 < (int64_t)Q4K_OOB && (w->k / 256 + 3) / 4 <= 64;
}
template <int XR>
static hipError_t launch_q4k_f32_t(const arfq_weight *w, int e, const float *x, float *y, hipStream_t s) {
    static std::atomic<uint64_t> lds_set{0};  // the attribute belongs to the kernel, per device
    if (hipError_t err = set_max_lds_once((const void *)gemv_q4k_f32<XR>, Q4K_F32_LDS_MAX, lds_set))
        return err;
    const int nblk = (int)(w->k / 256);
    const int64_t nb = w->n * nblk, eb = (int64_t)e * nb;
    gemv_q4k_f32<XR><<<(unsigned)q4k_f32s_grid(w), Q4K_F32_THREADS, q4k_f32s_lds(w), s>>>(
        (const uint8_t *)w->s0 + eb * 16, (uint32_t)(nb * 16), (const uint8_t *)w->s1 + eb * 128,
        (uint32_t)(nb * 128), x, y, (int)w->n, nblk);
    return hipGetLastError();
}
static hipError_t launch_q4k_f32(const arfq_weight *w, int e, const float *x, float *y, hipStream_t s) {
    switch (q4k_f32_xr(w, Q4K_F32_THREADS)) {
    case 1: return launch_q4k_f32_t<1>(w, e, x, y, s);
    case 2: return launch_q4k_f32_t<2>(w, e, x, y, s);
    case 3: return launch_q4k_f32_t<3>(w, e, x, y, s);
    default: return launch_q4k_f32_t<4>(w, e, x, y, s);
    }
}
template <int XR, int ACT>
static hipError_t launch_q4k_f32_glu_t(const arfq_weight *w, const float *g, const float *u, float *y,
                                       hipStream_t s) {
    static std::atomic<uint64_t> lds_set{0};
    if (hipError_t err = set_max_lds_once((const void *)gemv_q4k_f32_glu<XR, ACT>, Q4K_F32_LDS_MAX, lds_set))
        return err;
    const int64_t nb = w->n * (w->k / 256);
    gemv_q4k_f32_glu<XR, ACT><<<(unsigned)q4k_f32s_grid(w), Q4K_F32_THREADS, q4k_f32s_lds(w), s>>>(
        (const uint8_t *)w->s0, (uint32_t)(nb * 16), (const uint8_t *)w->s1, (uint32_t)(nb * 128), g, u, y,
        (int)w->n, (int)(w->k / 256));
    return hipGetLastError();
}
template <int ACT>
// (taken for k <= 8192 only, gemv_glu_supports: x is one round of loads)
static hipError_t launch_q4k_f32_glu(const arfq_weight *w, const float *g, const float *u, float *y,
                                     hipStream_t s) {
    if (q4k_f32_xr(w, Q4K_F32_THREADS) != 1) return hipErrorInvalidValue;
    return launch_q4k_f32_glu_t<1, ACT>(w, g, u, y, s);
}

// gate and up in one launch: half the single GEMV's workgroups per weight
static int64_t q4k_dual_grid(const arfq_weight *w) { return std::max<int64_t>(1, q4k_f32s_grid(w) / 2); }
bool gemv_dual_supports(const arfq_weight *a, const arfq_weight *b, int64_t m) {
    return m == 1 && a->qtype == ARFQ_Q4_K && b->qtype == ARFQ_Q4_K && a->n == b->n && a->k == b->k &&
           a->experts == 1 && b->experts == 1 && q4k_f32s_ok(a) &&
           q4k_f32_lds_rows(a, (a->n + q4k_dual_grid(a) - 1) / q4k_dual_grid(a)) <= Q4K_F32_LDS_MAX;
}
template <int XR>
static hipError_t launch_dual_t(const arfq_weight *a, const arfq_weight *b, const float *x, float *ya, float *yb,
                                hipStream_t s) {
    static std::atomic<uint64_t> lds_set{0};
    if (hipError_t err = set_max_lds_once((const void *)gemv_q4k_f32_dual<XR>, Q4K_F32_LDS_MAX, lds_set))
        return err;
    const int64_t g = q4k_dual_grid(a), nb = a->n * (a->k / 256);
    gemv_q4k_f32_dual<XR><<<dim3((unsigned)g, 2), Q4K_F32_THREADS, q4k_f32_lds_rows(a, (a->n + g - 1) / g), s>>>(
        (const uint8_t *)a->s0, (const uint8_t *)a->s1, (const uint8_t *)b->s0, (const uint8_t *)b->s1,
        (uint32_t)(nb * 16), (uint32_t)(nb * 128), x, ya, yb, (int)a->n, (int)(a->k / 256));
    return hipGetLastError();
}
hipError_t launch_gemv_dual(const arfq_weight *a, const arfq_weight *b, const float *x, float *ya, float *yb,
                            hipStream_t s) {
    if (!gemv_dual_supports(a, b, 1)) return hipErrorInvalidValue;
    switch (q4k_f32_xr(a, Q4K_F32_THREADS)) {
    case 1: return launch_dual_t<1>(a, b, x, ya, yb, s);
    case 2: return launch_dual_t<2>(a, b, x, ya, yb, s);
    case 3: return launch_dual_t<3>(a, b, x, ya, yb, s);
    default: return launch_dual_t<4>(a, b, x, ya, yb, s);
    }
}

// LDS of gemv_q4k_pairs with g workgroups per pair.
static size_t q4k_pairs_lds(const arfq_weight *w, int64_t g) { return q4k_f32_lds_rows(w, (w->n + g - 1) / g); }

bool gemv_pairs_supports(const arfq_weight *w) {
    return w->qtype == ARFQ_Q4_K && w->k % 256 == 0 && w->n * (w->k / 256) * 128 < (int64_t)Q4K_OOB &&
           q4k_pairs_lds(w, 1) <= Q4K_F32_LDS_MAX && (w->k / 256 + 3) / 4 <= 64;
}

// Workgroups per CU of the decode-pair GEMVs: two, or one for up to 8 pairs (one token's
// top-8: C5's experts at T = 1 ran 21.9 us against 23.2 with two, while at T = 4 and 16
// one per CU was 9 % and 13 % slower).
static int pairs_per_cu(int64_t P) { return P <= 8 ? 1 : 2; }

template <class XS>
static hipError_t launch_pairs_t(const arfq_weight *w, int64_t P, const int32_t *ids, const XS &xs,
                                 float *y, hipStream_t s) {
    const int cus = w->ctx->cus > 0 ? w->ctx->cus : 256;
    // about two workgroups per CU over all pairs (one at a single token's pairs), >= 4 rows
    // per workgroup
    const int64_t g = std::max<int64_t>(1, std::min<int64_t>((pairs_per_cu(P) * (int64_t)cus + P - 1) / P, w->n / 4));
    const int64_t nb = w->n * (w->k / 256);
    const dim3 grid((unsigned)g, (unsigned)P);
    const int nsub = (int)(w->k / 32);
    const size_t lds = q4k_pairs_lds(w, g);
    if (nsub * 4 <= Q4K_GEMV_THREADS) {
        static std::atomic<uint64_t> lds_set{0};
        if (hipError_t err = set_max_lds_once((const void *)gemv_q4k_pairs<1, XS>, Q4K_F32_LDS_MAX, lds_set))
            return err;
        gemv_q4k_pairs<1, XS><<<grid, Q4K_GEMV_THREADS, lds, s>>>(
            (const uint8_t *)w->s0, (const uint8_t *)w->s1, (uint32_t)(nb * 16), (uint32_t)(nb * 128), xs, y,
            (int)w->n, (int)(w->k / 256), ids, w->experts);
    } else {
        static std::atomic<uint64_t> lds_set{0};
        if (hipError_t err = set_max_lds_once((const void *)gemv_q4k_pairs<2, XS>, Q4K_F32_LDS_MAX, lds_set))
            return err;
        gemv_q4k_pairs<2, XS><<<grid, Q4K_GEMV_THREADS, lds, s>>>(
            (const uint8_t *)w->s0, (const uint8_t *)w->s1, (uint32_t)(nb * 16), (uint32_t)(nb * 128), xs, y,
            (int)w->n, (int)(w->k / 256), ids, w->experts);
    }
    return hipGetLastError();
}

template <int MX, int XR, int ACT>
static hipError_t launch_glu_t(const arfq_weight *w, int m, const float *g, const float *u, float *y,
                               hipStream_t s) {
    const int64_t nb = w->n * (w->k / 256);
    gemv_q4k_glu<MX, XR, ACT><<<(unsigned)q4k_gemv_grid(w), Q4K_GEMV_THREADS, q4k_gemv_lds(w, MX), s>>>(
        (const uint8_t *)w->s0, (uint32_t)(nb * 16), (const uint8_t *)w->s1, (uint32_t)(nb * 128), g, u,
        y, (int)w->n, (int)(w->k / 256), m);
    return hipGetLastError();
}
template <int MX, int ACT>
static hipError_t launch_glu_mx(const arfq_weight *w, int m, const float *g, const float *u, float *y,
                                hipStream_t s) {
    const int64_t rounds = ((int64_t)m * (w->k / 8) + Q4K_GEMV_THREADS - 1) / Q4K_GEMV_THREADS;
    if (rounds <= 1) return launch_glu_t<MX, 1, ACT>(w, m, g, u, y, s);
    if (rounds <= 2) return launch_glu_t<MX, 2, ACT>(w, m, g, u, y, s);
    return launch_glu_t<MX, 4, ACT>(w, m, g, u, y, s);
}
template <int ACT>
static hipError_t launch_gemv_glu_t(const arfq_weight *w, int64_t m, const float *g, const float *u, float *y,
                                    hipStream_t s, bool x16) {
    if (x16 && q4k_x16_ok(w, m)) {
        if (m == 1) return launch_glu_mx<1, ACT>(w, 1, g, u, y, s);
        if (m == 2) return launch_glu_mx<2, ACT>(w, 2, g, u, y, s);
        return launch_glu_mx<4, ACT>(w, (int)m, g, u, y, s);
    }
    return launch_q4k_f32_glu<ACT>(w, g, u, y, s);  // m == 1, q4k_f32s_ok
}
// The activation applied as the down GEMV reads its x: every workgroup then
// evaluates it over all of x (exp / tanh and an IEEE divide per element), which
// at the decode FFN's inter 17408 cost more than a launch of its own (the
// separate activation kernel, then the plain GEMV: 40.9 -> 38.9 and 41.1 ->
// 40.4 us per FFN on two boxes), so only up to GLU_FUSE_MAX_K elements of x (8192 for the
// 1024-thread f32 kernel, half that for the 512-thread 16-bit one).
constexpr int64_t GLU_FUSE_MAX_K = 8192;
// what launch_gemv_glu_t takes: the 16-bit kernel under x16 where it fits,
// otherwise the f32 kernel at m = 1, both up to those k
bool gemv_glu_supports(const arfq_weight *w, int64_t m, bool x16) {
    if (w->qtype != ARFQ_Q4_K || w->experts != 1) return false;
    if (x16 && q4k_x16_ok(w, m)) return w->k <= GLU_FUSE_MAX_K / 2;
    return m == 1 && q4k_f32s_ok(w) && w->k <= GLU_FUSE_MAX_K;
}
hipError_t launch_gemv_glu(const arfq_weight *w, int64_t m, const float *g, const float *u, float *y, int act,
                           hipStream_t s, bool x16) {
    if (!gemv_glu_supports(w, m, x16)) return hipErrorInvalidValue;
    if (act == ACT_GELU_TANH) return launch_gemv_glu_t<ACT_GELU_TANH>(w, m, g, u, y, s, x16);
    if (act == ACT_SILU) return launch_gemv_glu_t<ACT_SILU>(w, m, g, u, y, s, x16);
    return hipErrorInvalidValue;
}

template <class XS>
static hipError_t launch_pairs_dual_t(const arfq_weight *w0, const arfq_weight *w1, int64_t P,
                                      const int32_t *ids, const XS &xs, float *y0, float *y1, hipStream_t s) {
    const int cus = w0->ctx->cus > 0 ? w0->ctx->cus : 256;
    // about two workgroups per CU over both weights' pairs (one at a single token's pairs),
    // >= 4 rows per workgroup
    const int64_t g = std::max<int64_t>(
        1, std::min<int64_t>((pairs_per_cu(P) * (int64_t)cus + 2 * P - 1) / (2 * P), w0->n / 4));
    const int64_t nb = w0->n * (w0->k / 256);
    const dim3 grid((unsigned)g, (unsigned)P, 2);
    const size_t lds = q4k_pairs_lds(w0, g);
    auto go = [&](auto kern) -> hipError_t {
        static std::atomic<uint64_t> lds_set{0};
        if (hipError_t err = set_max_lds_once((const void *)kern, Q4K_F32_LDS_MAX, lds_set)) return err;
        kern<<<grid, Q4K_GEMV_THREADS, lds, s>>>((const uint8_t *)w0->s0, (const uint8_t *)w0->s1,
                                                 (const uint8_t *)w1->s0, (const uint8_t *)w1->s1,
                                                 (uint32_t)(nb * 16), (uint32_t)(nb * 128), xs, y0, y1,
                                                 (int)w0->n, (int)(w0->k / 256), ids, w0->experts);
        return hipGetLastError();
    };
    if ((int)(w0->k / 32) * 4 <= Q4K_GEMV_THREADS) return go(gemv_q4k_pairs_dual<1, XS>);
    return go(gemv_q4k_pairs_dual<2, XS>);
}

bool gemv_pairs_dual_supports(const arfq_weight *w0, const arfq_weight *w1) {
    return gemv_pairs_supports(w0) && gemv_pairs_supports(w1) && w1->qtype == w0->qtype &&
           w1->n == w0->n && w1->k == w0->k && w1->experts == w0->experts;
}

hipError_t launch_gemv_pairs_dual(const arfq_weight *w0, const arfq_weight *w1, int64_t P, const int32_t *ids,
                                  const void *x, int x_dtype, int x_div, float *y0, float *y1, hipStream_t s) {
    if (P == 0) return hipSuccess;
    if (!gemv_pairs_dual_supports(w0, w1) || P > 65535) return hipErrorInvalidValue;
    if (x_dtype == ARFQ_F16)
        return launch_pairs_dual_t(w0, w1, P, ids, XsRowF16{(const _Float16 *)x, w0->k, x_div}, y0, y1, s);
    return launch_pairs_dual_t(w0, w1, P, ids, XsRowF32{(const float *)x, w0->k, x_div}, y0, y1, s);
}

hipError_t launch_gemv_pairs(const arfq_weight *w, int64_t P, const int32_t *ids, const void *x,
                             int x_dtype, int x_div, const float *g, const float *u, float *y,
                             hipStream_t s) {
    if (P == 0) return hipSuccess;
    if (!gemv_pairs_supports(w) || P > 65535) return hipErrorInvalidValue;
    if (g) return launch_pairs_t(w, P, ids, XsSwiglu{g, u, w->k}, y, s);
    if (x_dtype == ARFQ_F16)
        return launch_pairs_t(w, P, ids, XsRowF16{(const _Float16 *)x, w->k, x_div}, y, s);
    return launch_pairs_t(w, P, ids, XsRowF32{(const float *)x, w->k, x_div}, y, s);
}

hipError_t launch_gemv(const arfq_weight *w, int e, int64_t m, const float *x, float *y,
                       hipStream_t s, bool x16) {
    if (!gemv_supports(w, m, x16)) return hipErrorInvalidValue;
    if (w->qtype == ARFQ_Q4_K) {
        if (x16 && q4k_x16_ok(w, m)) {
            if (m == 1) return launch_gemv_q4k<1>(w, e, 1, x, y, s);
            if (m == 2) return launch_gemv_q4k<2>(w, e, 2, x, y, s);
            return launch_gemv_q4k<4>(w, e, (int)m, x, y, s);
        }
        return launch_q4k_f32(w, e, x, y, s);  // m == 1, q4k_f32s_ok
    }
    if (w->qtype == ARFQ_Q5_K) {
        const DotQ5K f = dot_q5k(w, e);
        if (x16 && dot_ok(w, m)) {
            if (m == 1) return launch_dot<DotQ5K, 1>(f, w, 1, x, y, s);
            if (m == 2) return launch_dot<DotQ5K, 2>(f, w, 2, x, y, s);
            return launch_dot<DotQ5K, 4>(f, w, (int)m, x, y, s);
        }
        return launch_dot_f32(f, w, x, y, s);  // m == 1, dot_f32_ok
    }
    if (w->qtype == ARFQ_IQ4_XS) {
        const DotIQ4XS f = dot_iq4xs(w, e);
        if (x16 && dot_ok(w, m)) {
            if (m == 1) return launch_dot<DotIQ4XS, 1>(f, w, 1, x, y, s);
            if (m == 2) return launch_dot<DotIQ4XS, 2>(f, w, 2, x, y, s);
            return launch_dot<DotIQ4XS, 4>(f, w, (int)m, x, y, s);
        }
        return launch_dot_f32(f, w, x, y, s);  // m == 1, dot_f32_ok
    }
    if (w->qtype == ARFQ_Q6_K) {
        if (x16 && dot_ok(w, m)) {
            const DotQ6K f = dot_q6k(w, e);
            return m == 1 ? launch_dot<DotQ6K, 1>(f, w, 1, x, y, s) : launch_dot<DotQ6K, 2>(f, w, 2, x, y, s);
        }
        if (m == 1 && dot_f32_ok(w)) return launch_dot_f32(dot_q6k(w, e), w, x, y, s);
    }
    if (w->qtype == ARFQ_Q8_0) {
        if (m == 1) return launch_q80<1>(w, e, 1, x, y, s);
        if (m == 2) return launch_q80<2>(w, e, 2, x, y, s);
        return launch_q80<4>(w, e, (int)m, x, y, s);
    }
    // Q6_K, f32: gemv_q6k
    if (m == 1) return launch_gemv_t<4, 1>(w, e, 1, x, y, s);
    if (m == 2) return launch_gemv_t<4, 2>(w, e, 2, x, y, s);
    return launch_gemv_t<2, 4>(w, e, (int)m, x, y, s);
}

}  // namespace arfq
