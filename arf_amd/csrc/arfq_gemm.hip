// arfq_gemm.hip -- dequant-into-LDS MFMA GEMM for prefill and batched decode:
// y[m, n] (f32) = x[m, k] . W[n, k]^T with W in Q4_K, Q6_K or Q8_0.
//
// Workgroup tile: BM (x rows, 64 or 128) x 128 (weight rows), 256 threads in
// a 2 x 2 wave grid; each wave owns (BM/2) x 64 of the output as 32 x 32 tiles
// of v_mfma_f32_32x32x16_f16 with f32 accumulation.  K advances in steps of 64
// "slots".  Each step the workgroup
//   * dequantizes 128 weight rows x 64 slots to f16 in LDS (one 32-slot half
//     row per thread, weight in f32 then rounded to nearest f16),
//   * copies the matching f16 x tile into LDS,
//   * runs the MFMAs out of LDS (double buffered; rows padded by 16 bytes so
//     the 16-byte LDS reads of the MFMA operands are conflict-free).
// The next step's global loads are issued before the current step's MFMAs.
// Weight loads are ordinary (cached) loads: every weight tile is read by all
// the M tiles, and the XCD-aware order below keeps those re-reads in cache.
// A step's 64 slots are one natural unit of the format (two Q4_K sub-blocks,
// one 48-byte Q6_K chunk, two Q8_0 blocks); the x tile is gathered with the
// same slot -> k permutation, so the dot product is unchanged.
//
// Activations: f16 as given, or (XSPLIT) an f32 x pre-split into x = hi + lo
// with hi, lo in f16: two MFMAs per tile carry ~22 bits of x, so the only
// rounding left is the weights' f16 rounding.
// Skinny shapes use split-K: grid.y splits the steps, each split writes its
// own partial [m, n] slice and an ordered reduction adds them (deterministic).
//
// Reference behaviour: matmul_mm_q4ks.metal:65-290 (dequantize a weight tile
// into threadgroup memory as half, activations as half, simdgroup MMA with f32
// accumulation); oracles matmul_nt_q4ks / matmul_nt_q8_0
// (crates/arf-ml/src/matmul.rs:174-204, 363-400) and dequant_q6_k + matmul_nt.
//
// Workgroup -> tile order is XCD-aware when the M tiles divide by 8: the
// dispatcher places workgroup b on XCD b % 8, so XCD x keeps a fixed set of x
// tiles (which stay in its L2) and walks the weight tiles, which stream from
// the MALL.
#include "arfq_common.h"
#include "arfq_internal.h"

#include <algorithm>

namespace arfq {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int GM_BN = 128, GM_BK = 64, GM_THREADS = 256;
constexpr int GM_LD = GM_BK + 8;  // halves per LDS row (16 bytes of padding)

__host__ __device__ constexpr size_t gm_lds(int BM, bool xsplit) {
    return (size_t)2 * ((xsplit ? 2 : 1) * BM + GM_BN) * GM_LD * sizeof(_Float16);
}

__device__ __forceinline__ uint32_t pack2h(float a, float b) {
    const __half ha = __float2half_rn(a), hb = __float2half_rn(b);
    return (uint32_t)__half_as_ushort(ha) | ((uint32_t)__half_as_ushort(hb) << 16);
}

// ---- weight formats --------------------------------------------------------
// xk(st, q): k index of slot 8q of step st (slots 8q..8q+7 are 8 consecutive
// k);  load(): the raw data of half `ws` of weight row `row` for step st;
// deq(): its 32 weights as f16 pairs, o[4r..4r+3] = the 8 halves stored at
// slot run_off(ws, r).

// Q4_K: step st = sub-blocks 2p, 2p+1 (p = st % 4) of block st / 4; half ws =
// sub-block 2p + ws, slots 32ws + e = element 64p + 32ws + e.
struct FmtQ4K {
    struct Raw {
        uint4 c, h;
    };
    const uint4 *hdr, *qs;
    int nblk;
    __device__ static int xk(int st, int q) { return (st >> 2) * 256 + 64 * (st & 3) + 8 * q; }
    __device__ static int run_off(int ws, int r) { return 32 * ws + 8 * r; }
    __device__ Raw load(int64_t row, int st, int ws) const {
        const int64_t blk = row * nblk + (st >> 2);
        Raw r;
        r.c = qs[blk * 8 + 2 * (st & 3) + ws];
        r.h = hdr[blk];
        return r;
    }
    __device__ static void deq(const Raw &r, int st, int ws, uint32_t o[16]) {
        const int j = 2 * (st & 3) + ws;
        uint32_t sc, mm;
        q4k_scale_min(r.h.y, r.h.z, r.h.w, j, sc, mm);
        const float d1 = h2f(r.h.x) * (float)sc;
        const float m1 = h2f(r.h.x >> 16) * (float)mm;
        const uint32_t cw[4] = {r.c.x, r.c.y, r.c.z, r.c.w};
#pragma unroll
        for (int w = 0; w < 4; w++) {
            // dword w: byte i low nibble = element 8w+i, high nibble = element 8w+4+i
            const uint32_t lo = cw[w] & 0x0F0F0F0Fu, hi = (cw[w] >> 4) & 0x0F0F0F0Fu;
            o[4 * w + 0] = pack2h(fmaf(d1, (float)(lo & 0xffu), -m1), fmaf(d1, (float)((lo >> 8) & 0xffu), -m1));
            o[4 * w + 1] = pack2h(fmaf(d1, (float)((lo >> 16) & 0xffu), -m1), fmaf(d1, (float)(lo >> 24), -m1));
            o[4 * w + 2] = pack2h(fmaf(d1, (float)(hi & 0xffu), -m1), fmaf(d1, (float)((hi >> 8) & 0xffu), -m1));
            o[4 * w + 3] = pack2h(fmaf(d1, (float)((hi >> 16) & 0xffu), -m1), fmaf(d1, (float)(hi >> 24), -m1));
        }
    }
};

// Q6_K: step st = 48-byte chunk c = st % 4 of block st / 4 (n2 = c/2,
// isub = c%2); slot 16t + i is element 128*n2 + 16*isub + 32t + i (quadrant t,
// position i).  Half ws holds positions 8ws..8ws+7 of all four quadrants.
struct FmtQ6K {
    struct Raw {
        uint2 qa, qb, qh, sc;
        uint32_t d;
    };
    const uint2 *qb8;  // the 192-byte chunk streams as 8-byte units
    const uint2 *sc8;  // 16 scale bytes per block as 8-byte units
    const uint16_t *dd;
    int nblk;
    __device__ static int xk(int st, int q) {
        const int c = st & 3;
        return (st >> 2) * 256 + 128 * (c >> 1) + 16 * (c & 1) + 32 * (q >> 1) + 8 * (q & 1);
    }
    __device__ static int run_off(int ws, int r) { return 16 * r + 8 * ws; }
    __device__ Raw load(int64_t row, int st, int ws) const {
        const int64_t blk = row * nblk + (st >> 2);
        const int c = st & 3;
        const uint2 *ch = qb8 + blk * 24 + c * 6;  // ql_a[16] | ql_b[16] | qh[16]
        Raw r;
        r.qa = ch[ws];
        r.qb = ch[2 + ws];
        r.qh = ch[4 + ws];
        r.sc = sc8[blk * 2 + (c >> 1)];  // scales 8*n2 .. 8*n2+7
        r.d = dd[blk];
        return r;
    }
    __device__ static void deq(const Raw &r, int st, int, uint32_t o[16]) {
        const int isub = st & 1;
        const float d = h2f(r.d);
        const uint32_t scw[2] = {r.sc.x, r.sc.y};
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int si = isub + 2 * t;  // scale 8*n2 + isub + 2t
            const float s = d * (float)(int8_t)(scw[si >> 2] >> (8 * (si & 3)));
            const float m32 = -32.f * s;
            // t=0: ql_a low | qh bits 0-1;  t=1: ql_b low | qh 2-3;
            // t=2: ql_a high | qh 4-5;      t=3: ql_b high | qh 6-7
            const uint2 ql = (t & 1) ? r.qb : r.qa;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint32_t l = h ? ql.y : ql.x, hh = h ? r.qh.y : r.qh.x;
                const uint32_t nib = (t & 2) ? ((l >> 4) & 0x0F0F0F0Fu) : (l & 0x0F0F0F0Fu);
                const uint32_t q = nib | (((hh >> (2 * t)) & 0x03030303u) << 4);
                // s*q - 32s with one rounding == (d*sc)*(q-32) in f32
                o[4 * t + 2 * h] = pack2h(fmaf((float)(q & 0xffu), s, m32), fmaf((float)((q >> 8) & 0xffu), s, m32));
                o[4 * t + 2 * h + 1] = pack2h(fmaf((float)((q >> 16) & 0xffu), s, m32), fmaf((float)(q >> 24), s, m32));
            }
        }
    }
};

// Q8_0: step st = blocks 2st, 2st+1; half ws = block 2st + ws.
struct FmtQ80 {
    struct Raw {
        uint4 a, b;
        uint32_t d;
    };
    const uint4 *qs;
    const uint16_t *dd;
    int nblk;
    __device__ static int xk(int st, int q) { return st * 64 + 8 * q; }
    __device__ static int run_off(int ws, int r) { return 32 * ws + 8 * r; }
    __device__ Raw load(int64_t row, int st, int ws) const {
        const int64_t blk = row * nblk + 2 * st + ws;
        Raw r;
        r.a = qs[blk * 2];
        r.b = qs[blk * 2 + 1];
        r.d = dd[blk];
        return r;
    }
    __device__ static void deq(const Raw &r, int, int, uint32_t o[16]) {
        const float d = h2f(r.d);
        const uint32_t cw[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
        for (int w = 0; w < 8; w++) {
            const uint32_t v = cw[w];
            o[2 * w] = pack2h(d * (float)(int8_t)(v & 0xffu), d * (float)(int8_t)((v >> 8) & 0xffu));
            o[2 * w + 1] = pack2h(d * (float)(int8_t)((v >> 16) & 0xffu), d * (float)(int8_t)(v >> 24));
        }
    }
};

// ---- the GEMM --------------------------------------------------------------
template <class F, int BM, bool XSPLIT>
__global__ __launch_bounds__(GM_THREADS) void gemm_q(
    F fmt, const _Float16 *__restrict__ xh, const _Float16 *__restrict__ xl, float *__restrict__ y,
    int M, int N, int K, int mt, int xcd_order) {
    constexpr int TA = BM / 64;         // 32-row MFMA tiles per wave along m
    constexpr int XI = BM / 32;         // 16-byte x loads per thread and x matrix
    constexpr int NA = XSPLIT ? 2 : 1;  // x matrices (hi, lo)
    constexpr int ATILE = BM * GM_LD, BTILE = GM_BN * GM_LD;
    constexpr int STAGE = NA * ATILE + BTILE;
    extern __shared__ _Float16 lds[];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;

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
    const int m0 = tm * BM, n0 = tn * GM_BN;
    // split-K: this workgroup's range of steps
    const int nsteps = K / GM_BK;
    const int S = gridDim.y, sp = blockIdx.y;
    const int st0 = (int)((int64_t)sp * nsteps / S), st1 = (int)((int64_t)(sp + 1) * nsteps / S);

    // x: XI x 16 B per thread and matrix: row (tid>>3) + 32*i, slot run tid&7
    const int xr = tid >> 3, xq = tid & 7;
    // W: weight row n0 + (tid>>1), half tid&1
    const int wr = tid >> 1, ws = tid & 1;
    const int64_t wrow = min(n0 + wr, N - 1);  // rows past N are computed, never stored

    // x hi (or x) and x lo; a native vector type: arrays of the HIP uint4
    // struct were left in scratch memory by the compiler here
    u32x4 xa[XI], xb[XSPLIT ? XI : 1];
    typename F::Raw wv;
    auto gload = [&](int st) {
        const int kx = F::xk(st, xq);
#pragma unroll
        for (int i = 0; i < XI; i++) {
            const int64_t row = min(m0 + xr + 32 * i, M - 1);  // rows past M are never stored
            xa[i] = *reinterpret_cast<const u32x4 *>(xh + row * K + kx);
            if constexpr (XSPLIT) xb[i] = *reinterpret_cast<const u32x4 *>(xl + row * K + kx);
        }
        wv = fmt.load(wrow, st, ws);
    };
    auto lstore = [&](int buf, int st) {
        _Float16 *As = lds + buf * STAGE;
        _Float16 *Bs = As + NA * ATILE;
#pragma unroll
        for (int i = 0; i < XI; i++) {
            *reinterpret_cast<u32x4 *>(As + (xr + 32 * i) * GM_LD + 8 * xq) = xa[i];
            if constexpr (XSPLIT)
                *reinterpret_cast<u32x4 *>(As + ATILE + (xr + 32 * i) * GM_LD + 8 * xq) = xb[i];
        }
        uint32_t o[16];
        F::deq(wv, st, ws, o);
#pragma unroll
        for (int r = 0; r < 4; r++)
            *reinterpret_cast<uint4 *>(Bs + wr * GM_LD + F::run_off(ws, r)) =
                make_uint4(o[4 * r], o[4 * r + 1], o[4 * r + 2], o[4 * r + 3]);
    };

    floatx16 acc[TA][2];
#pragma unroll
    for (int a = 0; a < TA; a++)
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
            for (int i = 0; i < 16; i++) acc[a][b][i] = 0.f;

    const int lr = lane & 31, lk = (lane >> 5) * 8;
    if (st0 < st1) {
        gload(st0);
        lstore(0, st0);
    }
    __syncthreads();
    for (int st = st0; st < st1; st++) {
        const int buf = (st - st0) & 1;
        if (st + 1 < st1) gload(st + 1);
        const _Float16 *As = lds + buf * STAGE;
        const _Float16 *Bs = As + NA * ATILE;
#pragma unroll
        for (int kk = 0; kk < GM_BK / 16; kk++) {
            half8 af[NA][TA], bf[2];
#pragma unroll
            for (int a = 0; a < NA; a++)
#pragma unroll
                for (int t = 0; t < TA; t++)
                    af[a][t] = *reinterpret_cast<const half8 *>(
                        As + a * ATILE + (wm * (BM / 2) + 32 * t + lr) * GM_LD + 16 * kk + lk);
#pragma unroll
            for (int t = 0; t < 2; t++)
                bf[t] = *reinterpret_cast<const half8 *>(Bs + (wn * 64 + 32 * t + lr) * GM_LD + 16 * kk + lk);
#pragma unroll
            for (int a = 0; a < NA; a++)
#pragma unroll
                for (int t = 0; t < TA; t++)
#pragma unroll
                    for (int b = 0; b < 2; b++)
                        acc[t][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[a][t], bf[b], acc[t][b], 0, 0, 0);
        }
        if (st + 1 < st1) lstore(buf ^ 1, st + 1);
        __syncthreads();
    }
    // epilogue: lane holds column lane%32 of each 32x32 tile, rows
    // 8*(i/4) + 4*(lane/32) + i%4; split sp writes its own [M, N] slice
    float *out = y + (int64_t)sp * M * N;
#pragma unroll
    for (int t = 0; t < TA; t++) {
#pragma unroll
        for (int b = 0; b < 2; b++) {
            const int n = n0 + wn * 64 + 32 * b + lr;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int m = m0 + wm * (BM / 2) + 32 * t + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
                if (m < M && n < N) out[(int64_t)m * N + n] = acc[t][b][i];
            }
        }
    }
}

// y[i] = part[0][i] + part[1][i] + ... in split order
__global__ void splitk_reduce(const float *__restrict__ part, float *__restrict__ y, int64_t n,
                              int S) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float v = part[i];
    for (int s = 1; s < S; s++) v += part[(int64_t)s * n + i];
    y[i] = v;
}

// x (f32) -> hi = f16(x), lo = f16(x - hi)
__global__ void split_f32_kernel(const float *__restrict__ x, __half *__restrict__ hi,
                                 __half *__restrict__ lo, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = x[i];
    const __half h = __float2half_rn(v);
    hi[i] = h;
    lo[i] = __float2half_rn(v - __half2float(h));
}

__global__ void f32_to_f16_kernel(const float *__restrict__ x, __half *__restrict__ y, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = __float2half_rn(x[i]);
}

hipError_t launch_f32_to_f16(const float *x, __half *y, int64_t n, hipStream_t s) {
    f32_to_f16_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(x, y, n);
    return hipGetLastError();
}

hipError_t launch_split_f32(const float *x, __half *hi, __half *lo, int64_t n, hipStream_t s) {
    split_f32_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(x, hi, lo, n);
    return hipGetLastError();
}

bool gemm_supports(const arfq_weight *w, int64_t m) {
    if (m < 1 || m > INT32_MAX / 2 || w->n > INT32_MAX / 2 || w->k > INT32_MAX / 2) return false;
    switch (w->qtype) {
    case ARFQ_Q4_K:
    case ARFQ_Q6_K: return true;
    case ARFQ_Q8_0: return w->k % GM_BK == 0;
    default: return false;
    }
}

GemmPlan gemm_plan(const arfq_weight *w, int64_t m, bool xsplit) {
    GemmPlan p;
    p.bm = m > 64 ? 128 : 64;
    p.xsplit = xsplit;
    const int64_t mt = (m + p.bm - 1) / p.bm, nt = (w->n + GM_BN - 1) / GM_BN;
    const int nsteps = (int)(w->k / GM_BK);
    const int cus = w->ctx && w->ctx->cus > 0 ? w->ctx->cus : 256;
    // split K until ~2 workgroups per CU are in flight, keeping >= 8 steps a split
    int64_t S = std::max<int64_t>(1, (2 * (int64_t)cus) / std::max<int64_t>(1, mt * nt));
    S = std::min<int64_t>(S, std::max(1, nsteps / 8));
    p.splits = (int)std::min<int64_t>(S, 16);
    return p;
}

template <class F, int BM, bool XS>
static hipError_t launch_gemm_t(const F &fmt, const arfq_weight *w, int64_t m, const _Float16 *xh,
                                const _Float16 *xl, float *out, int S, hipStream_t s) {
    static bool attr_set = false;  // the attribute belongs to the kernel: set once per process
    constexpr size_t lds = gm_lds(BM, XS);
    if (!attr_set) {
        hipError_t err = hipFuncSetAttribute((const void *)gemm_q<F, BM, XS>,
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (err != hipSuccess) return err;
        attr_set = true;
    }
    const int mt = (int)((m + BM - 1) / BM), nt = (int)((w->n + GM_BN - 1) / GM_BN);
    const int xcd = (mt % 8 == 0) ? 1 : 0;
    const dim3 grid((unsigned)(mt * nt), (unsigned)S);
    gemm_q<F, BM, XS><<<grid, GM_THREADS, lds, s>>>(fmt, xh, xl, out, (int)m, (int)w->n, (int)w->k,
                                                   mt, xcd);
    return hipGetLastError();
}

template <class F>
static hipError_t launch_fmt(const F &fmt, const arfq_weight *w, int64_t m, const _Float16 *xh,
                             const _Float16 *xl, float *out, const GemmPlan &p, hipStream_t s) {
    if (p.bm == 128)
        return p.xsplit ? launch_gemm_t<F, 128, true>(fmt, w, m, xh, xl, out, p.splits, s)
                        : launch_gemm_t<F, 128, false>(fmt, w, m, xh, xl, out, p.splits, s);
    return p.xsplit ? launch_gemm_t<F, 64, true>(fmt, w, m, xh, xl, out, p.splits, s)
                    : launch_gemm_t<F, 64, false>(fmt, w, m, xh, xl, out, p.splits, s);
}

hipError_t launch_gemm(const arfq_weight *w, int e, int64_t m, const _Float16 *xh,
                       const _Float16 *xl, float *y, float *partials, const GemmPlan &p,
                       hipStream_t s) {
    if (p.xsplit != (xl != nullptr) || (p.splits > 1 && !partials)) return hipErrorInvalidValue;
    float *out = p.splits > 1 ? partials : y;
    hipError_t err;
    switch (w->qtype) {
    case ARFQ_Q4_K: {
        const int nblk = (int)(w->k / 256);
        const int64_t eb = (int64_t)e * w->n * nblk;
        const FmtQ4K f{(const uint4 *)w->s0 + eb, (const uint4 *)w->s1 + eb * 8, nblk};
        err = launch_fmt(f, w, m, xh, xl, out, p, s);
        break;
    }
    case ARFQ_Q6_K: {
        const int nblk = (int)(w->k / 256);
        const int64_t eb = (int64_t)e * w->n * nblk;
        const FmtQ6K f{(const uint2 *)w->s0 + eb * 24, (const uint2 *)w->s1 + eb * 2,
                       (const uint16_t *)w->s2 + eb, nblk};
        err = launch_fmt(f, w, m, xh, xl, out, p, s);
        break;
    }
    case ARFQ_Q8_0: {
        const int nblk = (int)(w->k / 32);
        const int64_t eb = (int64_t)e * w->n * nblk;
        const FmtQ80 f{(const uint4 *)w->s0 + eb * 2, (const uint16_t *)w->s1 + eb, nblk};
        err = launch_fmt(f, w, m, xh, xl, out, p, s);
        break;
    }
    default:
        return hipErrorInvalidValue;
    }
    if (err != hipSuccess || p.splits == 1) return err;
    const int64_t n = m * w->n;
    splitk_reduce<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(partials, y, n, p.splits);
    return hipGetLastError();
}

}  // namespace arfq
