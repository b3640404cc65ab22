// arfq_gemm.hip -- dense dequant-into-LDS MFMA GEMM for prefill and batched
// decode: y[m, n] (f32) = x[m, k] . W[n, k]^T with W in Q4_K, Q6_K, Q8_0, Q5_K
// or IQ4_XS.
// The tile loop (LDS staging, dequant, MFMA) is in arfq_gemm_tile.h.
//
// Skinny shapes use split-K: grid.y splits the K steps, each split writes its
// own partial [m, n] slice and an ordered reduction adds them (deterministic).
// Workgroup -> tile order is XCD-aware when the M tiles divide by 8: the
// dispatcher places workgroup b on XCD b % 8, so XCD x keeps a fixed set of x
// tiles (which stay in its L2) and walks the weight tiles, which stream from
// the MALL.
//
// Reference behaviour: matmul_mm_q4ks.metal:65-290; oracles matmul_nt_q4ks /
// matmul_nt_q8_0 (crates/arf-ml/src/matmul.rs:174-204, 363-400) and
// dequant_q6_k / dequant_q5_k / dequant_iq4_xs + matmul_nt for the others.
#include "arfq_gemm_tile.h"
#include "arfq_internal.h"
#include "arfq_skinny.h"
#include "arfq_gemm_bd.h"

#include <algorithm>

namespace arfq {

template <class F, int BM, bool XSPLIT>
__global__ __launch_bounds__(GM_THREADS, F::WG_PER_CU) void gemm_q(
    F fmt, const _Float16 *__restrict__ xh, const _Float16 *__restrict__ xl,
    const uint16_t *__restrict__ xs, const float *__restrict__ rs, float *__restrict__ y, int M,
    int N, int K, int mt, int xcd_order) {
    extern __shared__ __attribute__((aligned(16))) _Float16 lds[];
    const int tid = threadIdx.x;
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
    // split-K: this workgroup's range of steps (whole 256-element blocks for
    // the exact formats)
    const int S = gridDim.y, sp = blockIdx.y;
    const int unit = F::PHASED ? 4 : 1;  // steps whose decode depends on st % 4 start blocks
    const int nu = K / GM_BK / unit;
    const int st0 = unit * (int)((int64_t)sp * nu / S);
    const int st1 = unit * (int)((int64_t)(sp + 1) * nu / S);

    int64_t xrow[BM / 32], xsrow[BM / 32];
#pragma unroll
    for (int i = 0; i < BM / 32; i++) {  // rows past M are loaded (clamped), never stored
        const int64_t r = min(m0 + (tid >> 3) + 32 * i, M - 1);
        xrow[i] = r * K;
        xsrow[i] = r * (K / 16);
    }
    const int64_t wrow = min(n0 + (tid >> 1), N - 1);  // rows past N: computed, never stored

    floatx16 acc[BM / 64][2];
#pragma unroll
    for (int t = 0; t < BM / 64; t++)
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
            for (int i = 0; i < 16; i++) acc[t][b][i] = 0.f;
    gemm_tile_run<F, BM, XSPLIT>(fmt, wrow, xrow, xsrow, xh, xl, xs, st0, st1, acc, lds);

    // split sp writes its own [M, N] slice
    float *out = y + (int64_t)sp * M * N;
#pragma unroll
    for (int t = 0; t < BM / 64; t++) {
#pragma unroll
        for (int b = 0; b < 2; b++) {
            const int n = n0 + tile_out_col(b);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int m = m0 + tile_out_row<BM>(t, i);
                if (m < M && n < N) out[(int64_t)m * N + n] = rs ? acc[t][b][i] * rs[m] : acc[t][b][i];
            }
        }
    }
}

// threads and weight rows (column tile) of a skinny workgroup with TA x tiles
__host__ __device__ constexpr int sk_nt(int ta) { return ta == 4 ? 512 : SK_THREADS; }
__host__ __device__ constexpr int sk_ct(int ta) { return sk_nt(ta) / 2; }
// x buffers of the dense skinny loop: two (one barrier per block instead of
// two) where the second fits beside two workgroups per CU (one x tile: C3 m = 8
// 31.7 -> 31.2 us), else one
__host__ __device__ constexpr int SK_XB(int ta) { return ta == 1 ? 2 : 1; }

// Skinny products (m <= 64): workgroup = sk_ct(TA) weight rows x all m rows
// (a wave per 32 weight rows), over the 256-element blocks of split blockIdx.y
// (arfq_skinny.h).  x is f16, or f32
// rounded to f16 as it is staged.  With S = gridDim.y > 1 splits each
// workgroup stores its partial and sk_reduce_kernel, launched next, adds the S
// partials of every output in split order into y (deterministic: spread over
// every CU, where the last of a column tile's workgroups to arrive, summing
// them alone, left the chip idle for 4 / 9 / 18 us at C3 m = 8 / 32 / 64).
// An f32 x (XT = float, PARTS 3) is split into its three
// f16 parts (and their sub-block sums) as it is staged, the scales of its K
// range worked out here (no separate preparation launch).
// (held to 256 VGPRs: two 4-wave workgroups per CU; with four x tiles the LDS
// leaves room for one workgroup, of 8 waves: two per SIMD again)
template <class F, int TA, class XT, int PARTS, int GM = 0xFF>
__global__ __launch_bounds__(sk_nt(TA), TA == 4 ? 1 : 2) void gemm_sk(F fmt, const XT *__restrict__ x,
                                                      const uint16_t *__restrict__ xs,
                                                      const float *__restrict__ rs,
                                                      float *__restrict__ y, float *__restrict__ part,
                                                      int M, int N, int K,
                                                      int rss) {
    extern __shared__ __attribute__((aligned(16))) _Float16 lds[];
    constexpr int NT = sk_nt(TA), CT = NT / 2;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // (column tile, split) of this workgroup.  With four x tiles the
    // dispatcher's placement of workgroup L (x fastest) on XCD L % 8 is used:
    // XCD x takes items [x per, (x + 1) per) of the split-major order, a
    // contiguous run of splits whose x ranges then stay in its L2 (C3 m = 64:
    // x as 128 f16 rows is 4.5 MB, more than an L2; 52.1 -> 50.3 us); the last
    // total % 8 items go in order.  With one or two tiles (x within an L2)
    // that order measured slower (C3 m = 8: 27.7 -> 28.4 us, m = 32: 36.6 -> 37.9).
    const int nt = gridDim.x, total = nt * gridDim.y, per = total >> 3;
    const int L = blockIdx.y * nt + blockIdx.x;
    const int q = TA == 4 && L < 8 * per ? (L & 7) * per + (L >> 3) : L;
    const int tile = q % nt;
    const int n0 = tile * CT;
    const int nb = K / 256, S = gridDim.y, sp = q / nt;
    const int b0 = (int)((int64_t)sp * nb / S), b1 = (int)((int64_t)(sp + 1) * nb / S);
    // PARTS 2 (M <= 16 TA): x row r < M stages hi row r of x, row PO + r its lo
    // row M + r (PO = 16 in one 32-row tile, 32 = the second tile with two, 64 =
    // tiles 2 and 3 with four).
    // PARTS 3 (M <= 8, one tile): rows r, 8 + r and 16 + r stage the hi, mid and
    // lo rows r, M + r and 2M + r; a lane's accumulator holds rows r, r + 8 and
    // r + 16 of its column as elements i, i + 4 and i + 8.  Rows that stage
    // nothing read row 0 (their products land in rows never stored).
    constexpr bool PAIR = PARTS == 2;
    constexpr int PO = PARTS == 3 ? 8 : 16 * TA;
    static_assert(PARTS != 3 || TA == 1, "three parts fit one tile");
    constexpr bool FX = sizeof(XT) == 4;  // f32 x, split here
    static_assert(!FX || PARTS == 3, "an f32 x is split here into three parts only");
    const SkRows<TA, NT> rows =
        FX ? sk_rows<TA, NT>(M, K, [](int r) { return r; })
        : PARTS == 3 ? sk_rows<TA, NT>(16 + M, K, [M](int r) {
            return r < M ? r : r < 8 ? 0 : r < 8 + M ? M + r - 8 : r < 16 ? 0 : 2 * M + r - 16;
        })
        : PAIR ? sk_rows<TA, NT>(PO + M, K, [M](int r) { return r < M ? r : r >= PO ? M + r - PO : 0; })
               : sk_rows<TA, NT>(M, K, [](int r) { return r; });
    const int n = n0 + 32 * wave + (lane & 31);
    // the x rows' scales of this K range into LDS past the loop's own, before
    // the loop: the epilogue reads them there instead of loading per output
    float *lrs = reinterpret_cast<float *>(reinterpret_cast<char *>(lds) + sk_lds<F, TA, 1, NT, SK_XB(TA)>());
    if (rs && tid < 32 * TA) lrs[tid] = tid < M ? rs[(int64_t)sp * rss + tid] : 1.f;
    const F fm[1] = {fmt};
    const int64_t wrow0[1] = {n0 + 32 * wave};
    floatx16 acc[1][TA];
#pragma unroll
    for (int t = 0; t < TA; t++)
#pragma unroll
        for (int i = 0; i < 16; i++) acc[0][t][i] = 0.f;
    // PAIR with two or four tiles: the lo tiles' products go into the hi tiles' accumulators
    int xsh = 0;
    skinny_run<F, TA, 1, NT, XT, false, GM, PAIR && TA >= 2, true, SK_XB(TA), FX ? 3 : 0, FX>(
        fm, wrow0, N, rows, x, xs, b0, b1, acc, lds, PARTS == 3 ? 16 + M : PAIR ? PO + M : M, xsh);
    if constexpr (FX) {
        // the rows' scales over this K range (row tid / 32 from its lanes' xsh)
        if ((tid & 31) == 0) lrs[tid >> 5] = tid >> 5 < M ? ldexpf(1.f, -xsh) : 1.f;
        if (tid >= 8 && tid < 32) lrs[tid] = 1.f;
        __syncthreads();
    }
    if constexpr (PAIR && TA == 1) {
        // rows r and r + 16 of a lane's accumulator are elements i and i + 8
#pragma unroll
        for (int i = 0; i < 8; i++) acc[0][0][i] += acc[0][0][i + 8];
    }
    if constexpr (PARTS == 3) {
#pragma unroll
        for (int i = 0; i < 4; i++) acc[0][0][i] = (acc[0][0][i] + acc[0][0][i + 4]) + acc[0][0][i + 8];
    }
    if (S == 1) {
#pragma unroll
        for (int t = 0; t < TA; t++)
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int m = sk_out_row(t, i);
                // (m & 3 == i & 3: one 16-byte LDS read serves four rows)
                if (m < M && n < N)
                    y[(int64_t)m * N + n] =
                        FX || rs ? acc[0][t][i] * reinterpret_cast<const float4 *>(lrs)[m >> 2][i & 3]
                                 : acc[0][t][i];
            }
        return;
    }
    // x scaled per K range (rs[sp * rss + row]): the partial back to true units
    if (FX || rs) {
#pragma unroll
        for (int t = 0; t < TA; t++)
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int m = sk_out_row(t, i);
                acc[0][t][i] *= reinterpret_cast<const float4 *>(lrs)[m >> 2][i & 3];  // 1 past M
            }
    }
    // Split K.  Each wave stores its accumulators as they sit in registers:
    // float4 (row group gi = 4 t + g, lane) holds acc[t][4 g .. 4 g + 3], rows
    // 32 t + 8 g + 4 (lane / 32) + 0..3 of column n, for the GT 8-row groups
    // that hold rows < M; sk_reduce_kernel adds the splits (in split order)
    // after this launch.
    const int GT = (M + 7) >> 3;
    float4 *pw = reinterpret_cast<float4 *>(part) + ((((int64_t)sp * nt + tile) * (NT / 64) + wave) * GT) * 64 + lane;
#pragma unroll
    for (int t = 0; t < TA; t++)
#pragma unroll
        for (int g = 0; g < 4; g++)
            if (4 * t + g < GT)
                pw[(4 * t + g) * 64] = make_float4(acc[0][t][4 * g], acc[0][t][4 * g + 1], acc[0][t][4 * g + 2],
                                                   acc[0][t][4 * g + 3]);
}

// y of the skinny split-K: a thread per float4 of one split's partials, in the
// register order gemm_sk stores them ([split][column tile][wave][row group][lane]),
// its S splits added in split order; rows 32 t + 8 g + 4 (lane / 32) + 0..3 of
// column tile * ct + 32 wave + lane % 32 (row group gi = 4 t + g).  All S loads
// are in flight at once: straight-line code, the loads of splits past S reading
// past the end of the buffer, which returns 0 and moves no data (adding that 0
// changes nothing but a -0 sum into +0).
__global__ __launch_bounds__(256) void sk_reduce_kernel(const float *__restrict__ part, float *__restrict__ y,
                                                        int S, int nt, int nw, int GT, int ct, int M, int N) {
    const int64_t units = (int64_t)nt * nw * GT;  // float4 columns of one split, / 64
    const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (q >= units * 64) return;
    const int lane = (int)(q & 63);
    const int64_t u = q >> 6;
    const int gi = (int)(u % GT), wave = (int)((u / GT) % nw), tile = (int)(u / ((int64_t)GT * nw));
    const uint32_t split_bytes = (uint32_t)(units * 1024);
    const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(part), (short)0, (int)(split_bytes * (uint32_t)S), 0x00020000);
    u32x4 d[16];
#pragma unroll
    for (int j = 0; j < 16; j++)
        d[j] = __builtin_amdgcn_raw_buffer_load_b128(prs, ((uint32_t)j * split_bytes + (uint32_t)q * 16u) |
                                                              (uint32_t)(j >= S) << 31, 0, 0);
    float r[4];
#pragma unroll
    for (int c = 0; c < 4; c++) r[c] = __uint_as_float(d[0][c]);
#pragma unroll
    for (int j = 1; j < 16; j++)
#pragma unroll
        for (int c = 0; c < 4; c++) r[c] += __uint_as_float(d[j][c]);
    const int row = 32 * (gi >> 2) + 8 * (gi & 3) + 4 * (lane >> 5);
    const int n = tile * ct + 32 * wave + (lane & 31);
#pragma unroll
    for (int c = 0; c < 4; c++)
        if (row + c < M && n < N) y[(int64_t)(row + c) * N + n] = r[c];
}

// y[i] = part[0][i] + part[1][i] + ... in split order, times the row's x
// scale rs[i / N] when there is one
__global__ void splitk_reduce(const float *__restrict__ part, float *__restrict__ y, int64_t n,
                              int S, const float *__restrict__ rs, int64_t N) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float v = part[i];
    for (int s = 1; s < S; s++) v += part[(int64_t)s * n + i];
    y[i] = rs ? v * rs[i / N] : v;
}

hipError_t launch_xprep(const void *x, int x_dtype, int64_t m, int64_t k, _Float16 *xh,
                        _Float16 *xl, uint16_t *xs, float *rs, hipStream_t s, int parts, int rs_splits) {
    if (m == 0 || (!xh && !xl && !xs)) return hipSuccess;
    if (parts < 1 || parts > 3 || (parts == 3 && x_dtype != ARFQ_F32)) return hipErrorInvalidValue;
    if (k % 32 || k > INT32_MAX || (parts > 1 && (!xh || xl != xh + m * k))) return hipErrorInvalidValue;
    if (x_dtype != ARFQ_F32 && !xh && !xl && !rs) {  // the sums of an f16 x alone
        xsums_kernel<XSUM_WAVES><<<(unsigned)((m + XSUM_WAVES - 1) / XSUM_WAVES), 64 * XSUM_WAVES, 0, s>>>(
            (const _Float16 *)x, m, (int)k, xs);
        return hipGetLastError();
    }
    // segments: with rs, the skinny kernel's K ranges (whole 256-element
    // blocks) or the whole row; otherwise up to XPREP_THREADS * XPREP_NJ * 8
    // elements
    int S, unit;
    if (rs && rs_splits > 1) {
        if (k % 256 || rs_splits > k / 256) return hipErrorInvalidValue;
        S = rs_splits;
        unit = 256;
    } else if (rs) {
        S = 1;
        unit = 32;
    } else {
        unit = 32;
        constexpr int per = XPREP_THREADS * XPREP_NJ * 8 / 32;  // 32-element units per segment
        S = (int)((k / 32 + per - 1) / per);
    }
    if (m * S > INT32_MAX) return hipErrorInvalidValue;
    const unsigned grid = (unsigned)(m * S);
    if (x_dtype == ARFQ_F32)
        xprep_kernel<float><<<grid, XPREP_THREADS, 0, s>>>((const float *)x, m, (int)k, xh, xl, xs, rs,
                                                           parts - 1, S, unit);
    else
        xprep_kernel<_Float16><<<grid, XPREP_THREADS, 0, s>>>((const _Float16 *)x, m, (int)k, xh, xl,
                                                              xs, nullptr, parts - 1, S, unit);
    return hipGetLastError();
}

bool gemm_supports(const arfq_weight *w, int64_t m) {
    if (m < 1 || m > INT32_MAX / 2 || w->n > INT32_MAX / 2 || w->k > INT32_MAX / 2) return false;
    switch (w->qtype) {
    case ARFQ_Q4_K:
    case ARFQ_Q6_K:
    case ARFQ_Q5_K:
    case ARFQ_IQ4_XS: return true;
    case ARFQ_Q8_0: return w->k % GM_BK == 0;
    default: return false;
    }
}

// weight bytes per 256-element block of the direct-operand formats' largest
// stream (0: no such kernel); the buffer loads take 32-bit offsets
static int64_t bd_stream_bytes(int qtype) {
    switch (qtype) {
    case ARFQ_Q4_K:
    case ARFQ_IQ4_XS:
        return 128;
    case ARFQ_Q5_K:
        return 160;
    case ARFQ_Q6_K:
        return 192;
    case ARFQ_Q8_0:
        return 256;
    default:
        return 0;
    }
}

static size_t al256(size_t b) { return (b + 255) & ~(size_t)255; }

GemmPlan gemm_plan(const arfq_weight *w, int64_t m, int x_dtype, bool x16) {
    GemmPlan p;
    const int cus = w->ctx && w->ctx->cus > 0 ? w->ctx->cus : 256;
    const bool kind2 = w->qtype == ARFQ_Q4_K || w->qtype == ARFQ_Q5_K;  // min term: x sums
    p.skinny = m <= 64 && w->k % 256 == 0;
    p.bm = m > 64 ? 128 : 64;
    // prefill: the direct-operand kernel (one launch, no split-K) for every
    // format but IQ4_XS at f32 x (its weights are rounded to f16, so its x
    // keeps the hi + lo split of the tile loop below)
    const int64_t bdb = bd_stream_bytes(w->qtype);
    // (an f32 x enters it as hi + lo rows unless x16: twice the x bytes)
    const int64_t bdx = x_dtype == ARFQ_F32 && !x16 ? 2 : 1;
    p.bd = !p.skinny && m > 64 && bdb && w->k % 256 == 0 && !(w->qtype == ARFQ_IQ4_XS && x_dtype == ARFQ_F32) &&
           w->n * (w->k / 256) * bdb < ((int64_t)1 << 31) && bdx * m * w->k * 2 < ((int64_t)1 << 31);  // buffer loads
    // f32 x: scaled per row by a power of two into f16 range, then split into
    // f16 parts for the skinny kernel and the direct-operand prefill (hi + lo
    // rows: its tiles cover 64 rows at twice the MFMAs; one f16 part under x16),
    // or into f16 hi + lo for the tile loop (IQ4_XS prefill, whose weights are
    // rounded to f16: this way only one of the two operands is); the output
    // rows are multiplied back by the scale
    p.xsplit = !p.skinny && !p.bd && x_dtype == ARFQ_F32;
    p.convert = x_dtype == ARFQ_F32;
    // skinny kernel, f32 x: m <= 8 as three f16 parts (one 32-row x tile holds
    // three row blocks of 8: hi + mid + lo, exact for every x within 2^15 of its
    // row's max), m = 9..64 as hi + lo (~22 bits): the lo rows fill the other
    // half of the 32-row tile at m <= 16 (no extra MFMAs), a second tile at
    // m <= 32 and two more at m <= 64 (twice the MFMAs).  With x16
    // (ARFQ_OPT_GEMV_X16): one part, x rounded to f16.
    p.parts = p.skinny && x_dtype == ARFQ_F32 && !x16 ? (m <= 8 ? 3 : 2) : p.bd && bdx == 2 ? 2 : 1;
    // three parts (and their sub-block sums): formed by the skinny kernel as it
    // stages x (no preparation launch, no scratch for x)
    p.fx = p.skinny && p.parts == 3;
    if (p.fx) p.convert = false;
    // the exact Q4_K paths read x sub-block sums (min term; with fx the skinny
    // kernel forms them)
    p.sums = (p.skinny || p.bd) && kind2 && !p.fx;
    int64_t S;
    size_t bd_part = 0;
    if (p.bd) {
        S = 1;
        // the tiles past the last whole round of workgroups (one per CU) are
        // split into K ranges that fill that round; with XCD order the whole
        // tiles stay a multiple of the M tiles
        const int64_t rm = p.parts == 2 ? BD_BM / 2 : BD_BM;  // output rows per tile
        const int64_t mt = (m + rm - 1) / rm, nt = (w->n + BD_BN - 1) / BD_BN;
        const int64_t tiles = mt * nt, nb = w->k / 256;
        int64_t r = tiles % cus;
        if (mt % 8 == 0 && r % mt) r = std::min(tiles, (r / mt + 1) * mt);
        const int64_t chunks = r ? std::min<int64_t>({(int64_t)cus / r, nb, 16}) : 1;
        if (r && chunks >= 2) {
            p.bd_full = (int)(tiles - r);
            p.bd_chunks = (int)chunks;
            bd_part = (size_t)r * chunks * BD_BM * BD_BN * 4;
        } else {
            p.bd_full = (int)tiles;
        }
    } else if (p.skinny) {
        // split K (whole blocks, >= 2 per split) until ~2 workgroups per CU (~1 with
        // the four x tiles of f32 x at m > 32, whose LDS holds one workgroup per CU)
        const int64_t ct = sk_ct(p.parts == 2 && m > 32 ? 4 : 1), nt = (w->n + ct - 1) / ct, nb = w->k / 256;
        const int per_cu = p.parts == 2 && m > 32 ? 1 : 2;
        S = std::max<int64_t>(1, (per_cu * (int64_t)cus) / nt);
        S = std::min<int64_t>(S, std::max<int64_t>(1, nb / 2));
    } else {
        const int64_t mt = (m + p.bm - 1) / p.bm, nt = (w->n + GM_BN - 1) / GM_BN;
        const int unit = w->qtype == ARFQ_Q8_0 ? 1 : 4;
        const int64_t nu = w->k / GM_BK / unit;
        // split K until ~2 workgroups per CU are in flight, keeping >= 8 steps a split
        S = std::max<int64_t>(1, (2 * (int64_t)cus) / std::max<int64_t>(1, mt * nt));
        S = std::min<int64_t>(S, std::max<int64_t>(1, nu * unit / 8));
        S = std::min<int64_t>(S, nu);
    }
    p.splits = (int)std::min<int64_t>(S, 16);
    size_t o = 0;
    p.off_xh = o;
    o += p.convert ? al256((size_t)p.parts * m * w->k * 2) : 0;  // the lo (mid, lo) rows follow
    p.off_xl = o;
    o += p.xsplit ? al256((size_t)m * w->k * 2) : 0;
    p.off_xs = o;
    o += p.sums ? al256((size_t)p.parts * m * (w->k / 16) * 2) : 0;
    p.off_rs = o;  // skinny: one scale per row and split
    o += p.convert ? al256((size_t)(p.skinny ? p.splits : 1) * m * 4) : 0;
    p.off_part = o;
    if (p.skinny) {  // partials in register order: [split][column tile][wave][8-row group][lane] float4
        const int64_t ct = sk_ct(p.parts == 2 && m > 32 ? 4 : 1);
        o += p.splits > 1 ? al256((size_t)p.splits * ((w->n + ct - 1) / ct) * (ct / 32) *
                                  ((std::min<int64_t>(m, 64) + 7) / 8) * 1024)
                          : 0;
    }
    else
        o += p.splits > 1 ? al256((size_t)p.splits * m * w->n * 4) : al256(bd_part);
    p.scratch_bytes = o;
    return p;
}

template <class F, int TA, int PARTS, int GM = 0xFF, class XT = _Float16>
static hipError_t launch_sk_t(const F &fmt, const arfq_weight *w, int64_t m, const XT *x,
                              const uint16_t *xs, const float *rs, int rss, float *y, float *part,
                              int S, hipStream_t s) {
    if constexpr (F::KIND == 4 && TA == 1 && GM == 0xFF) {
        // at most 8 rows (8 hi + 8 lo with two parts, + 8 mid with three): the
        // per-sub-block scaling touches only the accumulator groups that hold them
        if (m <= 8)
            return launch_sk_t<F, 1, PARTS, PARTS == 3 ? 0x7 : PARTS == 2 ? 0x5 : 0x1, XT>(fmt, w, m, x, xs, rs, rss,
                                                                                          y, part, S, s);
    }
    constexpr int NT = sk_nt(TA), CT = NT / 2;
    constexpr size_t lds = sk_lds<F, TA, 1, NT, SK_XB(TA)>() + 32 * TA * 4;  // + the x rows' scales
    static std::atomic<uint64_t> lds_set{0};  // the attribute belongs to the kernel, per device
    if (hipError_t err = set_max_lds_once((const void *)gemm_sk<F, TA, XT, PARTS, GM>, lds, lds_set))
        return err;
    const int nt = (int)((w->n + CT - 1) / CT);
    const dim3 grid((unsigned)nt, (unsigned)S);
    gemm_sk<F, TA, XT, PARTS, GM><<<grid, NT, lds, s>>>(fmt, x, xs, rs, y, part, (int)m, (int)w->n, (int)w->k,
                                                           rss);
    if (hipError_t err = hipGetLastError()) return err;
    if (S > 1) {
        const int gt = (int)((m + 7) / 8);
        const int64_t threads = (int64_t)nt * (NT / 64) * gt * 64;
        sk_reduce_kernel<<<(unsigned)((threads + 255) / 256), 256, 0, s>>>(part, y, S, nt, NT / 64, gt, CT, (int)m,
                                                                           (int)w->n);
        return hipGetLastError();
    }
    return hipSuccess;
}

// S > 1 splits need S <= 16 and one zeroed counter per column tile.  x is
// f16 (an f32 x arrives prepared and scaled, rs[split * rss + row] its scale
// over each split's K range); with parts 2 (m <= 64) it is [2m, K]: the hi
// rows, then the lo rows; with parts 3 (m <= 8) the caller's f32 x [m, K] as
// xf, split into hi, mid and lo parts (and their sub-block sums) by the kernel
// itself.
template <class F>
static hipError_t launch_sk(const F &fmt, const arfq_weight *w, int64_t m, const _Float16 *x,
                            const uint16_t *xs, const float *rs, int rss, float *y, float *part,
                            int S, hipStream_t s, int parts, const float *xf = nullptr) {
    if (S > 1 && (S > 16 || !part)) return hipErrorInvalidValue;
    if (parts == 3) {
        if (m > 8) return hipErrorInvalidValue;
        if (!xf) return hipErrorInvalidValue;
        return launch_sk_t<F, 1, 3, 0xFF, float>(fmt, w, m, xf, nullptr, nullptr, 0, y, part, S, s);
    }
    if (parts == 2) {
        if (m > 64) return hipErrorInvalidValue;
        if (m <= 16) return launch_sk_t<F, 1, 2>(fmt, w, m, x, xs, rs, rss, y, part, S, s);
        if (m <= 32) return launch_sk_t<F, 2, 2>(fmt, w, m, x, xs, rs, rss, y, part, S, s);
        return launch_sk_t<F, 4, 2>(fmt, w, m, x, xs, rs, rss, y, part, S, s);
    }
    return m <= 32 ? launch_sk_t<F, 1, 1>(fmt, w, m, x, xs, rs, rss, y, part, S, s)
                   : launch_sk_t<F, 2, 1>(fmt, w, m, x, xs, rs, rss, y, part, S, s);
}

SkQ4K sk_q4k(const arfq_weight *w) {
    return {(const uint4 *)w->s0, (const uint4 *)w->s1, (int)(w->k / 256)};
}
SkQ6K sk_q6k(const arfq_weight *w) {
    return {(const uint2 *)w->s0, (const uint4 *)w->s1, (const uint16_t *)w->s2, (int)(w->k / 256)};
}
SkQ80 sk_q80(const arfq_weight *w) {
    return {(const uint4 *)w->s0, (const uint16_t *)w->s1, (int)(w->k / 32)};
}
SkQ5K sk_q5k(const arfq_weight *w) {
    return {(const uint4 *)w->s0, (const uint8_t *)w->s1, (int)(w->k / 256)};
}
SkIQ4XS sk_iq4xs(const arfq_weight *w) {
    return {(const uint2 *)w->s0, (const uint4 *)w->s1, (int)(w->k / 256)};
}

template <class F, int BM, bool XS>
static hipError_t launch_gemm_t(const F &fmt, const arfq_weight *w, int64_t m, const _Float16 *xh,
                                const _Float16 *xl, const uint16_t *xs, const float *rs, float *out,
                                int S, hipStream_t s) {
    constexpr size_t lds = gm_lds(BM, XS);
    static std::atomic<uint64_t> lds_set{0};  // the attribute belongs to the kernel, per device
    if (hipError_t err = set_max_lds_once((const void *)gemm_q<F, BM, XS>, lds, lds_set)) return err;
    const int mt = (int)((m + BM - 1) / BM), nt = (int)((w->n + GM_BN - 1) / GM_BN);
    const int xcd = (mt % 8 == 0) ? 1 : 0;
    const dim3 grid((unsigned)(mt * nt), (unsigned)S);
    gemm_q<F, BM, XS><<<grid, GM_THREADS, lds, s>>>(fmt, xh, xl, xs, rs, out, (int)m, (int)w->n,
                                                   (int)w->k, mt, xcd);
    return hipGetLastError();
}

template <class F>
static hipError_t launch_fmt(const F &fmt, const arfq_weight *w, int64_t m, const _Float16 *xh,
                             const _Float16 *xl, const uint16_t *xs, const float *rs, float *out,
                             const GemmPlan &p, hipStream_t s) {
    if (p.bm == 128)
        return p.xsplit ? launch_gemm_t<F, 128, true>(fmt, w, m, xh, xl, xs, rs, out, p.splits, s)
                        : launch_gemm_t<F, 128, false>(fmt, w, m, xh, xl, xs, rs, out, p.splits, s);
    return p.xsplit ? launch_gemm_t<F, 64, true>(fmt, w, m, xh, xl, xs, rs, out, p.splits, s)
                    : launch_gemm_t<F, 64, false>(fmt, w, m, xh, xl, xs, rs, out, p.splits, s);
}

FmtQ4K fmt_q4k(const arfq_weight *w) {
    return {(const uint4 *)w->s0, (const uint4 *)w->s1, (int)(w->k / 256)};
}
FmtQ6K fmt_q6k(const arfq_weight *w) {
    return {(const uint2 *)w->s0, (const uint2 *)w->s1, (const uint16_t *)w->s2, (int)(w->k / 256)};
}
FmtQ80 fmt_q80(const arfq_weight *w) {
    return {(const uint4 *)w->s0, (const uint16_t *)w->s1, (int)(w->k / 32)};
}

// Prefill: weights straight into the MFMA operands (arfq_gemm_bd.h)
template <class F, bool PX>
static hipError_t launch_bd_px(const F &f, const arfq_weight *w, int64_t m, const _Float16 *x,
                               const uint16_t *xs, const float *rs, float *y, float *part,
                               const GemmPlan &p, hipStream_t s) {
    constexpr int RM = PX ? BD_BM / 2 : BD_BM;
    const int mt = (int)((m + RM - 1) / RM), nt = (int)((w->n + BD_BN - 1) / BD_BN);
    const int tiles = mt * nt, nsplit = tiles - p.bd_full;
    const int xcd = (mt % 8 == 0 && p.bd_full % mt == 0) ? 1 : 0;
    if (nsplit && !part) return hipErrorInvalidValue;
    static std::atomic<uint64_t> lds_set{0};  // the attribute belongs to the kernel, per device
    if (hipError_t err = set_max_lds_once((const void *)gemm_bd<F, PX>, bd_lds<F>(), lds_set)) return err;
    const unsigned items = (unsigned)(p.bd_full + nsplit * p.bd_chunks);
    gemm_bd<F, PX><<<items, BD_THREADS, bd_lds<F>(), s>>>(f, x, xs, rs, y, part, (int)m, (int)w->n, (int)w->k, mt,
                                                       xcd, p.bd_full, p.bd_chunks);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess || !nsplit) return err;
    bd_reduce_kernel<<<dim3(RM * BD_BN / 1024, (unsigned)nsplit), 256, 0, s>>>(
        part, rs, y, (int)m, (int)w->n, mt, p.bd_full, p.bd_chunks, RM);
    return hipGetLastError();
}
// x as hi + lo rows (an f32 x, plan parts 2) or one f16 part
template <class F>
static hipError_t launch_bd_t(const F &f, const arfq_weight *w, int64_t m, const _Float16 *x,
                              const uint16_t *xs, const float *rs, float *y, float *part,
                              const GemmPlan &p, hipStream_t s) {
    return p.parts == 2 ? launch_bd_px<F, true>(f, w, m, x, xs, rs, y, part, p, s)
                        : launch_bd_px<F, false>(f, w, m, x, xs, rs, y, part, p, s);
}

static hipError_t launch_bd(const arfq_weight *w, int e, int64_t m, const _Float16 *x, const uint16_t *xs,
                            const float *rs, float *y, float *part, const GemmPlan &p, hipStream_t s) {
    const int64_t eb = (int64_t)e * w->n * (w->k / 256);
    switch (w->qtype) {
    case ARFQ_Q4_K:
        return launch_bd_t(BdQ4K{(const uint4 *)w->s0 + eb, (const uint4 *)w->s1 + eb * 8}, w, m, x, xs, rs, y,
                           part, p, s);
    case ARFQ_Q5_K:
        return launch_bd_t(BdQ5K{(const uint4 *)w->s0 + eb, (const uint8_t *)w->s1 + eb * 160}, w, m, x, xs, rs,
                           y, part, p, s);
    case ARFQ_IQ4_XS:
        return launch_bd_t(BdIQ4XS{(const uint2 *)w->s0 + eb, (const uint4 *)w->s1 + eb * 8}, w, m, x, xs, rs,
                           y, part, p, s);
    case ARFQ_Q6_K:  // scales beyond +-64 (flagged by the upload): sc * (q - 32) as hi + lo
        if (w->wide)
            return launch_bd_t(BdQ6KW{(const uint2 *)w->s0 + eb * 24, (const uint4 *)w->s1 + eb,
                                      (const uint16_t *)w->s2 + eb},
                               w, m, x, xs, rs, y, part, p, s);
        return launch_bd_t(BdQ6K{(const uint2 *)w->s0 + eb * 24, (const uint4 *)w->s1 + eb,
                                 (const uint16_t *)w->s2 + eb},
                           w, m, x, xs, rs, y, part, p, s);
    case ARFQ_Q8_0:
        return launch_bd_t(BdQ80{(const uint4 *)w->s0 + eb * 16, (const uint16_t *)w->s1 + eb * 8}, w, m, x, xs,
                           rs, y, part, p, s);
    default:
        return hipErrorInvalidValue;
    }
}

hipError_t launch_gemm(const arfq_weight *w, int e, int64_t m, const void *x, int x_dtype,
                       float *y, void *scratch,
                       const GemmPlan &p, hipStream_t s) {
    char *sc = (char *)scratch;
    if (p.scratch_bytes && !sc) return hipErrorInvalidValue;
    _Float16 *xh = p.convert ? (_Float16 *)(sc + p.off_xh) : (_Float16 *)x;
    _Float16 *xl = p.xsplit ? (_Float16 *)(sc + p.off_xl) : p.parts > 1 ? xh + m * w->k : nullptr;
    uint16_t *xs = p.sums ? (uint16_t *)(sc + p.off_xs) : nullptr;
    float *rs = p.convert ? (float *)(sc + p.off_rs) : nullptr;  // row scales of an f32 x
    if (p.convert || p.sums) {
        hipError_t err = launch_xprep(x, x_dtype, m, w->k, p.convert ? xh : nullptr, xl, xs, rs, s, p.parts,
                                      p.skinny ? p.splits : 1);
        if (err != hipSuccess) return err;
    }
    float *out = p.splits > 1 ? (float *)(sc + p.off_part) : y;
    hipError_t err;
    if (p.skinny) {
        // the split-K sum happens inside the kernel
        const _Float16 *xk = p.convert ? xh : (const _Float16 *)x;
        const float *xf = p.fx ? (const float *)x : nullptr;  // split by the kernel itself
        const int64_t eb = (int64_t)e * w->n * (w->k / 256);
        switch (w->qtype) {
        case ARFQ_Q4_K:
            return launch_sk(sk_q4k(w).shifted(eb), w, m, xk, xs, rs, (int)m, y, out,
                             p.splits, s, p.parts, xf);
        case ARFQ_Q6_K:  // scales within +-62 (the upload's flag): integer operands sc * (q - 32) / 2
            if (!w->over62)
                return launch_sk(SkQ6KI{sk_q6k(w)}.shifted(eb), w, m, xk, xs, rs, (int)m, y, out, p.splits, s,
                                 p.parts, xf);
            return launch_sk(sk_q6k(w).shifted(eb), w, m, xk, xs, rs, (int)m, y, out,
                             p.splits, s, p.parts, xf);
        case ARFQ_Q8_0:
            return launch_sk(sk_q80(w).shifted((int64_t)e * w->n * (w->k / 32)), w, m, xk, xs, rs,
                             (int)m, y, out, p.splits, s, p.parts, xf);
        case ARFQ_Q5_K:
            return launch_sk(sk_q5k(w).shifted(eb), w, m, xk, xs, rs, (int)m, y, out,
                             p.splits, s, p.parts, xf);
        case ARFQ_IQ4_XS:
            return launch_sk(sk_iq4xs(w).shifted(eb), w, m, xk, xs, rs, (int)m, y, out,
                             p.splits, s, p.parts, xf);
        default:
            return hipErrorInvalidValue;
        }
    } else if (p.bd) {
        return launch_bd(w, e, m, xh, xs, rs, y, (float *)(sc + p.off_part), p, s);
    } else switch (w->qtype) {
    case ARFQ_Q4_K: {
        const FmtQ4KR f{fmt_q4k(w).shifted((int64_t)e * w->n * (w->k / 256))};
        err = launch_fmt(f, w, m, xh, xl, xs, p.splits == 1 ? rs : nullptr, out, p, s);
        break;
    }
    case ARFQ_Q6_K: {
        const FmtQ6KR f{fmt_q6k(w).shifted((int64_t)e * w->n * (w->k / 256))};
        err = launch_fmt(f, w, m, xh, xl, xs, p.splits == 1 ? rs : nullptr, out, p, s);
        break;
    }
    case ARFQ_Q8_0: {
        const FmtQ80 f = fmt_q80(w).shifted((int64_t)e * w->n * (w->k / 32));
        err = launch_fmt(f, w, m, xh, xl, xs, p.splits == 1 ? rs : nullptr, out, p, s);
        break;
    }
    // Q5_K and IQ4_XS reach the tile loop only above 64 rows (128-row tiles)
    case ARFQ_Q5_K: {
        if (p.bm != 128) return hipErrorInvalidValue;
        const FmtQ5KR f = FmtQ5KR{(const uint4 *)w->s0, (const uint8_t *)w->s1, (int)(w->k / 256)}.shifted(
            (int64_t)e * w->n * (w->k / 256));
        const float *r1 = p.splits == 1 ? rs : nullptr;
        err = p.xsplit ? launch_gemm_t<FmtQ5KR, 128, true>(f, w, m, xh, xl, xs, r1, out, p.splits, s)
                       : launch_gemm_t<FmtQ5KR, 128, false>(f, w, m, xh, xl, xs, r1, out, p.splits, s);
        break;
    }
    case ARFQ_IQ4_XS: {
        if (p.bm != 128) return hipErrorInvalidValue;
        const FmtIQ4XSR f = FmtIQ4XSR{(const uint2 *)w->s0, (const uint4 *)w->s1, (int)(w->k / 256)}.shifted(
            (int64_t)e * w->n * (w->k / 256));
        const float *r1 = p.splits == 1 ? rs : nullptr;
        err = p.xsplit ? launch_gemm_t<FmtIQ4XSR, 128, true>(f, w, m, xh, xl, xs, r1, out, p.splits, s)
                       : launch_gemm_t<FmtIQ4XSR, 128, false>(f, w, m, xh, xl, xs, r1, out, p.splits, s);
        break;
    }
    default:
        return hipErrorInvalidValue;
    }
    if (err != hipSuccess || p.splits == 1) return err;
    const int64_t n = m * w->n;
    splitk_reduce<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(out, y, n, p.splits, rs, w->n);
    return hipGetLastError();
}

}  // namespace arfq
