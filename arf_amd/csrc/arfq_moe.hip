// arfq_moe.hip -- the expert-grouped MoE block on device:
//   route   -> ids[t, j], weights[t, j]       (top-k of the softmax per token)
//   group   -> (token, slot) pairs grouped by expert (row offsets per expert)
//              plus a list of up to MOE_BM-row tiles per expert
//   gate|up -> h[pair] = silu(x_t . gate_e^T) * (x_t . up_e^T)   (f32, grouped order)
//   hprep   -> h16 = h / rs (rs a power of two per row), sub-block sums of h16
//   down    -> o[t*top_k + j] = rs * (h16[pair] . down_e^T)     (f32)
//   combine -> y[t] = sum_j w[t, j] * o[t*top_k + j] in slot order
// The grouped GEMMs run the skinny weight-streaming MFMA loop
// (arfq_skinny.h) with exact integer weight operands.
//
// Reference behaviour: moe_route_msl.metal:18-98 / moe_batch_msl.metal:371-563
// (route, CSR by expert, swiglu, slot-ordered reduce), moe_mm_id_q4ks.metal:103-700
// (grouped mm_id over an expert tile list); oracle MoeMlp::forward
// (crates/arf-core/src/model/moe.rs:53-86), top_k_softmax (moe.rs:89-121),
// Mlp::forward (crates/arf-core/src/model/mlp.rs:20-24), silu
// (crates/arf-ml/src/lib.rs:160-162).
#include "arfq_gemm_tile.h"
#include "arfq_internal.h"
#include "arfq_skinny.h"

namespace arfq {

// ---- route -------------------------------------------------------------------
// One wave per token; lane l holds logits l, l+64, ... (E <= 64 * MOE_ROUTE_PL).
// softmax exactly as the reference: max, exp(l - max), sum in index order,
// divide; then top_k rounds of a wave argmax on (prob desc, index asc), which is
// the reference's stable sort + truncate; renormalise by the selected sum
// (summed in selection order) when norm != 0.
constexpr int MOE_ROUTE_PL = 16;  // up to 1024 experts

// Wave-wide max / min with every lane getting the result: a DPP butterfly
// inside each 16-lane row (xor 1, xor 2, half-row mirror, row mirror), then
// v_permlane16_swap and v_permlane32_swap across rows -- VALU only, no LDS
// round trip per step.
template <int CTRL>
__device__ __forceinline__ int route_dpp(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xf, 0xf, true);
}
template <class Op>
__device__ __forceinline__ int route_wave_reduce(int v, Op op) {
    v = op(v, route_dpp<0xB1>(v));   // quad_perm [1,0,3,2]
    v = op(v, route_dpp<0x4E>(v));   // quad_perm [2,3,0,1]
    v = op(v, route_dpp<0x141>(v));  // row_half_mirror
    v = op(v, route_dpp<0x140>(v));  // row_mirror
    const auto p16 = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
    v = op((int)p16[0], (int)p16[1]);
    const auto p32 = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
    return op((int)p32[0], (int)p32[1]);
}
__device__ __forceinline__ float route_wave_max(float v) {
    return __int_as_float(route_wave_reduce(__float_as_int(v), [](int a, int b) {
        return __float_as_int(fmaxf(__int_as_float(a), __int_as_float(b)));
    }));
}
__device__ __forceinline__ int route_wave_min(int v) {
    return route_wave_reduce(v, [](int a, int b) { return min(a, b); });
}

// The workgroups past the routing ones (blockIdx.x >= rblocks) form the x
// sub-block sums of an f16 x [tokens, K] for the grouped GEMMs instead (no
// dependence between the two, so one launch serves both).
template <int PL>
__global__ __launch_bounds__(256) void moe_route_kernel(const float *__restrict__ logits,
                                                        int64_t tokens, int E, int top_k,
                                                        int norm, int32_t *__restrict__ ids,
                                                        float *__restrict__ wts, int rblocks,
                                                        const _Float16 *__restrict__ x, int K,
                                                        uint16_t *__restrict__ xs) {
    const int lane = threadIdx.x & 63;
    if ((int)blockIdx.x >= rblocks) {  // uniform over the workgroup
        const int64_t row = (int64_t)(blockIdx.x - rblocks) * 4 + (threadIdx.x >> 6);
        if (row < tokens) xsums_row(x, K, xs, row);
        return;
    }
    const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= tokens) return;  // whole waves: every lane of a running wave is active
    const float *lg = logits + t * E;
    float v[PL];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < PL; j++) {
        const int i = j * 64 + lane;
        v[j] = i < E ? lg[i] : -INFINITY;
        mx = fmaxf(mx, v[j]);
    }
    mx = route_wave_max(mx);
#pragma unroll
    for (int j = 0; j < PL; j++) v[j] = (j * 64 + lane < E) ? expf(v[j] - mx) : 0.f;
    // sum in index order (the reference's sequential iterator sum); the slots
    // past E hold exact zeros, so summing whole rounds of 64 changes nothing
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < PL; j++) {
        if (j * 64 >= E) break;
        if (PL <= 4) {
#pragma unroll
            for (int l = 0; l < 64; l++) s += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[j]), l));
        } else {
            const int cnt = min(64, E - j * 64);
            for (int l = 0; l < cnt; l++) s += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[j]), l));
        }
    }
#pragma unroll
    for (int j = 0; j < PL; j++) v[j] = (j * 64 + lane < E) ? v[j] / s : -INFINITY;

    // top_k rounds: the wave's largest untaken probability, then the lowest
    // index holding it (the stable sort's order for ties)
    uint32_t taken = 0;
    float myw = 0.f;
    int myid = 0;
    float wsum = 0.f;
    for (int r = 0; r < top_k; r++) {
        float bp = -INFINITY;
        int bi = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < PL; j++) {
            const int i = j * 64 + lane;
            if (i < E && !((taken >> j) & 1u) && (v[j] > bp || bi == 0x7fffffff)) {
                bp = v[j];
                bi = i;
            }
        }
        const float wp = route_wave_max(bp);
        const int wi = route_wave_min(bi != 0x7fffffff && bp == wp ? bi : 0x7fffffff);
        if ((wi & 63) == lane) taken |= 1u << (wi >> 6);
        if (lane == r) {
            myw = wp;
            myid = wi;
        }
        wsum += wp;
    }
    if (lane < top_k) {
        ids[t * top_k + lane] = myid;
        wts[t * top_k + lane] = (norm && wsum > 0.f) ? myw / wsum : myw;
    }
}

// ---- group ---------------------------------------------------------------------
// One 1024-thread workgroup: count the (token, slot) pairs per expert, scan the
// counts into row offsets and a tile list (ceil(count / bm) tiles per expert),
// then place each pair at offset[e] + an LDS atomic cursor.  The order of the
// pairs inside an expert's rows is whatever the atomics give: every row is
// computed on its own and the combine sums each token's slots in slot order,
// so the output does not depend on it.  Pairs whose expert id is out of range
// are dropped.
constexpr int MOE_MAX_EXPERTS = 512;

__device__ __forceinline__ int block_excl_scan_1024(int v, int *tmp, int &total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int inc = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(inc, o);
        if (lane >= o) inc += u;
    }
    if (lane == 63) tmp[w] = inc;
    __syncthreads();
    int wbase = 0, tot = 0;
    for (int i = 0; i < 16; i++) {
        const int x = tmp[i];
        if (i < w) wbase += x;
        tot += x;
    }
    __syncthreads();
    total = tot;
    return wbase + inc - v;
}

__global__ __launch_bounds__(1024) void moe_group_kernel(const int32_t *__restrict__ ids,
                                                         int64_t P, int E, int bm,
                                                         int32_t *__restrict__ off,
                                                         int32_t *__restrict__ sorted,
                                                         int2 *__restrict__ tiles,
                                                         int32_t *__restrict__ ntiles) {
    __shared__ int cnt[MOE_MAX_EXPERTS];  // counts, then the placement cursors
    __shared__ int tmp[32];
    const int tid = threadIdx.x;
    // the first GR_KEEP ids of each thread stay in registers for the placement
    constexpr int GR_KEEP = 8;
    int keep[GR_KEEP];
#pragma unroll
    for (int i = 0; i < GR_KEEP; i++) {
        const int64_t p = tid + 1024 * (int64_t)i;
        keep[i] = p < P ? ids[p] : -1;
    }
    for (int e = tid; e < E; e += 1024) cnt[e] = 0;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < GR_KEEP; i++)
        if (keep[i] >= 0 && keep[i] < E) atomicAdd(&cnt[keep[i]], 1);
    for (int64_t p = tid + 1024 * (int64_t)GR_KEEP; p < P; p += 1024) {
        const int e = ids[p];
        if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    const int c = tid < E ? cnt[tid] : 0;
    const int tc = (c + bm - 1) / bm;
    int rows_total, tiles_total;
    const int ex_c = block_excl_scan_1024(c, tmp, rows_total);
    const int ex_t = block_excl_scan_1024(tc, tmp + 16, tiles_total);
    if (tid < E) {
        off[tid] = ex_c;
        for (int i = 0; i < tc; i++) tiles[ex_t + i] = make_int2(tid, ex_c + i * bm);
        cnt[tid] = ex_c;
    }
    if (tid == 0) {
        off[E] = rows_total;
        *ntiles = tiles_total;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < GR_KEEP; i++)
        if (keep[i] >= 0 && keep[i] < E) sorted[atomicAdd(&cnt[keep[i]], 1)] = tid + 1024 * i;
    for (int64_t p = tid + 1024 * (int64_t)GR_KEEP; p < P; p += 1024) {
        const int e = ids[p];
        if (e >= 0 && e < E) sorted[atomicAdd(&cnt[e], 1)] = (int32_t)p;
    }
}

// ---- grouped GEMMs ----------------------------------------------------------------
// Both run the skinny weight-streaming loop (arfq_skinny.h) over one expert
// tile of up to MOE_BM = 64 (token, slot) rows.
constexpr int MOE_BM = 64;

// gate|up: a work item is one tile x 128 columns of inter, taken by a
// workgroup of 8 waves: wave w < 4 streams gate rows n0 + 32 w, wave w + 4 the
// same rows of up (one weight per wave keeps two waves per SIMD).  After the
// loop the up waves hand their accumulators to the gate waves through LDS, and
// the gate waves write h = silu(g) * u in f32 (its range can exceed f16's;
// moe_hprep scales it).  The grid holds as many workgroups as fit on the
// device at once and each walks the items with a stride of the grid, so the
// item count (known only on the device) never leaves a part-filled last round
// of workgroups.
constexpr int MOE_GU_THREADS = 512;
// Two x buffers (one barrier per block instead of two): C5 183.2 -> 182.4 us;
// the workgroup holds a CU by its registers, so the LDS costs no occupancy.
constexpr int MOE_GU_XB = 2;
// LDS of gate|up: the loop's, then the tile rows' x scales [MOE_BM] floats.
template <class F>
__host__ __device__ constexpr size_t gu_scale_off() {
    return sk_lds<F, 2, 1, MOE_GU_THREADS, MOE_GU_XB>();
}
template <class F>
__global__ __launch_bounds__(MOE_GU_THREADS) void moe_gateup_kernel(
    F gate, F up, int64_t expert_blocks, const _Float16 *__restrict__ x,
    const uint16_t *__restrict__ xs, const float *__restrict__ xrs, int K, int inter, int top_k,
    const int32_t *__restrict__ off, const int32_t *__restrict__ sorted, const int2 *__restrict__ tiles,
    const int32_t *__restrict__ ntiles, float *__restrict__ h) {
    extern __shared__ __attribute__((aligned(16))) _Float16 lds[];
    const int ncol = (inter + 127) / 128;
    const int items = *ntiles * ncol;
    // workgroup b runs on XCD b % 8: XCD x walks items [x per, (x + 1) per), so
    // the column items of a tile share its x rows in one L2 (C5 142.2 -> 140.8
    // us with the same order in down; a stride of the grid over all items
    // put a tile's six column items on six XCDs)
    const int G = gridDim.x, nx = G % 8 == 0 ? 8 : 1, GX = G / nx;
    const int per = (items + nx - 1) / nx, xbase = ((int)blockIdx.x % nx) * per;
    const int xend = min(items, xbase + per);
    for (int it = xbase + (int)blockIdx.x / nx; it < xend; it += GX) {  // uniform over the workgroup
        const int tid = sk_tid(), lane = tid & 63;
        const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform
        const int wq = wave & 3;
        const bool is_up = wave >= 4;
        const int ti = it / ncol;
        const int2 tile = tiles[ti];
        const int e = tile.x, row0 = tile.y;
        const int rows = min(MOE_BM, off[e + 1] - row0);
        const int n0 = (it - ti * ncol) * 128 + 32 * wq;
        const SkRows<2, MOE_GU_THREADS> xr =
            sk_rows<2, MOE_GU_THREADS>(rows, K, [&](int r) { return sorted[row0 + r] / top_k; });
        const F fm[1] = {(is_up ? up : gate).shifted((int64_t)e * expert_blocks)};
        const int64_t wrow0[1] = {n0};
        // the tile rows' x scales, by up wave 0 into LDS past the loop's own:
        // one division and one dependent load pair per row, not per output,
        // and before the loop rather than after it
        float *exs = reinterpret_cast<float *>(reinterpret_cast<char *>(lds) + gu_scale_off<F>());
        if (xrs && wave == 4 && lane < rows) exs[lane] = xrs[sorted[row0 + lane] / top_k];
        floatx16 acc[1][2];
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int i = 0; i < 16; i++) acc[0][t][i] = 0.f;
        skinny_run<F, 2, 1, MOE_GU_THREADS, _Float16, true, 0xFF, false, false, MOE_GU_XB, 0, true>(
            fm, wrow0, inter, xr, x, xs, 0, K / 256, acc, lds, rows);
        // the loop ends with a barrier after its last LDS use: hand up to gate
        float *ex = reinterpret_cast<float *>(lds);  // [4 waves][2 tiles][16][64 lanes]
        if (is_up) {
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int i = 0; i < 16; i++) ex[((wq * 2 + t) * 16 + i) * 64 + lane] = acc[0][t][i];
        }
        __syncthreads();
        if (!is_up) {
            const int n = n0 + (lane & 31);
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const int r = sk_out_row(t, i);
                    if (r < rows && n < inter) {
                        float g = acc[0][t][i], u = ex[((wq * 2 + t) * 16 + i) * 64 + lane];
                        if (xrs) {  // the token row was stored divided by xrs (exact)
                            const float sc = reinterpret_cast<const float4 *>(exs)[r >> 2][i & 3];
                            g *= sc;
                            u *= sc;
                        }
                        // silu from the hardware exp2 and reciprocal (a few
                        // ulp): h goes to f16 (2^-11 relative) before down
                        // multiplies it; expf and an IEEE divide cost ~22 VALU
                        // per output here, the up waves idle meanwhile
                        const float sg =
                            g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.44269504f));
                        h[(int64_t)(row0 + r) * inter + n] = sg * u;
                    }
                }
        }
        __syncthreads();  // the hand-off area is the next item's x staging
    }
}

// h rows (f32) -> f16 copies scaled by a power of two per row, so that the
// largest |h| of the row is below 2^15: h16 = h / rs (exact scaling), the
// down GEMM multiplies its output row by rs.  For Q4_K down weights also the
// sub-block sums of h16 (bf16 hi + lo, the xs layout).  One wave per row.
// One wave per row; lane l handles elements 8 (l % 4) .. + 7 of sub-block
// (l / 4) + 16 q in pass q, so each quad owns a 32-element sub-block: the
// row's values stay in registers between the max and the conversion (up to
// HP_PASSES passes, inter <= 2048; longer rows are read twice), loads and
// stores are 16-byte and coalesced, and the sub-block sums are quad DPP sums.
constexpr int HP_PASSES = 4;
__global__ __launch_bounds__(256) void moe_hprep_kernel(const float *__restrict__ h, int64_t P,
                                                        int inter, _Float16 *__restrict__ h16,
                                                        uint16_t *__restrict__ hs,
                                                        float *__restrict__ rs) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= P) return;  // whole waves: every lane of a running wave is active
    const float *src = h + row * inter;
    const int nsub = inter / 32;
    const int npass = (nsub + 15) / 16;
    const int qd = lane & 3;
    auto load8 = [&](int q, float (&v)[8]) {
        const int sub = (lane >> 2) + 16 * q;
        if (sub < nsub) {
            const float4 *p4 = reinterpret_cast<const float4 *>(src + sub * 32 + 8 * qd);
            const float4 a = p4[0], b = p4[1];
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = 0.f;
        }
    };
    float val[HP_PASSES][8];
    float amax = 0.f;
    for (int q = 0; q < npass; q++) {
        float v[8];
        load8(q, v);
#pragma unroll
        for (int i = 0; i < 8; i++) amax = fmaxf(amax, fabsf(v[i]));
#pragma unroll
        for (int qq = 0; qq < HP_PASSES; qq++)
            if (qq == q)
#pragma unroll
                for (int i = 0; i < 8; i++) val[qq][i] = v[i];
    }
    amax = route_wave_max(amax);
    const int ex = amax > 0.f ? __builtin_amdgcn_frexp_expf(amax) : 0;  // amax < 2^ex
    const int sh = ex > 15 ? ex - 15 : 0;
    const float inv = ldexpf(1.f, -sh);
    if (lane == 0) rs[row] = ldexpf(1.f, sh);
    for (int q = 0; q < npass; q++) {
        float v[8];
        if (q < HP_PASSES) {
#pragma unroll
            for (int qq = 0; qq < HP_PASSES; qq++)
                if (qq == q)
#pragma unroll
                    for (int i = 0; i < 8; i++) v[i] = val[qq][i];
        } else {
            load8(q, v);
        }
        const int sub = (lane >> 2) + 16 * q;
        half8 hv;
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            hv[i] = (_Float16)(v[i] * inv);
            sum += (float)hv[i];
        }
        // the sub-block's sum over its quad, in quad order
        sum += __int_as_float(route_dpp<0xB1>(__float_as_int(sum)));
        sum += __int_as_float(route_dpp<0x4E>(__float_as_int(sum)));
        if (sub < nsub) {
            reinterpret_cast<half8 *>(h16 + row * inter + sub * 32)[qd] = hv;
            if (hs && qd == 0) {
                const uint32_t hi = bf16_bits(sum);
                const uint32_t lo = bf16_bits(sum - bf16_to_f32(hi));
                uint16_t *d = hs + row * (inter / 16) + (sub >> 3) * 16 + (sub & 7);
                d[0] = (uint16_t)hi;
                d[8] = (uint16_t)lo;
            }
        }
    }
}

// down: workgroup = one tile x 128 columns of hidden, two workgroups per CU
// (at most 256 registers per lane); rows are stored to o[pair index], scaled
// back by the row's h scale, so the combine can read each token's slots in
// order.  A plain grid here: its items differ in cost (one or two x tiles) and
// the dispatcher's dynamic placement beat a grid-stride loop (64 vs 76 us at
// 128 experts, top-8, 512 tokens).
template <class F>
__global__ __launch_bounds__(SK_THREADS, 2) void moe_down_kernel(
    F down, int64_t expert_blocks, const _Float16 *__restrict__ h, const uint16_t *__restrict__ hs,
    const float *__restrict__ rs, int K, int hidden, const int32_t *__restrict__ off,
    const int32_t *__restrict__ sorted, const int2 *__restrict__ tiles,
    const int32_t *__restrict__ ntiles, float *__restrict__ o) {
    extern __shared__ __attribute__((aligned(16))) _Float16 lds[];
    if ((int)blockIdx.x >= *ntiles) return;  // uniform over the workgroup
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int2 tile = tiles[blockIdx.x];
    const int e = tile.x, row0 = tile.y;
    const int rows = min(MOE_BM, off[e + 1] - row0);
    const int n0 = blockIdx.y * 128 + 32 * wave;
    const SkRows<2> xr = sk_rows<2>(rows, K, [&](int r) { return row0 + r; });
    // the output row and h scale of tile row `tid`, loaded before the loop and
    // handed over through LDS after it (not two loads per output at the end)
    int orow = 0;
    float ors = 0.f;
    if (tid < rows) {
        orow = sorted[row0 + tid];
        ors = rs[row0 + tid];
    }
    const F fm[1] = {down.shifted((int64_t)e * expert_blocks)};
    const int64_t wrow0[1] = {n0};
    floatx16 acc[1][2];
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int i = 0; i < 16; i++) acc[0][t][i] = 0.f;
    // (Q6_K: the second loop copy would not fit the registers)
    skinny_run<F, 2, 1, SK_THREADS, _Float16, F::KIND != 4, 0xFF, false, false, 1, 0, true>(fm, wrow0, hidden, xr, h, hs, 0, K / 256,
                                                           acc, lds, rows);
    // the loop ends with a barrier after its last LDS use
    int *lrow = reinterpret_cast<int *>(lds);                // [64]
    float *lrs = reinterpret_cast<float *>(lds) + MOE_BM;    // [64]
    if (tid < MOE_BM) {
        lrow[tid] = orow;
        lrs[tid] = ors;
    }
    __syncthreads();
    const int n = n0 + (lane & 31);
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int r = sk_out_row(t, i);
            if (r < rows && n < hidden) o[(int64_t)lrow[r] * hidden + n] = acc[0][t][i] * lrs[r];
        }
}

// down, x-stationary, where a tile's h16 rows over all of K fit in LDS beside
// eight weight slabs (C5: K = 768, 142 KB): workgroup = one tile x DXS_COLS
// columns of hidden, 8 waves.  The tile's rows and their sub-block sums are
// staged once; then each wave streams its own weight rows -- passes of
// 8 x 32 rows, each over every K block, the next block's weights in flight --
// with no barrier in the loop (the slabs are wave-private and x does not
// change).  Per pass the wave stores its 32 columns of the tile's rows to
// o[pair index], times the row's h scale.  Against the tile x 128-column
// workgroups above: one x staging and one pipeline start per 1024 columns
// instead of per 128, and no per-block barrier.
constexpr int DXS_THREADS = 512;
constexpr size_t MOE_DXS_LDS_MAX = 160 * 1024;
constexpr int DXS_COLS = 1024;  // columns per workgroup: passes of 8 waves x 32 rows
template <class F>
__host__ __device__ constexpr size_t dxs_lds(int K) {
    return (size_t)MOE_BM * (K + 8) * 2                          // h16 rows [64][K + 8]
           + (size_t)MOE_BM * (K / 256) * 32                     // their sums [64][K / 256][16]
           + (size_t)MOE_BM * 8                                  // pair index, h scale per row
           + (size_t)(DXS_THREADS / 64) * 32 * (F::RB + 16);     // one weight slab per wave
}
template <class F>
__global__ __launch_bounds__(DXS_THREADS, 1) void moe_down_xs_kernel(
    F down, int64_t expert_blocks, const _Float16 *__restrict__ h, const uint16_t *__restrict__ hs,
    const float *__restrict__ rs, int K, int hidden, const int32_t *__restrict__ off,
    const int32_t *__restrict__ sorted, const int2 *__restrict__ tiles, const int32_t *__restrict__ ntiles,
    float *__restrict__ o) {
    constexpr int KIND = F::KIND;
    constexpr int RL = F::RB / 16, NI = 32 * F::RB / 1024, SL = F::RB + 16;
    extern __shared__ __attribute__((aligned(16))) _Float16 lds[];
    const int ncb = (hidden + DXS_COLS - 1) / DXS_COLS;
    // workgroup L runs on XCD L % 8: XCD x takes items [x per, (x + 1) per) of
    // the real ones, so the column items of a tile share its rows in one L2
    const int total = *ntiles * ncb, L = (int)blockIdx.x;
    if (L >= total) return;  // uniform over the workgroup
    const int per = total >> 3;
    const int q = L < 8 * per ? (L & 7) * per + (L >> 3) : L;
    const int ti = q / ncb;
    const int tid = sk_tid(), lane = tid & 63, wave = tid >> 6, lr = lane & 31;
    const int2 tile = tiles[ti];
    const int e = tile.x, row0 = tile.y;
    const int rows = min(MOE_BM, off[e + 1] - row0);
    const int c0 = (q - ti * ncb) * DXS_COLS;
    const int nb = K / 256, xld = K + 8;
    _Float16 *xs_l = lds;                                                        // [64][xld]
    uint16_t *ss_l = reinterpret_cast<uint16_t *>(lds + MOE_BM * xld);           // [64][nb][16]
    int *lrow = reinterpret_cast<int *>(ss_l + MOE_BM * nb * 16);               // [64]
    float *lrs = reinterpret_cast<float *>(lrow + MOE_BM);                       // [64]
    uint8_t *slab = reinterpret_cast<uint8_t *>(lrs + MOE_BM) + (size_t)wave * 32 * SL;
    // the tile's rows (rows past the tile repeat its last: their products land
    // in rows never stored), 16 bytes a thread at a time
    const int kc8 = K / 8;
    for (int c = tid; c < MOE_BM * kc8; c += DXS_THREADS) {
        const int r = c / kc8, kc = c - r * kc8;
        *reinterpret_cast<u32x4 *>(xs_l + r * xld + 8 * kc) =
            *reinterpret_cast<const u32x4 *>(h + (int64_t)(row0 + min(r, rows - 1)) * K + 8 * kc);
    }
    if constexpr (KIND == 2) {
        const int sc8 = nb * 2;  // 16-byte pieces of a row's sums
        for (int c = tid; c < MOE_BM * sc8; c += DXS_THREADS) {
            const int r = c / sc8, j = c - r * sc8;
            *reinterpret_cast<u32x4 *>(ss_l + r * nb * 16 + 8 * j) =
                *reinterpret_cast<const u32x4 *>(hs + (int64_t)(row0 + min(r, rows - 1)) * (K / 16) + 8 * j);
        }
    }
    if (tid < MOE_BM) {
        lrow[tid] = tid < rows ? sorted[row0 + tid] : 0;
        lrs[tid] = tid < rows ? rs[row0 + tid] : 0.f;
    }
    __syncthreads();

    const F fm = down.shifted((int64_t)e * expert_blocks);
    const int npass = min(DXS_COLS, hidden - c0 + 255) / 256;  // passes with a column < hidden
    const int S = npass * nb;  // steps (pass, block)
    auto wrow_of = [&](int st) { return c0 + 256 * (st / nb) + 32 * wave; };
    // two steps of weights in flight: register set j holds the steps st with
    // st % 2 == j, wbs[j] their scales.  The weight loads are non-temporal
    // (each byte is used once): the L2 keeps the staged rows' sources and
    // the gate|up outputs instead
    u32x4 rv[2][NI];
    typename F::Blk wbs[2][1], wbn[1];
    auto wload = [&](u32x4 (&r)[NI], int st) {
        const int wr = wrow_of(st), b = st % nb;
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int c = 64 * i + lane;
            const int64_t row = min(wr + c / RL, hidden - 1);
            r[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(fm.raw(row, b) + 16 * (c % RL)));
        }
    };
    auto wstore = [&](const u32x4 (&r)[NI]) {
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int c = 64 * i + lane;
            *reinterpret_cast<u32x4 *>(slab + (c / RL) * SL + 16 * (c % RL)) = r[i];
        }
    };
    auto loop = [&](auto tu) {
        constexpr int TU = decltype(tu)::value;
        floatx16 acc[1][2], cb[1][2], cq[1][KIND == 3 ? 2 : 1];
        auto zero = [&]() {
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int i = 0; i < 16; i++) acc[0][t][i] = 0.f;
        };
        zero();
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int sj = min(j, S - 1);
            wbs[j][0] = fm.load_blk(min(wrow_of(sj) + lr, hidden - 1), sj % nb);
            wload(rv[j], sj);
        }
        auto step = [&](u32x4 (&r)[NI], typename F::Blk (&wb)[1], int st) {
            const int b = st % nb, sn = min(st + 2, S - 1);  // past the end: a re-read of the last step
            wstore(r);
            wbn[0] = fm.load_blk(min(wrow_of(sn) + lr, hidden - 1), sn % nb);
            __builtin_amdgcn_sched_barrier(0);
            wload(r, sn);
            __builtin_amdgcn_sched_barrier(0);
            sk_block<F, 2, TU, 1, 0xFF, false, false>(
                slab, wb, [&](int t) { return xs_l + (32 * t + lr) * xld + 256 * b; },
                [&](int t) { return ss_l + ((32 * t + lr) * nb + b) * 16; }, lr, lane >> 5, acc, cb, cq);
            wb[0] = wbn[0];
            if (b == nb - 1) {
                // the pass's 32 columns of every tile row
                const int n = wrow_of(st) + lr;
#pragma unroll
                for (int t = 0; t < TU; t++)
#pragma unroll
                    for (int i = 0; i < 16; i++) {
                        const int r = sk_out_row(t, i);
                        if (r < rows && n < hidden) o[(int64_t)lrow[r] * hidden + n] = acc[0][t][i] * lrs[r];
                    }
                zero();
            }
        };
        for (int st = 0; st < S; st += 2) {
            step(rv[0], wbs[0], st);
            if (st + 1 < S) step(rv[1], wbs[1], st + 1);
        }
    };
    if (rows <= 32)
        loop(std::integral_constant<int, 1>{});
    else
        loop(std::integral_constant<int, 2>{});
}

// ---- combine -------------------------------------------------------------------
// y[t, c] = ((0 + w0*o0) + w1*o1) + ... over the token's slots in order, each
// product and sum rounded separately (the reference's out[t] += w_j * y_j).
// Grid: (hidden / 4 / 256 column blocks, tokens); 4 columns per thread.
__global__ void moe_combine_kernel(const float *__restrict__ o, const int32_t *__restrict__ ids,
                                   const float *__restrict__ wts, int top_k, int E, int hidden,
                                   float *__restrict__ y, int accumulate) {
#pragma clang fp contract(off)
    const int64_t t = blockIdx.y;
    const int c4 = blockIdx.x * blockDim.x + threadIdx.x;
    if (4 * c4 >= hidden) return;
    // accumulate: y already holds the shared experts' sum, added first as in
    // MoeMlp::forward (moe.rs:62-67: out = 0 + shared, then += w_j * y_j)
    float4 acc = accumulate ? reinterpret_cast<const float4 *>(y + t * hidden)[c4] : make_float4(0.f, 0.f, 0.f, 0.f);
    for (int j = 0; j < top_k; j++) {
        const int e = ids[t * top_k + j];
        if (e < 0 || e >= E) continue;  // dropped pair: contributes nothing
        const float w = wts[t * top_k + j];
        const float4 v = reinterpret_cast<const float4 *>(o + (t * top_k + j) * hidden)[c4];
        acc.x = acc.x + w * v.x;
        acc.y = acc.y + w * v.y;
        acc.z = acc.z + w * v.z;
        acc.w = acc.w + w * v.w;
    }
    reinterpret_cast<float4 *>(y + t * hidden)[c4] = acc;
}

// ---- gated activation ------------------------------------------------------
// h = act(g) * u: SwiGLU or GeGLU (glu<ACT>, arfq_common.h), the same
// expressions as the fused down GEMVs and the gate|up kernel.
template <int ACT>
__global__ void glu_kernel(const float *__restrict__ g, const float *__restrict__ u, float *__restrict__ h,
                           int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) h[i] = glu<ACT>(g[i], u[i]);
}

hipError_t launch_glu(const float *g, const float *u, float *h, int64_t n, int act, hipStream_t s) {
    if (n == 0) return hipSuccess;
    const unsigned grid = (unsigned)((n + 255) / 256);
    if (act == ACT_GELU_TANH)
        glu_kernel<ACT_GELU_TANH><<<grid, 256, 0, s>>>(g, u, h, n);
    else if (act == ACT_SILU)
        glu_kernel<ACT_SILU><<<grid, 256, 0, s>>>(g, u, h, n);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

// ---- launchers -----------------------------------------------------------------

hipError_t launch_moe_route(const float *logits, int64_t tokens, int E, int top_k, int norm,
                            int32_t *ids, float *wts, hipStream_t s, const _Float16 *x, int64_t k,
                            uint16_t *xs) {
    if (tokens == 0) return hipSuccess;
    if (xs && (k % 32 || k > INT32_MAX)) return hipErrorInvalidValue;
    const unsigned rb = (unsigned)((tokens + 3) / 4);
    const unsigned grid = xs ? 2 * rb : rb;
    if (E <= 64)
        moe_route_kernel<1><<<grid, 256, 0, s>>>(logits, tokens, E, top_k, norm, ids, wts, rb, x, (int)k, xs);
    else if (E <= 128)
        moe_route_kernel<2><<<grid, 256, 0, s>>>(logits, tokens, E, top_k, norm, ids, wts, rb, x, (int)k, xs);
    else if (E <= 256)
        moe_route_kernel<4><<<grid, 256, 0, s>>>(logits, tokens, E, top_k, norm, ids, wts, rb, x, (int)k, xs);
    else
        moe_route_kernel<MOE_ROUTE_PL><<<grid, 256, 0, s>>>(logits, tokens, E, top_k, norm, ids, wts, rb, x,
                                                            (int)k, xs);
    return hipGetLastError();
}

hipError_t launch_moe_group(const int32_t *ids, int64_t P, int E, int32_t *off, int32_t *sorted,
                            void *tiles, int32_t *ntiles, hipStream_t s) {
    moe_group_kernel<<<1, 1024, 0, s>>>(ids, P, E, MOE_BM, off, sorted, (int2 *)tiles, ntiles);
    return hipGetLastError();
}

int64_t moe_max_tiles(int64_t P, int E) { return (P + MOE_BM - 1) / MOE_BM + E; }

// Workgroups of a grid-stride grouped GEMM: as many as fit on the device at
// once (workgroups per CU from the occupancy query, cached per kernel in
// `fit`), never more than the items can use.
static unsigned moe_grid(const void *fn, int threads, size_t lds, std::atomic<int> &fit,
                         const arfq_weight *w, int64_t max_items) {
    int per_cu = fit.load(std::memory_order_relaxed);
    if (per_cu == 0) {
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, threads, lds) != hipSuccess ||
            per_cu < 1)
            per_cu = 1;
        fit.store(per_cu, std::memory_order_relaxed);
    }
    const int64_t cus = w->ctx && w->ctx->cus > 0 ? w->ctx->cus : 1;
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>(max_items, per_cu * cus));
}

template <class F>
static hipError_t gateup_t(const F &g, const F &u, const arfq_weight *gw, const _Float16 *x,
                           const uint16_t *xs, const float *xrs, int top_k, const int32_t *off,
                           const int32_t *sorted, const void *tiles, const int32_t *ntiles,
                           int64_t max_tiles, float *h, hipStream_t s) {
    constexpr size_t lds = gu_scale_off<F>() + MOE_BM * 4;
    static_assert(gu_scale_off<F>() >= (size_t)4 * 2 * 16 * 64 * 4, "room for the up -> gate hand-off");
    static_assert(gu_scale_off<F>() % 4 == 0, "aligned x scales");
    static std::atomic<uint64_t> lds_set{0};  // the attribute belongs to the kernel, per device
    if (hipError_t err = set_max_lds_once((const void *)moe_gateup_kernel<F>, lds, lds_set)) return err;
    const int64_t eb = gw->n * g.nblk;
    static std::atomic<int> fit{0};
    const unsigned grid = moe_grid((const void *)moe_gateup_kernel<F>, MOE_GU_THREADS, lds, fit, gw,
                                   max_tiles * ((gw->n + 127) / 128));
    moe_gateup_kernel<F><<<grid, MOE_GU_THREADS, lds, s>>>(g, u, eb, x, xs, xrs, (int)gw->k,
                                                       (int)gw->n, top_k, off, sorted,
                                                       (const int2 *)tiles, ntiles, h);
    return hipGetLastError();
}

template <class F>
static hipError_t down_t(const F &d, const arfq_weight *dw, const _Float16 *h, const uint16_t *hs,
                         const float *rs, const int32_t *off, const int32_t *sorted,
                         const void *tiles, const int32_t *ntiles, int64_t max_tiles, float *o,
                         hipStream_t s) {
    const size_t xlds = dxs_lds<F>((int)dw->k);
    if (xlds <= MOE_DXS_LDS_MAX) {  // the tile's rows fit beside the slabs: x-stationary
        static std::atomic<uint64_t> lds_set{0};
        if (hipError_t err = set_max_lds_once((const void *)moe_down_xs_kernel<F>, MOE_DXS_LDS_MAX, lds_set))
            return err;
        const int64_t eb = dw->n * d.nblk;
        const unsigned grid = (unsigned)(max_tiles * ((dw->n + DXS_COLS - 1) / DXS_COLS));
        moe_down_xs_kernel<F><<<grid, DXS_THREADS, xlds, s>>>(d, eb, h, hs, rs, (int)dw->k, (int)dw->n, off,
                                                             sorted, (const int2 *)tiles, ntiles, o);
        return hipGetLastError();
    }
    constexpr size_t lds = sk_lds<F, 2, 1>();
    static std::atomic<uint64_t> lds_set{0};  // the attribute belongs to the kernel, per device
    if (hipError_t err = set_max_lds_once((const void *)moe_down_kernel<F>, lds, lds_set)) return err;
    const int64_t eb = dw->n * d.nblk;
    const dim3 grid((unsigned)max_tiles, (unsigned)((dw->n + 127) / 128));
    moe_down_kernel<F><<<grid, SK_THREADS, lds, s>>>(d, eb, h, hs, rs, (int)dw->k, (int)dw->n, off,
                                                     sorted, (const int2 *)tiles, ntiles, o);
    return hipGetLastError();
}

SkQ4K sk_q4k(const arfq_weight *w);  // arfq_gemm.hip
SkQ6K sk_q6k(const arfq_weight *w);
SkQ80 sk_q80(const arfq_weight *w);
SkQ5K sk_q5k(const arfq_weight *w);
SkIQ4XS sk_iq4xs(const arfq_weight *w);

hipError_t launch_moe_gateup(const arfq_weight *gate, const arfq_weight *up, const _Float16 *x,
                             const uint16_t *xs, const float *xrs, int top_k, const int32_t *off,
                             const int32_t *sorted, const void *tiles, const int32_t *ntiles,
                             int64_t max_tiles, float *h, hipStream_t s) {
    switch (gate->qtype) {
    case ARFQ_Q4_K:
        return gateup_t(sk_q4k(gate), sk_q4k(up), gate, x, xs, xrs, top_k, off, sorted, tiles, ntiles,
                        max_tiles, h, s);
    case ARFQ_Q6_K:
        return gateup_t(sk_q6k(gate), sk_q6k(up), gate, x, xs, xrs, top_k, off, sorted, tiles, ntiles,
                        max_tiles, h, s);
    case ARFQ_Q8_0:
        return gateup_t(sk_q80(gate), sk_q80(up), gate, x, xs, xrs, top_k, off, sorted, tiles, ntiles,
                        max_tiles, h, s);
    case ARFQ_Q5_K:
        return gateup_t(sk_q5k(gate), sk_q5k(up), gate, x, xs, xrs, top_k, off, sorted, tiles, ntiles,
                        max_tiles, h, s);
    case ARFQ_IQ4_XS:
        return gateup_t(sk_iq4xs(gate), sk_iq4xs(up), gate, x, xs, xrs, top_k, off, sorted, tiles,
                        ntiles, max_tiles, h, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_moe_down(const arfq_weight *down, const _Float16 *h, const uint16_t *hs,
                           const float *rs, const int32_t *off,
                           const int32_t *sorted, const void *tiles, const int32_t *ntiles,
                           int64_t max_tiles, float *o, hipStream_t s) {
    switch (down->qtype) {
    case ARFQ_Q4_K:
        return down_t(sk_q4k(down), down, h, hs, rs, off, sorted, tiles, ntiles, max_tiles, o, s);
    case ARFQ_Q6_K:
        return down_t(sk_q6k(down), down, h, hs, rs, off, sorted, tiles, ntiles, max_tiles, o, s);
    case ARFQ_Q8_0:
        return down_t(sk_q80(down), down, h, hs, rs, off, sorted, tiles, ntiles, max_tiles, o, s);
    case ARFQ_Q5_K:
        return down_t(sk_q5k(down), down, h, hs, rs, off, sorted, tiles, ntiles, max_tiles, o, s);
    case ARFQ_IQ4_XS:
        return down_t(sk_iq4xs(down), down, h, hs, rs, off, sorted, tiles, ntiles, max_tiles, o, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_moe_hprep(const float *h, int64_t P, int inter, _Float16 *h16, uint16_t *hs,
                            float *rs, hipStream_t s) {
    if (P == 0) return hipSuccess;
    moe_hprep_kernel<<<(unsigned)((P + 3) / 4), 256, 0, s>>>(h, P, inter, h16, hs, rs);
    return hipGetLastError();
}

hipError_t launch_moe_combine(const float *o, const int32_t *ids, const float *wts, int64_t tokens,
                              int top_k, int E, int64_t hidden, float *y, bool accumulate, hipStream_t s) {
    if (tokens == 0) return hipSuccess;
    const dim3 grid((unsigned)((hidden / 4 + 255) / 256), (unsigned)tokens);
    moe_combine_kernel<<<grid, 256, 0, s>>>(o, ids, wts, top_k, E, (int)hidden, y, accumulate ? 1 : 0);
    return hipGetLastError();
}

}  // namespace arfq
