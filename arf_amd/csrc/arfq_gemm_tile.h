// arfq_gemm_tile.h -- the dequant-into-LDS MFMA tile loop shared by the dense
// GEMM (arfq_gemm.hip) and the expert-grouped MoE GEMMs (arfq_moe.hip).
//
// A workgroup of 256 threads (2 x 2 waves) computes a BM x 128 output tile
// (BM = 64 or 128 x rows, 128 weight rows).  Each wave owns (BM/2) x 64
// outputs as 32 x 32 tiles of v_mfma_f32_32x32x16_f16 with f32 accumulation.
// K advances in steps of 64 "slots".  Each step the workgroup
//   * converts 128 weight rows x 64 slots to f16 in LDS (one 32-slot half row
//     per thread),
//   * copies the matching f16 x tile(s) into LDS,
//   * runs the MFMAs out of LDS (double buffered; rows padded by 16 bytes so
//     the 16-byte LDS reads of the MFMA operands are conflict-free).
// The next step's global loads are issued before the current step's MFMAs.
// A step's 64 slots are one natural unit of the format (two Q4_K sub-blocks,
// one 48-byte Q6_K chunk, two Q8_0 blocks); the x tile is gathered with the
// same slot -> k permutation, so the dot product is unchanged.
//
// Exact weights (Q4_K, Q6_K).  The LDS tile does not hold the weights but the
// integers that multiply the block scale: sc_j * q (Q4_K, <= 63 * 15) and
// sc * (q - 32) (Q6_K), exact in f16, made with packed f16 math from the code
// bits.  Each 256-weight block (4 steps) accumulates into its own registers,
// and at the block's end acc += d * C_block.  Q4_K's min term
// -dmin * sum_j m_j * X_j (X_j: the x sub-block sums, given as bf16 hi + lo
// pairs in xs[row][block][16]) goes straight into acc as two bf16 MFMAs, with
// -dmin * m_j split into bf16 hi + lo.  So y = sum_b (d_b * sum sc*q*x -
// dmin_b * sum m*X) as the reference factorises it
// (crates/arf-ml/src/matmul.rs:327-358); the roundings left are the f32 sums
// and the 16-bit splits of the (small) min term.  (Q6_K: the product sc*(q-32) is exact for |sc| <= 64,
// and rounded to f16 otherwise.)  Q8_0 is stored as d*q rounded to f16.
//
// Activations: f16, or (XSPLIT) an f32 x pre-split into x = hi + lo with hi,
// lo in f16: two MFMAs per tile carry ~22 bits of x.
//
// Reference behaviour: matmul_mm_q4ks.metal:65-290 and moe_mm_id_q4ks.metal
// (dequantize a weight tile into threadgroup memory, simdgroup MMA with f32
// accumulation).
#pragma once
#include "arfq_common.h"

namespace arfq {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int GM_BN = 128, GM_BK = 64, GM_THREADS = 256;
constexpr int GM_LD = GM_BK + 8;  // halves per LDS row: 64 slots + 8 pad (see below)

// LDS bytes of a tile loop: two stages of A (x) and B (weights) tiles, plus
// per weight row the block scale d and the min-term operand (-dmin * m_j as
// bf16 hi, lo).  The 8-half pad of each A row carries the x sub-block sums of
// the block (stage 0 pad: X hi, stage 1 pad: X lo); the 64-slot tile stores
// never touch the pads.
__host__ __device__ constexpr size_t gm_lds(int BM, bool xsplit) {
    return (size_t)2 * ((xsplit ? 2 : 1) * BM + GM_BN) * GM_LD * sizeof(_Float16) +
           (size_t)GM_BN * sizeof(float) + (size_t)GM_BN * 16 * sizeof(uint16_t);
}

// Plain (cached) vector loads into native vector registers.  Weight tiles are
// read by every M tile of the output, so they are not streamed past the cache.
__device__ __forceinline__ u32x4 ldv(const uint4 *p) { return *reinterpret_cast<const u32x4 *>(p); }
__device__ __forceinline__ u32x2 ldv(const uint2 *p) { return *reinterpret_cast<const u32x2 *>(p); }

__device__ __forceinline__ uint32_t pack2h(float a, float b) {
    const __half ha = __float2half_rn(a), hb = __float2half_rn(b);
    return (uint32_t)__half_as_ushort(ha) | ((uint32_t)__half_as_ushort(hb) << 16);
}
__device__ __forceinline__ half2v as_h2(uint32_t u) { return __builtin_bit_cast(half2v, u); }
__device__ __forceinline__ uint32_t as_u(half2v h) { return __builtin_bit_cast(uint32_t, h); }
__device__ __forceinline__ half2v h2splat(float f) {
    const _Float16 h = (_Float16)f;
    return half2v{h, h};
}
// v_pk_fma_f16 (one rounding per half)
__device__ __forceinline__ uint32_t pk_fma(uint32_t a, half2v b, half2v c) {
    return as_u(__builtin_elementwise_fma(as_h2(a), b, c));
}
// f32 -> bf16 bits, round to nearest even (finite inputs)
__device__ __forceinline__ uint32_t bf16_bits(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float bf16_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// ---- weight formats --------------------------------------------------------
// KIND 0: the tile holds the weights rounded to f16; KIND 1: exact integers
// times the block scale d; KIND 2: as 1, minus dmin * (mins . x sub-block sums).
// xk(st, q): k index of slot 8q of step st (slots 8q..8q+7 are 8 consecutive
// k);  load(): the raw data of half `ws` of weight row `row` for step st;
// deq(): its 32 values as f16 pairs, o[4r..4r+3] = the 8 halves at slot
// run_off(ws, r), given the step's phase ph = st % 4 (a compile-time constant
// in the unrolled tile loop, so no branch on it survives);  scale(): (d, dmin) of the raw's block;  mins(): the block's
// 8 sub-block mins as 4 bf16 pairs.

// Q4_K: step st = sub-blocks 2p, 2p+1 (p = st % 4) of block st / 4; half ws =
// sub-block 2p + ws, slots 32ws + e = element 64p + 32ws + e.
struct FmtQ4K {
    static constexpr int KIND = 2;
    static constexpr bool PHASED = true;  // deq depends on st % 4
    static constexpr int WG_PER_CU = 1;   // the tile kernel's launch bound (workgroups per CU)
    struct Raw {
        u32x4 c, h;
    };
    const uint4 *hdr, *qs;
    int nblk;
    // the same matrix shifted by `nb` blocks (an expert's first block)
    __host__ __device__ FmtQ4K shifted(int64_t nb) const { return {hdr + nb, qs + nb * 8, nblk}; }
    __device__ static int xk(int st, int q) { return (st >> 2) * 256 + 64 * (st & 3) + 8 * q; }
    __device__ static int run_off(int ws, int r) { return 32 * ws + 8 * r; }
    // ph = st % 4 (a compile-time constant at the call site): only the header
    // dwords the step uses are loaded -- d|dmin and the mins (dwords 0, 2) only
    // for phase 1, whose raw also feeds the block's scale and min-term
    // operands.  A wide load whose lanes die early lets the register allocator
    // reuse them while the load is in flight, which costs a full wait.
    __device__ Raw load(int64_t row, int st, int ws, int ph) const {
        const int64_t blk = row * nblk + (st >> 2);
        Raw r;
        r.c = ldv(qs + blk * 8 + 2 * (st & 3) + ws);
        const uint32_t *hp = reinterpret_cast<const uint32_t *>(hdr + blk);
        if (ph == 1) {
            r.h = ldv(hdr + blk);
        } else {
            r.h.x = 0u;
            r.h.y = hp[1];
            r.h.z = 0u;
            r.h.w = ph >= 2 ? hp[3] : 0u;
        }
        return r;
    }
    // sc_j * q as f16.  Low nibbles become 1024 + q (0x6400 | q) and
    // (1024 + q) * sc - 1024 * sc = sc * q; high nibbles, left in place, become
    // 1024 + 16 q and (1024 + 16 q) * (sc / 16) - 64 * sc = sc * q.  Each FMA is
    // exact (the result is an integer <= 945).
    __device__ static void deq(const Raw &r, int ph, int ws, uint32_t o[16]) {
        const int j = 2 * ph + ws;
        uint32_t sc, mm;
        q4k_scale_min(r.h.y, r.h.z, r.h.w, j, sc, mm);
        const float scf = (float)sc;
        const half2v s1 = h2splat(scf), c1 = h2splat(-1024.f * scf);
        const half2v s16 = h2splat(scf * 0.0625f), c16 = h2splat(-64.f * scf);
        const uint32_t cw[4] = {r.c.x, r.c.y, r.c.z, r.c.w};
#pragma unroll
        for (int w = 0; w < 4; w++) {
            // dword w: byte i low nibble = element 8w+i, high nibble = element 8w+4+i
            const uint32_t t01 = __builtin_amdgcn_perm(0u, cw[w], 0x0c010c00u);  // b0 . b1 .
            const uint32_t t23 = __builtin_amdgcn_perm(0u, cw[w], 0x0c030c02u);  // b2 . b3 .
            o[4 * w + 0] = pk_fma((t01 & 0x000F000Fu) | 0x64006400u, s1, c1);
            o[4 * w + 1] = pk_fma((t23 & 0x000F000Fu) | 0x64006400u, s1, c1);
            o[4 * w + 2] = pk_fma((t01 & 0x00F000F0u) | 0x64006400u, s16, c16);
            o[4 * w + 3] = pk_fma((t23 & 0x00F000F0u) | 0x64006400u, s16, c16);
        }
    }
    __device__ static float2 scale(const Raw &r) {
        return make_float2(h2f(r.h.x), h2f(r.h.x >> 16));
    }
    __device__ static void mins(const Raw &r, uint32_t m[4]) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint32_t s0, m0, s1, m1;
            q4k_scale_min(r.h.y, r.h.z, r.h.w, 2 * i, s0, m0);
            q4k_scale_min(r.h.y, r.h.z, r.h.w, 2 * i + 1, s1, m1);
            m[i] = bf16_bits((float)m0) | (bf16_bits((float)m1) << 16);
        }
    }
};

// Q6_K: step st = 48-byte chunk c = st % 4 of block st / 4 (n2 = c/2,
// isub = c%2); slot 16t + i is element 128*n2 + 16*isub + 32t + i (quadrant t,
// position i).  Half ws holds positions 8ws..8ws+7 of all four quadrants.
struct FmtQ6K {
    static constexpr int KIND = 1;
    static constexpr bool PHASED = true;
    static constexpr int WG_PER_CU = 1;
    struct Raw {
        u32x2 qa, qb, qh, sc;
        uint32_t d;
    };
    const uint2 *qb8;  // the 192-byte chunk streams as 8-byte units
    const uint2 *sc8;  // 16 scale bytes per block as 8-byte units
    const uint16_t *dd;
    int nblk;
    __host__ __device__ FmtQ6K shifted(int64_t nb) const {
        return {qb8 + nb * 24, sc8 + nb * 2, dd + nb, nblk};
    }
    __device__ static int xk(int st, int q) {
        const int c = st & 3;
        return (st >> 2) * 256 + 128 * (c >> 1) + 16 * (c & 1) + 32 * (q >> 1) + 8 * (q & 1);
    }
    __device__ static int run_off(int ws, int r) { return 16 * r + 8 * ws; }
    __device__ Raw load(int64_t row, int st, int ws, int) const {
        const int64_t blk = row * nblk + (st >> 2);
        const int c = st & 3;
        const uint2 *ch = qb8 + blk * 24 + c * 6;  // ql_a[16] | ql_b[16] | qh[16]
        Raw r;
        r.qa = ldv(ch + ws);
        r.qb = ldv(ch + 2 + ws);
        r.qh = ldv(ch + 4 + ws);
        r.sc = ldv(sc8 + blk * 2 + (c >> 1));  // scales 8*n2 .. 8*n2+7
        r.d = dd[blk];
        return r;
    }
    // sc * (q - 32) as f16: q as 1024 + q (0x6400 | q), minus 1056, times sc.
    __device__ static void deq(const Raw &r, int ph, int, uint32_t o[16]) {
        const int isub = ph & 1;
        const uint32_t scw[2] = {r.sc.x, r.sc.y};
        const half2v m1056 = h2splat(-1056.f);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int si = isub + 2 * t;  // scale 8*n2 + isub + 2t
            const half2v s = h2splat((float)(int8_t)(scw[si >> 2] >> (8 * (si & 3))));
            // t=0: ql_a low | qh bits 0-1;  t=1: ql_b low | qh 2-3;
            // t=2: ql_a high | qh 4-5;      t=3: ql_b high | qh 6-7
            const u32x2 ql = (t & 1) ? r.qb : r.qa;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint32_t l = h ? ql.y : ql.x, hh = h ? r.qh.y : r.qh.x;
#pragma unroll
                for (int pr = 0; pr < 2; pr++) {
                    const uint32_t sel = pr ? 0x0c030c02u : 0x0c010c00u;
                    const uint32_t lp = __builtin_amdgcn_perm(0u, l, sel);
                    const uint32_t hp = __builtin_amdgcn_perm(0u, hh, sel);
                    const uint32_t nib = (t & 2) ? ((lp >> 4) & 0x000F000Fu) : (lp & 0x000F000Fu);
                    const uint32_t top = ((hp >> (2 * t)) & 0x00030003u) << 4;
                    const half2v q = as_h2(nib | top | 0x64006400u);
                    o[4 * t + 2 * h + pr] = as_u((q + m1056) * s);
                }
            }
        }
    }
    __device__ static float2 scale(const Raw &r) { return make_float2(h2f(r.d), 0.f); }
    __device__ static void mins(const Raw &, uint32_t m[4]) { m[0] = m[1] = m[2] = m[3] = 0; }
};

// Q4_K and Q6_K with the weights rounded to f16 (KIND 0): the prefill tiles
// (m > 64), where MFMA throughput, not bytes, is the bound and the register
// file holds no room for per-block accumulators.  One rounding per weight
// (relative error <= 2^-11).  The reference's dense prefill tile holds f32
// weights by default and f16 only under MM_HALF_FRAG
// (matmul_mm_q4ks.metal:161-171); its MoE tiles are f16
// (moe_mm_id_q4ks.metal:34-46).
struct FmtQ4KR : FmtQ4K {
    static constexpr int KIND = 0;
    __host__ __device__ FmtQ4KR shifted(int64_t nb) const { return {FmtQ4K::shifted(nb)}; }
    __device__ Raw load(int64_t row, int st, int ws, int) const {
        const int64_t blk = row * nblk + (st >> 2);
        Raw r;
        r.c = ldv(qs + blk * 8 + 2 * (st & 3) + ws);
        r.h = ldv(hdr + blk);
        return r;
    }
    __device__ static void deq(const Raw &r, int ph, int ws, uint32_t o[16]) {
        const int j = 2 * ph + ws;
        uint32_t sc, mm;
        q4k_scale_min(r.h.y, r.h.z, r.h.w, j, sc, mm);
        const float d1 = h2f(r.h.x) * (float)sc;
        const float m1 = h2f(r.h.x >> 16) * (float)mm;
        const uint32_t cw[4] = {r.c.x, r.c.y, r.c.z, r.c.w};
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const uint32_t lo = cw[w] & 0x0F0F0F0Fu, hi = (cw[w] >> 4) & 0x0F0F0F0Fu;
            o[4 * w + 0] = pack2h(fmaf(d1, (float)(lo & 0xffu), -m1), fmaf(d1, (float)((lo >> 8) & 0xffu), -m1));
            o[4 * w + 1] = pack2h(fmaf(d1, (float)((lo >> 16) & 0xffu), -m1), fmaf(d1, (float)(lo >> 24), -m1));
            o[4 * w + 2] = pack2h(fmaf(d1, (float)(hi & 0xffu), -m1), fmaf(d1, (float)((hi >> 8) & 0xffu), -m1));
            o[4 * w + 3] = pack2h(fmaf(d1, (float)((hi >> 16) & 0xffu), -m1), fmaf(d1, (float)(hi >> 24), -m1));
        }
    }
};

struct FmtQ6KR : FmtQ6K {
    static constexpr int KIND = 0;
    __host__ __device__ FmtQ6KR shifted(int64_t nb) const { return {FmtQ6K::shifted(nb)}; }
    // s*q - 32s with one rounding == (d*sc)*(q-32) in f32, then f16
    __device__ static void deq(const Raw &r, int ph, int, uint32_t o[16]) {
        const int isub = ph & 1;
        const float d = h2f(r.d);
        const uint32_t scw[2] = {r.sc.x, r.sc.y};
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int si = isub + 2 * t;
            const float sf = d * (float)(int8_t)(scw[si >> 2] >> (8 * (si & 3)));
            const float m32 = -32.f * sf;
            const u32x2 ql = (t & 1) ? r.qb : r.qa;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint32_t l = h ? ql.y : ql.x, hh = h ? r.qh.y : r.qh.x;
                const uint32_t nib = (t & 2) ? ((l >> 4) & 0x0F0F0F0Fu) : (l & 0x0F0F0F0Fu);
                const uint32_t q = nib | (((hh >> (2 * t)) & 0x03030303u) << 4);
                o[4 * t + 2 * h] = pack2h(fmaf((float)(q & 0xffu), sf, m32), fmaf((float)((q >> 8) & 0xffu), sf, m32));
                o[4 * t + 2 * h + 1] = pack2h(fmaf((float)((q >> 16) & 0xffu), sf, m32), fmaf((float)(q >> 24), sf, m32));
            }
        }
    }
};

// Q5_K with the weights rounded to f16 (KIND 0, prefill): Q4_K's step map
// (step st = sub-blocks 2p, 2p + 1, p = st % 4; half ws = sub-block 2p + ws,
// slots 32 ws + e = element e of that sub-block) over ggml's block layout
// qh[32] | qs[128] after the 16-byte header.  Element e of sub-block s is the
// low (s even) or high nibble of qs[32 (s / 2) + e] plus bit s of qh[e] as
// bit 4; its weight (d * sc) * q - dmin * m (dequant_q5_k,
// crates/arf-core/src/model/gguf.rs:2053-2090) is formed in f32 and rounded
// once to f16.
struct FmtQ5KR {
    static constexpr int KIND = 0;
    static constexpr bool PHASED = true;
    static constexpr int WG_PER_CU = 2;  // within 256 registers (one per CU took 268)
    struct Raw {
        u32x4 q0, q1, h0, h1, hd;
    };
    const uint4 *hdr;
    const uint8_t *q;  // qh | qs, 160 bytes per block
    int nblk;
    __host__ __device__ FmtQ5KR shifted(int64_t nb) const { return {hdr + nb, q + nb * 160, nblk}; }
    __device__ static int xk(int st, int qd) { return (st >> 2) * 256 + 64 * (st & 3) + 8 * qd; }
    __device__ static int run_off(int ws, int r) { return 32 * ws + 8 * r; }
    __device__ Raw load(int64_t row, int st, int, int) const {
        const int64_t blk = row * nblk + (st >> 2);
        const uint4 *b = reinterpret_cast<const uint4 *>(q + blk * 160);
        Raw r;
        r.h0 = ldv(b);
        r.h1 = ldv(b + 1);
        r.q0 = ldv(b + 2 + 2 * (st & 3));
        r.q1 = ldv(b + 3 + 2 * (st & 3));
        r.hd = ldv(hdr + blk);
        return r;
    }
    __device__ static void deq(const Raw &r, int ph, int ws, uint32_t o[16]) {
        const int s = 2 * ph + ws;
        uint32_t sc, mm;
        q4k_scale_min(r.hd.y, r.hd.z, r.hd.w, s, sc, mm);
        const float d1 = h2f(r.hd.x) * (float)sc;
        const float m1 = h2f(r.hd.x >> 16) * (float)mm;
        const uint32_t qw[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
        const uint32_t hw[8] = {r.h0.x, r.h0.y, r.h0.z, r.h0.w, r.h1.x, r.h1.y, r.h1.z, r.h1.w};
#pragma unroll
        for (int w = 0; w < 8; w++) {
            // elements 4w .. 4w + 3, one per byte
            const uint32_t v = ((qw[w] >> (4 * ws)) & 0x0F0F0F0Fu) | bit_to4(hw[w], s);
            o[2 * w] = pack2h(fmaf(d1, (float)(v & 0xffu), -m1), fmaf(d1, (float)((v >> 8) & 0xffu), -m1));
            o[2 * w + 1] = pack2h(fmaf(d1, (float)((v >> 16) & 0xffu), -m1), fmaf(d1, (float)(v >> 24), -m1));
        }
    }
    __device__ static float2 scale(const Raw &) { return make_float2(1.f, 0.f); }
    __device__ static void mins(const Raw &, uint32_t m[4]) { m[0] = m[1] = m[2] = m[3] = 0; }
};

// IQ4_XS with the weights rounded to f16 (KIND 0, prefill): the same step map
// (half ws = sub-block 2p + ws); the 16 code bytes of sub-block s hold its
// elements 0..15 in the low nibbles and 16..31 in the high ones.  Weight
// (d * (ls - 32)) * kvalues[code] in f32 (dequant_iq4_xs,
// crates/arf-core/src/model/gguf.rs:1937-1976), rounded once to f16.
struct FmtIQ4XSR {
    static constexpr int KIND = 0;
    static constexpr bool PHASED = true;
    static constexpr int WG_PER_CU = 2;
    struct Raw {
        u32x4 c;
        u32x2 h;  // d | scales_h << 16, scales_l
    };
    const uint2 *hdr;
    const uint4 *qs;
    int nblk;
    __host__ __device__ FmtIQ4XSR shifted(int64_t nb) const { return {hdr + nb, qs + nb * 8, nblk}; }
    __device__ static int xk(int st, int qd) { return (st >> 2) * 256 + 64 * (st & 3) + 8 * qd; }
    __device__ static int run_off(int ws, int r) { return 32 * ws + 8 * r; }
    __device__ Raw load(int64_t row, int st, int ws, int) const {
        const int64_t blk = row * nblk + (st >> 2);
        Raw r;
        r.c = ldv(qs + blk * 8 + 2 * (st & 3) + ws);
        r.h = ldv(hdr + blk);
        return r;
    }
    __device__ static void deq(const Raw &r, int ph, int ws, uint32_t o[16]) {
        const int s = 2 * ph + ws;
        const int ls = (int)(((r.h.y >> (4 * s)) & 0xFu) | (((r.h.x >> (16 + 2 * s)) & 3u) << 4));
        const float dl = h2f(r.h.x) * (float)(ls - 32);
        const float m128 = -128.f * dl;  // exact
        const uint32_t cw[4] = {r.c.x, r.c.y, r.c.z, r.c.w};
#pragma unroll
        for (int nib = 0; nib < 2; nib++)
#pragma unroll
            for (int w = 0; w < 4; w++) {
                // elements 16 nib + 4w .. + 3: kv + 128 per byte
                const uint32_t sel = (cw[w] >> (4 * nib)) & 0x0F0F0F0Fu;
                const uint32_t v = iq4nl_lookup<0x80808080u>(sel);  // kv + 128 per byte
                // (kv + 128) * dl - 128 dl = kv * dl, one rounding
                o[8 * nib + 2 * w] = pack2h(fmaf(dl, (float)(v & 0xffu), m128), fmaf(dl, (float)((v >> 8) & 0xffu), m128));
                o[8 * nib + 2 * w + 1] = pack2h(fmaf(dl, (float)((v >> 16) & 0xffu), m128), fmaf(dl, (float)(v >> 24), m128));
            }
    }
    __device__ static float2 scale(const Raw &) { return make_float2(1.f, 0.f); }
    __device__ static void mins(const Raw &, uint32_t m[4]) { m[0] = m[1] = m[2] = m[3] = 0; }
};

// Q8_0: step st = blocks 2st, 2st+1; half ws = block 2st + ws.  Weights d*q
// rounded to f16.
struct FmtQ80 {
    static constexpr int KIND = 0;
    static constexpr bool PHASED = false;
    static constexpr int WG_PER_CU = 1;
    struct Raw {
        u32x4 a, b;
        uint32_t d;
    };
    const uint4 *qs;
    const uint16_t *dd;
    int nblk;
    __host__ __device__ FmtQ80 shifted(int64_t nb) const { return {qs + nb * 2, dd + nb, nblk}; }
    __device__ static int xk(int st, int q) { return st * 64 + 8 * q; }
    __device__ static int run_off(int ws, int r) { return 32 * ws + 8 * r; }
    __device__ Raw load(int64_t row, int st, int ws, int) const {
        const int64_t blk = row * nblk + 2 * st + ws;
        Raw r;
        r.a = ldv(qs + blk * 2);
        r.b = ldv(qs + blk * 2 + 1);
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
    __device__ static float2 scale(const Raw &) { return make_float2(1.f, 0.f); }
    __device__ static void mins(const Raw &, uint32_t m[4]) { m[0] = m[1] = m[2] = m[3] = 0; }
};

// ---- the tile loop ----------------------------------------------------------
template <int BM, bool XSPLIT>
struct TileShape {
    static constexpr int TA = BM / 64;         // 32-row MFMA tiles per wave along m
    static constexpr int XI = BM / 32;         // x rows loaded per thread (16 B each)
    static constexpr int NA = XSPLIT ? 2 : 1;  // x matrices (hi, lo)
    static constexpr int ATILE = BM * GM_LD, BTILE = GM_BN * GM_LD;
    static constexpr int STAGE = NA * ATILE + BTILE;
};

// Accumulates acc[t][b] += x_tile . W_tile^T over steps [st0, st1).
//   wrow     this thread's weight row (tile row tid >> 1, clamped in range)
//   xrow[i]  element offset (row * K) into xh / xl of this thread's i-th x row
//            (tile row (tid >> 3) + 32 i)
//   xsrow[i] element offset (row * K / 16) into xs of the same rows: the x
//            sub-block sums, 16 bf16 per 256-element block (8 hi, then 8 lo);
//            read only for KIND 2 formats
// For formats whose decode depends on st % 4 (PHASED: Q4_K, Q6_K) st0 and st1
// are multiples of 4 (whole 256-element blocks); Q8_0 ranges are arbitrary.
// Global loads run D steps ahead of the MFMAs in a register ring (D = 4 for
// 64-row tiles, which stream weights, 2 when x comes as hi + lo; 2 for
// 128-row tiles, 1 with hi + lo x, whose registers go to the second A tile;
// at C4's shape D = 2 against 1 took Q6_K 811 -> 767 us, IQ4_XS 732 -> 713,
// Q5_K 766 -> 752, Q8_0 701 -> 694, and D = 4 no further); a load past st1
// re-reads step st1 - 1 (a cache hit), which keeps the ring free of branches.
// The caller zeroes acc and owns `lds` (gm_lds(BM, XSPLIT) bytes).
template <class F, int BM, bool XSPLIT>
__device__ __forceinline__ void gemm_tile_run(const F &fmt, int64_t wrow,
                                              const int64_t (&xrow)[BM / 32],
                                              const int64_t (&xsrow)[BM / 32],
                                              const _Float16 *__restrict__ xh,
                                              const _Float16 *__restrict__ xl,
                                              const uint16_t *__restrict__ xs, int st0, int st1,
                                              floatx16 (&acc)[BM / 64][2], _Float16 *lds) {
    using S = TileShape<BM, XSPLIT>;
    constexpr int TA = S::TA, XI = S::XI, NA = S::NA, ATILE = S::ATILE, STAGE = S::STAGE;
    constexpr int KIND = F::KIND;
    constexpr int D = BM == 64 ? (XSPLIT ? 2 : 4) : (XSPLIT ? 1 : 2);  // prefetch depth (steps), divides 4
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    const int xr = tid >> 3, xq = tid & 7;
    const int wr = tid >> 1, ws = tid & 1;
    float *sdv_lds = reinterpret_cast<float *>(lds + 2 * STAGE);        // d per weight row
    uint16_t *bv_lds = reinterpret_cast<uint16_t *>(sdv_lds + GM_BN);  // -dmin*m hi[8] lo[8]

    // the ring: x hi (or x), x lo and the raw weight data of D steps.  Native
    // vector types: arrays of the HIP uint4 struct were left in scratch memory
    // by the compiler.
    u32x4 xa[D][XI], xb[D][XSPLIT ? XI : 1];
    typename F::Raw wv[D];
    u32x4 xsv[KIND == 2 ? XI : 1];  // x sub-block sums of the next block to stage
    auto gload = [&](int slot, int st, int ph) {
        const int kx = F::xk(st, xq);
#pragma unroll
        for (int i = 0; i < XI; i++) {
            xa[slot][i] = *reinterpret_cast<const u32x4 *>(xh + xrow[i] + kx);
            if constexpr (XSPLIT) xb[slot][i] = *reinterpret_cast<const u32x4 *>(xl + xrow[i] + kx);
        }
        wv[slot] = fmt.load(wrow, st, ws, ph);
    };
    // the x sub-block sums of block blk: thread xq & 1 takes the hi or lo half
    auto xsload = [&](u32x4 (&dst)[KIND == 2 ? XI : 1], int blk) {
        if constexpr (KIND == 2) {
#pragma unroll
            for (int i = 0; i < XI; i++)
                dst[i] = *reinterpret_cast<const u32x4 *>(xs + xsrow[i] + blk * 16 + 8 * (xq & 1));
        }
    };
    auto lstore = [&](int buf, int slot, int ph) {
        _Float16 *As = lds + buf * STAGE;
        _Float16 *Bs = As + NA * ATILE;
#pragma unroll
        for (int i = 0; i < XI; i++) {
            *reinterpret_cast<u32x4 *>(As + (xr + 32 * i) * GM_LD + 8 * xq) = xa[slot][i];
            if constexpr (XSPLIT)
                *reinterpret_cast<u32x4 *>(As + ATILE + (xr + 32 * i) * GM_LD + 8 * xq) = xb[slot][i];
        }
        uint32_t o[16];
        F::deq(wv[slot], ph, ws, o);
#pragma unroll
        for (int r = 0; r < 4; r++)
            *reinterpret_cast<uint4 *>(Bs + wr * GM_LD + F::run_off(ws, r)) =
                make_uint4(o[4 * r], o[4 * r + 1], o[4 * r + 2], o[4 * r + 3]);
    };
    // a block's scale and min-term operands (from the raw of one of its steps)
    auto bstore = [&](int slot) {
        if (ws == 0) {
            const float2 dd = F::scale(wv[slot]);
            sdv_lds[wr] = dd.x;
            if constexpr (KIND == 2) {
                uint32_t m[4];
                F::mins(wv[slot], m);
                uint32_t hi[4], lo[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    uint32_t h2[2], l2[2];
#pragma unroll
                    for (int u = 0; u < 2; u++) {
                        const float v = -dd.y * bf16_to_f32((m[i] >> (16 * u)) & 0xffffu);
                        h2[u] = bf16_bits(v);
                        l2[u] = bf16_bits(v - bf16_to_f32(h2[u]));
                    }
                    hi[i] = h2[0] | (h2[1] << 16);
                    lo[i] = l2[0] | (l2[1] << 16);
                }
                *reinterpret_cast<uint4 *>(bv_lds + wr * 16) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
                *reinterpret_cast<uint4 *>(bv_lds + wr * 16 + 8) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
            }
        }
        if constexpr (KIND == 2) {
            if (xq < 2) {
#pragma unroll
                for (int i = 0; i < XI; i++)
                    *reinterpret_cast<u32x4 *>(lds + xq * STAGE + (xr + 32 * i) * GM_LD + GM_BK) = xsv[i];
            }
        }
    };

    const int lr = lane & 31, lk = (lane >> 5) * 8;
    auto mfma_step = [&](int buf, floatx16 (&c)[TA][2]) {
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
            for (int b = 0; b < 2; b++)
                bf[b] = *reinterpret_cast<const half8 *>(Bs + (wn * 64 + 32 * b + lr) * GM_LD + 16 * kk + lk);
#pragma unroll
            for (int a = 0; a < NA; a++)
#pragma unroll
                for (int t = 0; t < TA; t++)
#pragma unroll
                    for (int b = 0; b < 2; b++)
                        c[t][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[a][t], bf[b], c[t][b], 0, 0, 0);
        }
    };
    // block end (exact formats): acc += d * C_block (+ the Q4_K min term, two
    // bf16 MFMAs into a zeroed temporary).  acc is only touched by VALU ops and
    // the block sums only by MFMAs, which keeps each in one register file.
    auto block_end = [&](floatx16 (&cb)[TA][2]) {
        const float d0 = sdv_lds[wn * 64 + lr], d1 = sdv_lds[wn * 64 + 32 + lr];
        floatx16 cm[TA][2];
        if constexpr (KIND == 2) {
            // A: stage h pad = X hi (h = 0) / X lo (h = 1); B: (-dmin m) hi, then lo
            const int h = lane >> 5;
            bf16x8 am[TA], bh[2], bl[2];
#pragma unroll
            for (int t = 0; t < TA; t++)
                am[t] = *reinterpret_cast<const bf16x8 *>(
                    lds + h * STAGE + (wm * (BM / 2) + 32 * t + lr) * GM_LD + GM_BK);
#pragma unroll
            for (int b = 0; b < 2; b++) {
                const uint16_t *bvr = bv_lds + (wn * 64 + 32 * b + lr) * 16;
                bh[b] = *reinterpret_cast<const bf16x8 *>(bvr);
                bl[b] = *reinterpret_cast<const bf16x8 *>(bvr + 8);
            }
#pragma unroll
            for (int t = 0; t < TA; t++)
#pragma unroll
                for (int b = 0; b < 2; b++) {
                    floatx16 z;
#pragma unroll
                    for (int i = 0; i < 16; i++) z[i] = 0.f;
                    cm[t][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(am[t], bh[b], z, 0, 0, 0);
                    cm[t][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(am[t], bl[b], cm[t][b], 0, 0, 0);
                }
        }
#pragma unroll
        for (int t = 0; t < TA; t++)
#pragma unroll
            for (int b = 0; b < 2; b++)
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    float a = fmaf(b ? d1 : d0, cb[t][b][i], acc[t][b][i]);
                    if constexpr (KIND == 2) a += cm[t][b][i];
                    acc[t][b][i] = a;
                    cb[t][b][i] = 0.f;
                }
    };

    floatx16 cb[TA][2];
#pragma unroll
    for (int t = 0; t < TA; t++)
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
            for (int i = 0; i < 16; i++) cb[t][b][i] = 0.f;
    // prologue: D steps in flight, the first one staged
#pragma unroll
    for (int d = 0; d < D; d++) gload(d, min(st0 + d, st1 - 1), d & 3);
    xsload(xsv, st0 >> 2);
    lstore(0, 0, 0);
    __syncthreads();
    for (int g = st0; g < st1; g += 4) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int st = g + j;
            if (KIND == 0 && st >= st1) break;  // Q8_0 ranges need not be whole groups of 4
            // slot j % D was staged (step st) last iteration: refill it D ahead
            gload(j % D, min(st + D, st1 - 1), (j + D) & 3);
            // the next block's sums, after this block's were staged (j == 0)
            if (KIND == 2 && j == (D == 4 ? 1 : 3)) xsload(xsv, min((st >> 2) + 1, (st1 >> 2) - 1));
            if constexpr (KIND == 0) {
                mfma_step(j & 1, acc);
            } else {
                mfma_step(j & 1, cb);
                if (j == 3) block_end(cb);
            }
            lstore((j & 1) ^ 1, (j + 1) % D, (j + 1) & 3);  // step st + 1 (stale past st1)
            if (KIND != 0 && j == 0) bstore((j + 1) % D);  // block st / 4: raw of step st + 1, sums xsv
            __syncthreads();
        }
    }
}

// Output coordinates of accumulator element i of tile (t, b) for this lane:
// lane holds column lane % 32 of each 32 x 32 tile, rows 8*(i/4) + 4*(lane/32) + i%4.
template <int BM>
__device__ __forceinline__ int tile_out_row(int t, int i) {
    const int lane = threadIdx.x & 63, wm = (threadIdx.x >> 6) & 1;
    return wm * (BM / 2) + 32 * t + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
}
__device__ __forceinline__ int tile_out_col(int b) {
    const int lane = threadIdx.x & 63, wn = threadIdx.x >> 7;
    return wn * 64 + 32 * b + (lane & 31);
}

// ---- activation preparation ------------------------------------------------
// Row-major [M, K] activation (K a multiple of 32) in segments: workgroup b
// takes segment sp = b % S of row b / S, the elements [e(sp), e(sp + 1)) with
// e(j) = unit * floor(j * (K / unit) / S); one thread per 8 consecutive
// elements, so a quad of lanes covers a 32-element sub-block and every load
// and store is 16 bytes wide and coalesced.  A segment of at most
// XPREP_THREADS * XPREP_NJ * 8 elements is read once, into registers.  Writes x as f16
// (and, when `xl` is set, the f16 remainder x - hi) and, when `xs` is set, the
// sub-block sum X (of the values the MFMAs will see: each lane's 8 in order,
// then the quad's four partial sums pairwise) as bf16 hi + lo into
// xs[row][k / 256][j] and [8 + j] (j = sub-block within block).
// With `pair` set (1: two parts, 2: three), xl must be xh + M * K: the lo
// remainders x - hi (with three parts rounded to f16 as the mid part, whose
// remainder x - hi - mid follows as rows 2M .. 3M - 1) are stored as rows
// M .. 2M - 1 after the hi rows, and xs holds the sums of each hi row at row
// r, of each lo (mid) row at row M + r and of each third-part row at 2M + r;
// otherwise the sums are of hi + lo.
// With `rs` set (f32 x), each segment is first scanned for its max |x| and
// its elements are stored divided by rs[sp * M + row] = 2^(e - 15), e the
// exponent of that max (max in [2^(e-1), 2^e)): an exact power-of-two scaling
// that puts the segment's largest value in [2^14, 2^15), so no finite f32 x
// overflows f16 and small values do not fall into f16 subnormals.  The
// consumers multiply their partial sums over the segment by its scale (with
// S = 1: the output rows).  Segments whose max is 0 or not finite keep
// rs = 1.
constexpr int XPREP_THREADS = 512;
constexpr int XPREP_NJ = 2;  // 8-element chunks per thread loaded together
template <typename TIn>
__device__ __forceinline__ void xprep_load8(const TIn *__restrict__ p, float v[8]) {
    if constexpr (sizeof(TIn) == 4) {
        const float4 a = reinterpret_cast<const float4 *>(p)[0];
        const float4 b = reinterpret_cast<const float4 *>(p)[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
        const half8 a = reinterpret_cast<const half8 *>(p)[0];
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = (float)a[i];
    }
}
// The sub-block sums alone, for an f16 x (no copy, split or scale): one wave
// per row, lane l taking the 32-element sub-blocks l, l + 64, ... with the
// loads of four sub-blocks in flight at once.  Each sum is the one
// xprep_kernel forms for the same input, in the same order: the four 8-element
// runs each summed left to right, then (r0 + r1) + (r2 + r3).
constexpr int XSUM_WAVES = 4;
// One wave: the sums of row `row` (row < M) into xs.
__device__ __forceinline__ void xsums_row(const _Float16 *__restrict__ x, int K, uint16_t *__restrict__ xs,
                                          int64_t row) {
    const int lane = threadIdx.x & 63, nsb = K / 32;
    const half8 *src = reinterpret_cast<const half8 *>(x + row * K);
    uint16_t *dst = xs + row * (K / 16);
    for (int s0 = 0; s0 < nsb; s0 += 64 * 4) {
        half8 v[4][4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int sb = min(s0 + lane + 64 * q, nsb - 1);  // past the end: a re-read, not stored
#pragma unroll
            for (int c = 0; c < 4; c++) v[q][c] = src[4 * sb + c];
        }
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int sb = s0 + lane + 64 * q;
            float r[4];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                float t = 0.f;
#pragma unroll
                for (int i = 0; i < 8; i++) t += (float)v[q][c][i];
                r[c] = t;
            }
            const float sum = (r[0] + r[1]) + (r[2] + r[3]);
            if (sb < nsb) {
                const uint32_t hi = bf16_bits(sum);
                uint16_t *d = dst + (sb >> 3) * 16 + (sb & 7);
                d[0] = (uint16_t)hi;
                d[8] = (uint16_t)bf16_bits(sum - bf16_to_f32(hi));
            }
        }
    }
}
template <int NW>  // rows (waves) per workgroup
__global__ __launch_bounds__(64 * NW) void xsums_kernel(const _Float16 *__restrict__ x, int64_t M, int K,
                                                       uint16_t *__restrict__ xs) {
    const int64_t row = (int64_t)blockIdx.x * NW + (threadIdx.x >> 6);
    if (row >= M) return;  // whole waves
    xsums_row(x, K, xs, row);
}

template <typename TIn>
__global__ __launch_bounds__(XPREP_THREADS) void xprep_kernel(
    const TIn *__restrict__ x, int64_t M, int K, _Float16 *__restrict__ xh, _Float16 *__restrict__ xl,
    uint16_t *__restrict__ xs, float *__restrict__ rs, int pair, int S, int unit) {
    __shared__ float wmax[XPREP_THREADS / 64];
    const int64_t row = blockIdx.x / S;
    const int sp = blockIdx.x % S, tid = threadIdx.x;
    const int nu = K / unit;
    const int c0 = unit / 8 * (int)((int64_t)sp * nu / S);  // first and last + 1 8-element chunk
    const int c1 = unit / 8 * (int)((int64_t)(sp + 1) * nu / S);
    const int nch = K / 8;
    const TIn *xr = x + row * K;
    // up to XPREP_NJ chunks per thread are loaded together (all in flight), then
    // processed; a longer segment is walked in rounds of that many (twice with rs)
    constexpr int NJ = XPREP_NJ, STEP = XPREP_THREADS * NJ;
    float v[NJ][8];
    auto load_round = [&](int base) {
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const int ch = base + tid + XPREP_THREADS * j;
            if (ch < c1) xprep_load8(xr + (int64_t)ch * 8, v[j]);
        }
    };
    const bool once = c1 - c0 <= STEP;  // the segment in registers
    if (once) load_round(c0);
    int sh = 0;  // elements are stored times 2^sh
    if (rs) {
        float amax = 0.f;
        for (int base = c0; base < c1; base += STEP) {
            if (!once) load_round(base);
#pragma unroll
            for (int j = 0; j < NJ; j++)
                if (base + tid + XPREP_THREADS * j < c1)
#pragma unroll
                    for (int i = 0; i < 8; i++) amax = fmaxf(amax, fabsf(v[j][i]));
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
        if ((tid & 63) == 0) wmax[tid >> 6] = amax;
        __syncthreads();
        amax = wmax[0];
#pragma unroll
        for (int w = 1; w < XPREP_THREADS / 64; w++) amax = fmaxf(amax, wmax[w]);
        if (amax > 0.f && amax < INFINITY) sh = 15 - __builtin_amdgcn_frexp_expf(amax);
        if (tid == 0) rs[(int64_t)sp * M + row] = ldexpf(1.f, -sh);
    }
    // c0 % 4 == 0 and the strides are multiples of 4: a quad's lanes run the
    // same iterations, so the quad DPP sums below see the whole sub-block
    for (int base = c0; base < c1; base += STEP) {
        if (!once) load_round(base);
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const int ch = base + tid + XPREP_THREADS * j;
            if (ch >= c1) break;
            const int64_t g = row * nch + ch;
            half8 hv, lv, ov;  // hi, lo (the mid part with three parts), lo of three
            float sum = 0.f, suml = 0.f, sumo = 0.f;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float u = sh ? ldexpf(v[j][i], sh) : v[j][i];
                hv[i] = (_Float16)u;
                const float r1 = u - (float)hv[i];  // exact
                lv[i] = (_Float16)r1;
                sum += (xl && !pair) ? ((float)hv[i] + (float)lv[i]) : (float)hv[i];
                suml += (float)lv[i];
                if (pair == 2) {
                    ov[i] = (_Float16)(r1 - (float)lv[i]);  // r1 - lo exact; two bits or fewer
                    sumo += (float)ov[i];
                }
            }
            if (xh) reinterpret_cast<half8 *>(xh)[g] = hv;
            if (xl) reinterpret_cast<half8 *>(xl)[g] = lv;
            if (pair == 2) reinterpret_cast<half8 *>(xl)[g + M * nch] = ov;
            if (xs) {
                // (s0 + s1) + (s2 + s3) on every lane of the quad (quad_perm [1,0,3,2], then [2,3,0,1])
                auto quad_sum = [](float t) {
                    t += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(t), 0xB1, 0xf, 0xf, true));
                    return t + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(t), 0x4E, 0xf, 0xf, true));
                };
                sum = quad_sum(sum);
                if (pair) suml = quad_sum(suml);
                if (pair == 2) sumo = quad_sum(sumo);
                if ((ch & 3) == 0) {
                    const int sub = ch >> 2;
                    auto put = [&](int64_t r, float t) {
                        const uint32_t hi = bf16_bits(t);
                        const uint32_t lo = bf16_bits(t - bf16_to_f32(hi));
                        uint16_t *d = xs + r * (K / 16) + (sub >> 3) * 16 + (sub & 7);
                        d[0] = (uint16_t)hi;
                        d[8] = (uint16_t)lo;
                    };
                    put(row, sum);
                    if (pair) put(M + row, suml);
                    if (pair == 2) put(2 * M + row, sumo);
                }
            }
        }
    }
}

}  // namespace arfq
