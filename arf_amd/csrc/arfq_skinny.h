// arfq_skinny.h -- weight-streaming MFMA tile loop for skinny products
// (m <= 64 activation rows): batched decode and the MoE expert tiles.
//
// A workgroup is 4 waves; wave w owns 32 weight rows and all (up to 64) x
// rows of the tile.  Per 256-element block each wave loads its 32 rows'
// weight bytes with fully coalesced 16-byte loads (whole cache lines: a load
// that touched 32 rows at once would leave the L1 miss queue, not HBM, as the
// limit), one block ahead of use, and parks them in a wave-private LDS slab.
// From the slab each lane reads, per step, the bytes of the
// v_mfma_f32_32x32x16_f16 B operand it owns -- lane l holds weight row l % 32
// and, per MFMA, 8 consecutive k of its half (l / 32) -- so no barrier guards
// the weights.  x is staged in LDS one block at a time and shared by the 4
// waves (two barriers per block).
//
// The weight operand is exact: Q4_K lanes hold sc_j * q as f16 integers;
// each block accumulates separately and is scaled by the lane's own d at the
// block end (lane l's C column is its weight row, so d is a register, not a
// broadcast).  Q4_K's min term -dmin * sum_j m_j * X_j enters as two bf16
// MFMAs against the x sub-block sums X_j.  Q5_K is Q4_K with a 5-bit q.
// IQ4_XS lanes hold the codebook values, Q8_0 lanes the int8 codes and Q6_K
// lanes q - 32; each MFMA (two for IQ4_XS) covers one sub-block (one Q8_0
// block) and its result is scaled by that sub-block's d * (ls - 32) (d,
// d * sc) in f32.
//
// K-slot map of step p (64 elements) of block b: lane half h and MFMA kk use
// elements a_off(p, kk, h) + 0..7 of the block; the x operand is read from LDS
// with the same map, so the contraction is unchanged.
//
// Reference behaviour: matmul_vec_q4ks_batch_msl.metal:104-288 (B <= 64 rows
// share each unpacked weight) with the arithmetic of matmul_nt_q4ks /
// matmul_nt_q8_0 (crates/arf-ml/src/matmul.rs:174-204,322-400) and
// dequant_q6_k (crates/arf-core/src/model/gguf.rs:2092-2131).
#pragma once
#include "arfq_gemm_tile.h"

namespace arfq {

constexpr int SK_THREADS = 256;
constexpr int SK_XLD = 256 + 8;  // halves per x row in LDS (16 bytes of padding)


// threadIdx.x behind an empty asm: values derived from it are computed where
// it is read, so in a kernel that loops over work items they are not hoisted
// out of that loop (where they would stay live across the whole loop body and
// crowd the tile loop's registers).
__device__ __forceinline__ int sk_tid() {
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

__device__ __forceinline__ half8 u4_to_h8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    return __builtin_bit_cast(half8, u32x4{a, b, c, d});
}

// ---- formats ------------------------------------------------------------------
// RB: bytes of one weight row's 256-element block in the main stream, loaded
// coalesced by the wave (RB / 16 lanes per row, whole cache lines) into its
// LDS slab [32 rows][RB + 16].  frag(): the lane's B operands of step p from
// its slab row (LDS) and its block data.  load_blk(): the lane's own-row block
// data (scales), one small load per block.

// Q4_K: step p = sub-blocks 2p (h = 0), 2p + 1 (h = 1); MFMA kk = dword kk of
// the lane's sub-block (elements 8kk .. 8kk + 7, sigma nibble order).
struct SkQ4K {
    static constexpr int KIND = 2, RB = 128;
    struct Blk {
        u32x4 h;
    };
    const uint4 *hdr, *qs;
    int nblk;
    __host__ __device__ SkQ4K shifted(int64_t nb) const { return {hdr + nb, qs + nb * 8, nblk}; }
    __device__ static int a_off(int p, int kk, int h) { return 64 * p + 32 * h + 8 * kk; }
    __device__ const uint8_t *raw(int64_t row, int b) const {
        return reinterpret_cast<const uint8_t *>(qs + (row * nblk + b) * 8);
    }
    __device__ Blk load_blk(int64_t row, int b) const { return {ldv(hdr + row * nblk + b)}; }
    __device__ static float2 scale(const Blk &k) { return make_float2(h2f(k.h.x), h2f(k.h.x >> 16)); }
    // B operands of step p: sc_j * q, j = 2p + h.  v_perm puts two code bytes
    // in the low bytes of two halves with 0x64 above them; masking keeps
    // 0x64 and the low nibble (the f16 1024 + q) or the high nibble
    // (1024 + 16 q); then (1024 + q) * sc - 1024 sc and
    // (1024 + 16 q) * (sc / 16) - 64 sc are exact packed f16 FMAs.
    __device__ static void frag(const uint8_t *srow, const Blk &k, int p, int h, half8 f[4]) {
        const u32x4 c = *reinterpret_cast<const u32x4 *>(srow + 32 * p + 16 * h);
        uint32_t sc, mm;
        q4k_scale_min(k.h.y, k.h.z, k.h.w, 2 * p + h, sc, mm);
        const float scf = (float)sc;
        const half2v s1 = h2splat(scf), c1 = h2splat(-1024.f * scf);
        const half2v s16 = h2splat(scf * 0.0625f), c16 = h2splat(-64.f * scf);
        const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
        for (int w = 0; w < 4; w++) {
            // dword w: byte i low nibble = element 8w+i, high nibble = element 8w+4+i
            const uint32_t t01 = __builtin_amdgcn_perm(0x64646464u, cw[w], 0x04010400u);  // b0 64 b1 64
            const uint32_t t23 = __builtin_amdgcn_perm(0x64646464u, cw[w], 0x04030402u);  // b2 64 b3 64
            f[w] = u4_to_h8(pk_fma(t01 & 0x640F640Fu, s1, c1), pk_fma(t23 & 0x640F640Fu, s1, c1),
                            pk_fma(t01 & 0x64F064F0u, s16, c16), pk_fma(t23 & 0x64F064F0u, s16, c16));
        }
    }
    // min-term B operands: (-dmin * m_j) as bf16 hi and lo, j = 0..7
    __device__ static void minsb(const Blk &k, bf16x8 &hi, bf16x8 &lo) {
        const float dmin = h2f(k.h.x >> 16);
        uint32_t hv[4], lv[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint32_t h2[2], l2[2];
#pragma unroll
            for (int u = 0; u < 2; u++) {
                uint32_t sc, mm;
                q4k_scale_min(k.h.y, k.h.z, k.h.w, 2 * i + u, sc, mm);
                const float v = -dmin * (float)mm;
                h2[u] = bf16_bits(v);
                l2[u] = bf16_bits(v - bf16_to_f32(h2[u]));
            }
            hv[i] = h2[0] | (h2[1] << 16);
            lv[i] = l2[0] | (l2[1] << 16);
        }
        hi = __builtin_bit_cast(bf16x8, u32x4{hv[0], hv[1], hv[2], hv[3]});
        lo = __builtin_bit_cast(bf16x8, u32x4{lv[0], lv[1], lv[2], lv[3]});
    }
};

// Q6_K: step p = 48-byte chunk p (n2 = p/2, isub = p%2); lane half h takes
// positions 8h .. 8h + 7 of the 4 quadrants; MFMA kk = quadrant kk:
// element 128 n2 + 16 isub + 32 kk + 8 h + i.
struct SkQ6K {
    // exact operands: the codes q - 32 as f16; MFMA kk of step p covers one
    // 16-element sub-block, whose product is scaled by its own d * sc in f32
    // (KIND 4)
    static constexpr int KIND = 4, RB = 192;
    struct Blk {
        u32x4 sc;  // the 16 i8 scales
        uint32_t d;
    };
    const uint2 *qb8;  // 192-byte chunk streams as 8-byte units
    const uint4 *sc16;
    const uint16_t *dd;
    int nblk;
    __host__ __device__ SkQ6K shifted(int64_t nb) const {
        return {qb8 + nb * 24, sc16 + nb, dd + nb, nblk};
    }
    __device__ static int a_off(int p, int kk, int h) {
        return 128 * (p >> 1) + 16 * (p & 1) + 32 * kk + 8 * h;
    }
    __device__ const uint8_t *raw(int64_t row, int b) const {
        return reinterpret_cast<const uint8_t *>(qb8 + (row * nblk + b) * 24);
    }
    __device__ Blk load_blk(int64_t row, int b) const {
        return {ldv(sc16 + row * nblk + b), dd[row * nblk + b]};
    }
    __device__ static float2 scale(const Blk &k) { return make_float2(h2f(k.d), 0.f); }
    // d * sc of the sub-block MFMA kk of step p covers (dequant_q6_k's
    // d * sc * (q - 32), crates/arf-core/src/model/gguf.rs:2092-2131, with the
    // product d * sc formed first as there)
    __device__ static float sub_scale(const Blk &k, int p, int kk) {
        const int si = 8 * (p >> 1) + (p & 1) + 2 * kk;
        const uint32_t scw[4] = {k.sc.x, k.sc.y, k.sc.z, k.sc.w};
        return h2f(k.d) * (float)(int8_t)(scw[si >> 2] >> (8 * (si & 3)));
    }
    // The codes q (0..63) of positions 4j .. 4j + 3 of quadrant t, one per byte:
    // the ql nibble (ql_b for odd t, the high nibble for t >= 2) and qh bits
    // 2t, 2t + 1 as bits 4, 5.  Bits a shift carries into a neighbouring byte
    // land outside that byte's mask.
    __device__ static uint32_t codes(const u32x2 &qa, const u32x2 &qb, const u32x2 &qh, int t, int j) {
        const uint32_t l = (t & 1) ? qb[j] : qa[j];
        const uint32_t lo = (t & 2) ? l >> 4 : l;
        const uint32_t hi = t == 0 ? qh[j] << 4 : t == 1 ? qh[j] << 2 : t == 2 ? qh[j] : qh[j] >> 2;
        return (lo & 0x0F0F0F0Fu) | (hi & 0x30303030u);
    }
    // q - 32: v_perm puts two code bytes under 0x64 (the f16 1024 + q), less
    // 1056, exact
    __device__ static void frag(const uint8_t *srow, const Blk &, int p, int h, half8 f[4]) {
        const uint8_t *ch = srow + 48 * p;  // ql_a[16] | ql_b[16] | qh[16]
        const u32x2 qa = *reinterpret_cast<const u32x2 *>(ch + 8 * h);
        const u32x2 qb = *reinterpret_cast<const u32x2 *>(ch + 16 + 8 * h);
        const u32x2 qh = *reinterpret_cast<const u32x2 *>(ch + 32 + 8 * h);
        const half2v m1056 = h2splat(-1056.f);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            uint32_t o[4];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const uint32_t q = codes(qa, qb, qh, t, j);
                o[2 * j] = as_u(as_h2(__builtin_amdgcn_perm(0x64646464u, q, 0x04010400u)) + m1056);
                o[2 * j + 1] = as_u(as_h2(__builtin_amdgcn_perm(0x64646464u, q, 0x04030402u)) + m1056);
            }
            f[t] = u4_to_h8(o[0], o[1], o[2], o[3]);
        }
    }
    __device__ static void minsb(const Blk &, bf16x8 &hi, bf16x8 &lo) {
        hi = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
        lo = hi;
    }
};

// Q6_K with every sub-block scale in [-62, 62] (the upload's flag; the
// synthetic and many GGUF tensors): exact integer operands sc * (q - 32) / 2
// (|.| <= 992, a multiple of 1/2: exact in f16) in units of d, so the whole
// block accumulates in one set of registers and is scaled by 2d at the block
// end (KIND 1) instead of by d * sc after every MFMA.  One packed FMA per two
// weights: (1024 + q) * (sc / 2) - 528 sc, whose constant is an f16 value while
// |sc| <= 62 (33 * 63 needs 12 bits).  Same slab layout and step map as SkQ6K.
struct SkQ6KI : SkQ6K {
    static constexpr int KIND = 1;
    __host__ __device__ SkQ6KI shifted(int64_t nb) const { return {SkQ6K::shifted(nb)}; }
    __device__ static float2 scale(const Blk &k) { return make_float2(2.f * h2f(k.d), 0.f); }
    __device__ static void frag(const uint8_t *srow, const Blk &k, int p, int h, half8 f[4]) {
        const uint8_t *ch = srow + 48 * p;
        const u32x2 qa = *reinterpret_cast<const u32x2 *>(ch + 8 * h);
        const u32x2 qb = *reinterpret_cast<const u32x2 *>(ch + 16 + 8 * h);
        const u32x2 qh = *reinterpret_cast<const u32x2 *>(ch + 32 + 8 * h);
        // scale bytes as sc + 128 (unsigned)
        const uint32_t scw[4] = {k.sc.x ^ 0x80808080u, k.sc.y ^ 0x80808080u, k.sc.z ^ 0x80808080u,
                                 k.sc.w ^ 0x80808080u};
        const half2v half = h2splat(0.5f), m576 = h2splat(-576.f), m1056 = h2splat(-1056.f);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int si = 8 * (p >> 1) + (p & 1) + 2 * t;  // the sub-block of MFMA t
            // the f16 1152 + sc in both halves; * 1/2 - 576 = sc / 2, exact
            const uint32_t sel = 0x04000400u | (uint32_t)(si & 3) * 0x00010001u;
            const half2v s = as_h2(pk_fma(__builtin_amdgcn_perm(0x64646464u, scw[si >> 2], sel), half, m576));
            const half2v c = s * m1056;  // -528 sc
            uint32_t o[4];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const uint32_t q = codes(qa, qb, qh, t, j);
                o[2 * j] = pk_fma(__builtin_amdgcn_perm(0x64646464u, q, 0x04010400u), s, c);
                o[2 * j + 1] = pk_fma(__builtin_amdgcn_perm(0x64646464u, q, 0x04030402u), s, c);
            }
            f[t] = u4_to_h8(o[0], o[1], o[2], o[3]);
        }
    }
};

// Q8_0: step p of 256-element block b = Q8_0 blocks 8b + 2p (h = 0) and
// 8b + 2p + 1 (h = 1); MFMA kk = bytes 8kk .. 8kk + 7 of the lane's block.
// Weights d * q rounded to f16 (the format's scale is per 32 weights).
struct SkQ80 {
    // exact operands: the int8 codes as f16; MFMAs 0, 1 of step p cover Q8_0
    // block 2p, MFMAs 2, 3 block 2p + 1, and each block's product is scaled by
    // its own d in f32 (KIND 3, as IQ4_XS)
    static constexpr int KIND = 3, RB = 256;
    struct Blk {
        u32x4 d;  // the 8 f16 scales of the 8 Q8_0 blocks
    };
    const uint4 *qs;
    const uint16_t *dd;
    int nblk;  // Q8_0 blocks per row
    __host__ __device__ SkQ80 shifted(int64_t nb) const { return {qs + nb * 2, dd + nb, nblk}; }
    __device__ static int a_off(int p, int kk, int h) { return 64 * p + 32 * (kk >> 1) + 16 * (kk & 1) + 8 * h; }
    __device__ const uint8_t *raw(int64_t row, int b) const {
        return reinterpret_cast<const uint8_t *>(qs + (row * nblk + 8 * b) * 2);
    }
    __device__ Blk load_blk(int64_t row, int b) const {
        return {*reinterpret_cast<const u32x4 *>(dd + row * nblk + 8 * b)};
    }
    // d of Q8_0 blocks 2p and 2p + 1
    __device__ static float2 sub_scales(const Blk &k, int p) {
        const uint32_t dw = k.d[p];
        return make_float2(h2f(dw), h2f(dw >> 16));
    }
    __device__ static void frag(const uint8_t *srow, const Blk &, int p, int h, half8 f[4]) {
        // byte q ^ 0x80 = q + 128 under the f16 pattern of 1024 is 1152 + q,
        // less 1152: q exactly
        const half2v one = h2splat(1.f), m1152 = h2splat(-1152.f);
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            const u32x2 c = *reinterpret_cast<const u32x2 *>(srow + a_off(p, kk, h));
            uint32_t o[4];
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const uint32_t v = c[u] ^ 0x80808080u;
                o[2 * u] = pk_fma(__builtin_amdgcn_perm(0x64646464u, v, 0x04010400u), one, m1152);
                o[2 * u + 1] = pk_fma(__builtin_amdgcn_perm(0x64646464u, v, 0x04030402u), one, m1152);
            }
            f[kk] = u4_to_h8(o[0], o[1], o[2], o[3]);
        }
    }
    __device__ static float2 scale(const Blk &) { return make_float2(1.f, 0.f); }
    __device__ static void minsb(const Blk &, bf16x8 &hi, bf16x8 &lo) {
        hi = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
        lo = hi;
    }
};

// Q5_K: Q4_K's step map, header, scales and min term; the slab row is ggml's
// qh[32] | qs[128].  Element e of sub-block s = 2p + h is the low (h = 0) or
// high (h = 1) nibble of qs[32p + e] plus bit s of qh[e] as bit 4 (0..31), so
// the B operand sc_j * q <= 63 * 31 is an exact f16 integer.
// (dequant_q5_k, crates/arf-core/src/model/gguf.rs:2053-2090)
struct SkQ5K {
    static constexpr int KIND = 2, RB = 160;
    using Blk = SkQ4K::Blk;
    const uint4 *hdr;
    const uint8_t *q;
    int nblk;
    __host__ __device__ SkQ5K shifted(int64_t nb) const { return {hdr + nb, q + nb * 160, nblk}; }
    __device__ static int a_off(int p, int kk, int h) { return 64 * p + 32 * h + 8 * kk; }
    __device__ const uint8_t *raw(int64_t row, int b) const { return q + (row * nblk + b) * 160; }
    __device__ Blk load_blk(int64_t row, int b) const { return {ldv(hdr + row * nblk + b)}; }
    __device__ static float2 scale(const Blk &k) { return SkQ4K::scale(k); }
    __device__ static void frag(const uint8_t *srow, const Blk &k, int p, int h, half8 f[4]) {
        const u32x4 q0 = *reinterpret_cast<const u32x4 *>(srow + 32 + 32 * p);
        const u32x4 q1 = *reinterpret_cast<const u32x4 *>(srow + 48 + 32 * p);
        const u32x4 h0 = *reinterpret_cast<const u32x4 *>(srow);
        const u32x4 h1 = *reinterpret_cast<const u32x4 *>(srow + 16);
        const int s = 2 * p + h;
        uint32_t sc, mm;
        q4k_scale_min(k.h.y, k.h.z, k.h.w, s, sc, mm);
        const float scf = (float)sc;
        // (1024 + q) * sc - 1024 sc: one fused rounding of the exact q * sc
        const half2v s1 = h2splat(scf), c1 = h2splat(-1024.f * scf);
        const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        const uint32_t hw[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            uint32_t o[4];
#pragma unroll
            for (int u = 0; u < 2; u++) {
                // elements 8kk + 4u + 0..3 of the sub-block, one per byte
                const uint32_t v = ((qw[2 * kk + u] >> (4 * h)) & 0x0F0F0F0Fu) | bit_to4(hw[2 * kk + u], s);
                o[2 * u] = pk_fma(__builtin_amdgcn_perm(0x64646464u, v, 0x04010400u), s1, c1);
                o[2 * u + 1] = pk_fma(__builtin_amdgcn_perm(0x64646464u, v, 0x04030402u), s1, c1);
            }
            f[kk] = u4_to_h8(o[0], o[1], o[2], o[3]);
        }
    }
    __device__ static void minsb(const Blk &k, bf16x8 &hi, bf16x8 &lo) { SkQ4K::minsb(k, hi, lo); }
};

// IQ4_XS (KIND 3: exact codes, a scale per sub-block): step p = sub-blocks
// 2p (MFMAs kk = 0, 1) and 2p + 1 (kk = 2, 3), so each MFMA stays inside one
// sub-block and its f32 result is scaled by d * (ls - 32) of that sub-block
// (ls - 32 times a code can pass 2048, where f16 integers stop being exact).
// The slab row is qs[128], sub-block s in bytes 16s .. 16s + 15 (elements
// 0..15 the low nibbles, 16..31 the high ones); MFMA kk, lane half h takes
// element 16 (kk & 1) + 8h + i of its sub-block: nibble (kk & 1) of byte 8h + i.
// The B operand is the codebook value kv (exact in f16).
// (dequant_iq4_xs, crates/arf-core/src/model/gguf.rs:1937-1976)
struct SkIQ4XS {
    static constexpr int KIND = 3, RB = 128;
    struct Blk {
        u32x2 h;  // d | scales_h << 16, scales_l
    };
    const uint2 *hdr;
    const uint4 *qs;
    int nblk;
    __host__ __device__ SkIQ4XS shifted(int64_t nb) const { return {hdr + nb, qs + nb * 8, nblk}; }
    __device__ static int a_off(int p, int kk, int h) { return 64 * p + 32 * (kk >> 1) + 16 * (kk & 1) + 8 * h; }
    __device__ const uint8_t *raw(int64_t row, int b) const {
        return reinterpret_cast<const uint8_t *>(qs + (row * nblk + b) * 8);
    }
    __device__ Blk load_blk(int64_t row, int b) const { return {ldv(hdr + row * nblk + b)}; }
    // d * (ls - 32) of sub-blocks 2p and 2p + 1
    __device__ static float2 sub_scales(const Blk &k, int p) {
        const float d = h2f(k.h.x);
        float r[2];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int s = 2 * p + u;
            const int ls = (int)(((k.h.y >> (8 * p + 4 * u)) & 0xFu) | (((k.h.x >> (16 + 2 * s)) & 3u) << 4));
            r[u] = d * (float)(ls - 32);
        }
        return make_float2(r[0], r[1]);
    }
    __device__ static void frag(const uint8_t *srow, const Blk &, int p, int h, half8 f[4]) {
        // kvalues_iq4nl + 128 as bytes: entries 0..7 and 8..15, little-endian
        constexpr uint32_t T0lo = 0xBFAD9881u ^ 0x80808080u, T0hi = 0xF6EADDCFu ^ 0x80808080u;
        constexpr uint32_t T1lo = 0x26190D01u ^ 0x80808080u, T1hi = 0x71594535u ^ 0x80808080u;
        const half2v one = h2splat(1.f), m1152 = h2splat(-1152.f);
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const u32x2 c = *reinterpret_cast<const u32x2 *>(srow + 16 * (2 * p + u) + 8 * h);
#pragma unroll
            for (int nib = 0; nib < 2; nib++) {
                uint32_t o[4];
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const uint32_t sel = (c[j] >> (4 * nib)) & 0x0F0F0F0Fu;
                    const uint32_t s7 = sel & 0x07070707u;
                    const uint32_t v0 = __builtin_amdgcn_perm(T0hi, T0lo, s7);
                    const uint32_t v1 = __builtin_amdgcn_perm(T1hi, T1lo, s7);
                    // a byte-mask blend: iq4nl_lookup's third v_perm measured 25.5 -> 25.9 us
                    // at m = 8 here
                    const uint32_t hi = (sel >> 3) & 0x01010101u;
                    const uint32_t mask = (hi << 8) - hi;  // 0xFF in the bytes whose code is >= 8
                    const uint32_t v = (v1 & mask) | (v0 & ~mask);
                    // (1024 + kv + 128) - 1152 = kv, exact
                    o[2 * j] = pk_fma(__builtin_amdgcn_perm(0x64646464u, v, 0x04010400u), one, m1152);
                    o[2 * j + 1] = pk_fma(__builtin_amdgcn_perm(0x64646464u, v, 0x04030402u), one, m1152);
                }
                f[2 * u + nib] = u4_to_h8(o[0], o[1], o[2], o[3]);
            }
        }
    }
    __device__ static float2 scale(const Blk &) { return make_float2(1.f, 0.f); }
    __device__ static void minsb(const Blk &, bf16x8 &hi, bf16x8 &lo) {
        hi = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
        lo = hi;
    }
};

// ---- the loop -------------------------------------------------------------------
// x staging: XR = 32 TA rows x 256 k per block = XR * 32 chunks of 16 B over
// the NT threads; thread tid stages chunks c = tid + NT i (row c / 32 =
// (tid >> 5) + (NT / 32) i, k 8 * (tid & 31)) and, for KIND 2, 16 B of the
// sums of row min(tid >> 1, XR - 1).
template <int TA, int NT = SK_THREADS>
struct SkRows {
    static constexpr int XC = 32 * TA * 32 / NT;  // chunks per thread
    int64_t x[XC];  // element offset (row * K) of row (tid >> 5) + (NT / 32) i
    int64_t s;      // element offset (row * K / 16) of row min(tid >> 1, XR - 1)
};

// LDS of the loop: XB buffers of the x block of XR rows (+ its sub-block sums)
// and one weight slab [32][RB + 16] per wave and weight.
template <class F, int TA, int NW, int NT = SK_THREADS, int XB = 1>
constexpr size_t sk_lds() {
    return (size_t)XB * (32 * TA * SK_XLD * 2 + 32 * TA * 32) + (size_t)(NT / 64) * NW * 32 * (F::RB + 16);
}

// The MFMAs of one 256-element block: the wave's NW x 32 weight rows (slab
// rows 32 w + lr, scales wbk; lr = lane % 32, h = lane / 32, as the caller
// has them) against the x tiles t < TU, whose row 32 t + lr of this block
// starts at xrow(t) (LDS, the k order of
// F::a_off) and, for KIND 2, whose sub-block sums (bf16 hi[8] | lo[8]) start
// at srow(t); then the block end of KIND 1 / 2 (the min term's two MFMAs
// into acc, then acc += d * cb).  cb and cq are the block's own accumulators.
// (GM, MERGE, PIN:
// as skinny_loop.)
template <class F, int TA, int TU, int NW, int GM, bool MERGE, bool PIN, class XRow, class SRow>
__device__ __forceinline__ void sk_block(const uint8_t *slab, const typename F::Blk (&wbk)[NW], XRow xrow,
                                         SRow srow, int lr, int h, floatx16 (&acc)[NW][TA], floatx16 (&cb)[NW][TA],
                                         floatx16 (&cq)[NW][F::KIND == 3 ? TA : 1]) {
    constexpr int KIND = F::KIND;
    constexpr int TO = MERGE ? TU / 2 : TU;  // accumulator tiles written
    constexpr int SL = F::RB + 16;           // slab row stride (bytes)
#pragma unroll
    for (int p = 0; p < 4; p++) {
        if constexpr (PIN && TO == 2) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int w = 0; w < NW; w++) {
            half8 bf[4];
            F::frag(slab + (w * 32 + lr) * SL, wbk[w], p, h, bf);
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                if constexpr (KIND == 4) {
                    // one sub-block per MFMA (both x tiles with MERGE), times its d * sc
                    floatx16 c[TO], z;
#pragma unroll
                    for (int i = 0; i < 16; i++) z[i] = 0.f;
#pragma unroll
                    for (int t = 0; t < TU; t++) {
                        const half8 af = *reinterpret_cast<const half8 *>(xrow(t) + F::a_off(p, kk, h));
                        const int ti = MERGE ? t % TO : t;
                        c[ti] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf[kk], MERGE && t >= TO ? c[ti] : z,
                                                                       0, 0, 0);
                    }
                    const float ss = F::sub_scale(wbk[w], p, kk);
#pragma unroll
                    for (int ti = 0; ti < TO; ti++)
#pragma unroll
                        for (int i = 0; i < 16; i++)
                            if ((GM >> (4 * ti + (i >> 2))) & 1) acc[w][ti][i] = fmaf(ss, c[ti][i], acc[w][ti][i]);
                } else {
#pragma unroll
                    for (int t = 0; t < TU; t++) {
                        const half8 af = *reinterpret_cast<const half8 *>(xrow(t) + F::a_off(p, kk, h));
                        const int ti = MERGE ? t % TO : t;
                        const bool cont = MERGE && t >= TO;  // a lo tile adds onto its hi tile's chain
                        floatx16 z;
#pragma unroll
                        for (int i = 0; i < 16; i++) z[i] = 0.f;
                        if constexpr (KIND == 3) {
                            floatx16 &c = kk < 2 ? cb[w][ti] : cq[w][ti];
                            c = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf[kk], kk % 2 == 0 && !cont ? z : c,
                                                                       0, 0, 0);
                        } else if constexpr (KIND != 0) {
                            cb[w][ti] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                                af, bf[kk], p == 0 && kk == 0 && !cont ? z : cb[w][ti], 0, 0, 0);
                        } else {
                            acc[w][ti] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf[kk], acc[w][ti], 0, 0, 0);
                        }
                    }
                }
            }
            if constexpr (KIND == 3) {
                // the step's two sub-blocks, each times its own d * (ls - 32)
                const float2 ss = F::sub_scales(wbk[w], p);
#pragma unroll
                for (int ti = 0; ti < TO; ti++)
#pragma unroll
                    for (int i = 0; i < 16; i++)
                        acc[w][ti][i] = fmaf(ss.y, cq[w][ti][i], fmaf(ss.x, cb[w][ti][i], acc[w][ti][i]));
            }
        }
    }
    if constexpr (KIND == 1 || KIND == 2) {
        // block end: the min term (two bf16 MFMAs, in true units) onto acc,
        // then acc += d * C_block.  (Kept in registers of its own, the min
        // term took 24-32 more VGPRs: the MoE gate|up 250 -> 226, the x-
        // stationary down 198 -> 166, and no spill in Q5_K's down; the times
        // did not move.)
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float2 dd = F::scale(wbk[w]);
            if constexpr (KIND == 2) {
                bf16x8 bh, bl;
                F::minsb(wbk[w], bh, bl);
#pragma unroll
                for (int t = 0; t < TU; t++) {
                    const bf16x8 am = *reinterpret_cast<const bf16x8 *>(srow(t) + 8 * h);
                    const int ti = MERGE ? t % TO : t;
                    acc[w][ti] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(am, bh, acc[w][ti], 0, 0, 0);
                    acc[w][ti] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(am, bl, acc[w][ti], 0, 0, 0);
                }
            }
#pragma unroll
            for (int ti = 0; ti < TO; ti++)
#pragma unroll
                for (int i = 0; i < 16; i++) acc[w][ti][i] = fmaf(dd.x, cb[w][ti][i], acc[w][ti][i]);
        }
    }
}

// Accumulates acc[w][t] (w < NW weights, t < TA 32-row x tiles) over the
// 256-element blocks [b0, b1) for the wave's 32 weight rows wrow0[w] ..
// wrow0[w] + 31 (rows past nrows are clamped: computed, never to be stored).
// The block loop of skinny_run for the first TU (<= TA) x tiles.
// GM: the 8-row accumulator groups (bit 4 t + g: rows 32 t + 8 g .. + 7) that
// hold real rows; KIND 4 scales only those (the others stay 0).  MERGE: the
// second half of the x tiles (TU / 2 .. TU - 1) holds the low halves of the
// first half's rows (f32 x as f16 hi + lo), so tile t's products go into tile
// t % (TU / 2)'s accumulators (the second half of acc is left as it is).  PIN:
// with two accumulator tiles, hold the scheduler to one step's operands at a
// time (left free, it hoists all four steps' operand builds and x reads; the
// dense skinny GEMM at C3 m = 64 ran 57.6 -> 53.0 us with the step boundary
// held, the MoE tiles 1 % slower).  XB = 2: two x buffers; the next block's x
// goes into the one not being read, which leaves one barrier per block
// instead of two, for a second x buffer of LDS.  XP = 3: x is the caller's f32
// [m <= 8, K] and is split here (one 32-row tile, 256 threads): thread tid
// stages elements 8 (tid % 32) .. + 7 of row rows.x[0] (row tid / 32,
// clamped to m - 1) as the f16 parts of x * 2^xsh -- hi, mid = the rounded
// remainder, lo = the rounded remainder of that -- into tile rows r, 8 + r and
// 16 + r (r = tid / 32), where xsh (returned) puts the largest |x| of the
// row over blocks [b0, b1) in [2^14, 2^15), and for KIND 2 each part's
// sub-block sums (its lanes' 8 in order, then the quad's (s0 + s1) + (s2 + s3))
// as bf16 hi + lo: the arithmetic of xprep_kernel with three parts, without
// its launch.  Rows 24..31 of the tile stage nothing (their products land in
// rows never stored).  WNT: the weights are loaded non-temporal.
template <class F, int TA, int TU, int NW, int NT, class XT, int GM = 0xFF, bool MERGE = false,
          bool PIN = false, int XB = 1, int XP = 0, bool WNT = false>
__device__ __forceinline__ void skinny_loop(const F (&fmt)[NW], const int64_t (&wrow0)[NW],
                                            int64_t nrows, const SkRows<TA, NT> &rows,
                                            const XT *__restrict__ x,
                                            const uint16_t *__restrict__ xs, int b0, int b1,
                                            floatx16 (&acc)[NW][TA], _Float16 *lds, int &xsh) {
    constexpr int KIND = F::KIND;
    constexpr int XR = 32 * TA;       // x rows staged
    static_assert(!MERGE || TU % 2 == 0, "merged tiles come in (hi, lo) halves");
    constexpr int XC = SkRows<TA, NT>::XC;
    constexpr int RL = F::RB / 16;          // lanes per weight row in a coalesced load
    constexpr int NI = 32 * F::RB / 1024;   // 16-byte loads per lane per block
    constexpr int SL = F::RB + 16;          // slab row stride (bytes)
    const int tid = sk_tid(), lane = tid & 63, wave = tid >> 6;
    const int h = lane >> 5, lr = lane & 31;
    static_assert(XB == 1 || XB == 2, "one or two x buffers");
    _Float16 *xl = lds;                                                   // [XB][XR][SK_XLD]
    uint16_t *sl = reinterpret_cast<uint16_t *>(lds + XB * XR * SK_XLD);  // [XB][XR][16]
    uint8_t *slab = reinterpret_cast<uint8_t *>(sl + XB * XR * 16) + (size_t)wave * NW * 32 * SL;
    int xb = 0;  // the x buffer this block reads

    // x chunks of 8 elements: one 16-byte load of f16, two of f32 (rounded to
    // f16 when stored to LDS)
    constexpr int XW = sizeof(XT) / 2;
    static_assert(XW == 1 || XW == 2, "x is f16 or f32");
    static_assert(XP == 0 || (XP == 3 && XW == 2 && TA == 1 && TU == 1 && NT == 256),
                  "three parts formed here: f32 x, one tile of 256 threads");
    constexpr int XU = XP == 3 ? 1 : XC * TU / TA;  // chunks of the x rows in use
    u32x4 xv[XU * XW], sv;
    auto xload = [&](int b) {
#pragma unroll
        for (int i = 0; i < XU; i++)
#pragma unroll
            for (int j = 0; j < XW; j++)
                xv[XW * i + j] = *reinterpret_cast<const u32x4 *>(x + rows.x[i] + 256 * b +
                                                                  8 * (tid & 31) + 4 * j);
        // the sums' load sits in the same branch as their store: loaded
        // unconditionally, it was sunk next to the store, where its wait
        // covered every load in flight
        if constexpr (KIND == 2 && XP == 0) {
            if (tid < 64 * TU) sv = *reinterpret_cast<const u32x4 *>(xs + rows.s + 16 * b + 8 * (tid & 1));
        }
    };
    auto xstore = [&](int to) {
        if constexpr (XP == 3) {
            half8 hp[3];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float u = ldexpf(__uint_as_float(xv[i >> 2][i & 3]), xsh);
                hp[0][i] = (_Float16)u;
                const float r1 = u - (float)hp[0][i];  // exact
                hp[1][i] = (_Float16)r1;
                hp[2][i] = (_Float16)(r1 - (float)hp[1][i]);  // exact difference
            }
#pragma unroll
            for (int q = 0; q < 3; q++)
                *reinterpret_cast<half8 *>(xl + (to * XR + 8 * q + (tid >> 5)) * SK_XLD + 8 * (tid & 31)) = hp[q];
            if constexpr (KIND == 2) {
#pragma unroll
                for (int q = 0; q < 3; q++) {
                    float t = 0.f;
#pragma unroll
                    for (int i = 0; i < 8; i++) t += (float)hp[q][i];
                    // the quad of lanes holding the sub-block: (s0 + s1) + (s2 + s3) on each
                    t += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(t), 0xB1, 0xf, 0xf, true));
                    t += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(t), 0x4E, 0xf, 0xf, true));
                    if ((tid & 3) == 0) {
                        const uint32_t hi = bf16_bits(t);
                        uint16_t *d = sl + (to * XR + 8 * q + (tid >> 5)) * 16 + ((tid & 31) >> 2);
                        d[0] = (uint16_t)hi;
                        d[8] = (uint16_t)bf16_bits(t - bf16_to_f32(hi));
                    }
                }
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < XU; i++) {
            u32x4 v;
            if constexpr (XW == 1) {
                v = xv[i];
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const u32x4 &f = xv[2 * i + (j >> 1)];
                    v[j] = pack_f16x2(__uint_as_float(f[2 * (j & 1)]), __uint_as_float(f[2 * (j & 1) + 1]));
                }
            }
            *reinterpret_cast<u32x4 *>(xl + (to * XR + (tid >> 5) + (NT / 32) * i) * SK_XLD + 8 * (tid & 31)) = v;
        }
        if constexpr (KIND == 2) {
            if (tid < 64 * TU) *reinterpret_cast<u32x4 *>(sl + (to * XR + (tid >> 1)) * 16 + 8 * (tid & 1)) = sv;
        }
    };

    // weights: each wave loads its 32 rows x RB bytes of a block with NI
    // coalesced 16-byte loads per lane (flat chunk c = 64 i + lane: row c / RL,
    // bytes 16 (c % RL)), one block ahead of use.  With WNT the loads are
    // non-temporal: each weight byte is used once, so the L2 keeps the x rows
    // that every column tile re-reads instead (C3 m = 8 27.9 -> 27.2 us, C5
    // 160.8 -> 156.9 us with the MoE kernels; at m = 9..64 slower, m = 32
    // 36.2 -> 38.4 us, same box)
    u32x4 rv[NW][NI];
    typename F::Blk wb[NW], wbn[NW];
    auto wload = [&](int b) {
#pragma unroll
        for (int w = 0; w < NW; w++)
#pragma unroll
            for (int i = 0; i < NI; i++) {
                const int c = 64 * i + lane;
                const int64_t row = min(wrow0[w] + c / RL, nrows - 1);
                const u32x4 *p = reinterpret_cast<const u32x4 *>(fmt[w].raw(row, b) + 16 * (c % RL));
                if constexpr (WNT)
                    rv[w][i] = __builtin_nontemporal_load(p);
                else
                    rv[w][i] = *p;
            }
    };
    auto wstore = [&]() {
#pragma unroll
        for (int w = 0; w < NW; w++)
#pragma unroll
            for (int i = 0; i < NI; i++) {
                const int c = 64 * i + lane;
                *reinterpret_cast<u32x4 *>(slab + (w * 32 + c / RL) * SL + 16 * (c % RL)) = rv[w][i];
            }
    };
    int64_t myrow[NW];
#pragma unroll
    for (int w = 0; w < NW; w++) myrow[w] = min(wrow0[w] + lr, nrows - 1);

#pragma unroll
    for (int w = 0; w < NW; w++) wb[w] = fmt[w].load_blk(myrow[w], b0);
    wload(b0);
    if constexpr (XP == 3) {
        // the row's largest |x| over the K range, four blocks' loads in flight
        // (issued behind the first weights, whose arrival the prologue waits
        // for anyway)
        const XT *xr = x + rows.x[0] + 8 * (tid & 31);
        float amax = 0.f;
        for (int b = b0; b < b1; b += 4) {
            float4 t[4][2];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int bb = min(b + u, b1 - 1);
                t[u][0] = *reinterpret_cast<const float4 *>(xr + 256 * bb);
                t[u][1] = *reinterpret_cast<const float4 *>(xr + 256 * bb + 4);
            }
#pragma unroll
            for (int u = 0; u < 4; u++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(t[u][j].x), fabsf(t[u][j].y)),
                                             fmaxf(fabsf(t[u][j].z), fabsf(t[u][j].w))));
        }
#pragma unroll
        for (int o = 16; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));  // the row's 32 lanes
        xsh = amax > 0.f && amax < INFINITY ? 15 - __builtin_amdgcn_frexp_expf(amax) : 0;
    }
    xload(b0);
    xstore(0);
    __syncthreads();

    // KIND 3: cb holds the step's first sub-block (MFMAs 0, 1), cq its second
    floatx16 cb[NW][TA], cq[NW][KIND == 3 ? TA : 1];
    for (int b = b0; b < b1; b++) {
        const int bn = min(b + 1, b1 - 1);  // past the end: a re-read of the last block
        wstore();                            // block b's weights (loaded one block ago)
        // loads of the next block, in the order their data is waited for:
        // the scales and x at this block's end, the weights at the next
        // block's start (vector loads complete in order, so a weight load
        // issued first would hold up the x hand-off)
#pragma unroll
        for (int w = 0; w < NW; w++) wbn[w] = fmt[w].load_blk(myrow[w], bn);
        xload(bn);
        __builtin_amdgcn_sched_barrier(0);
        wload(bn);
        // keep the scheduler from sinking the loads: they must be in flight
        // during this block, not issued at its end
        __builtin_amdgcn_sched_barrier(0);
        sk_block<F, TA, TU, NW, GM, MERGE, PIN>(
            slab, wb, [&](int t) { return xl + (xb * XR + 32 * t + lr) * SK_XLD; },
            [&](int t) { return sl + (xb * XR + 32 * t + lr) * 16; }, lr, h, acc, cb, cq);
#pragma unroll
        for (int w = 0; w < NW; w++) wb[w] = wbn[w];
        if constexpr (XB == 2) {
            xstore(xb ^ 1);  // nobody reads that buffer: its block ended at the last barrier
            xb ^= 1;
            __syncthreads();
        } else {
            __syncthreads();  // every wave is done with this block's x
            xstore(0);
            __syncthreads();
        }
    }
}

// `rows` gives the x rows this thread stages; xrows (<= 32 TA) of them are
// real.  With TA = 2, xrows <= 32 and SHORT (tiles of varying height), the
// second x tile is neither staged nor multiplied (acc[w][1] is left as it
// is).  All threads of the workgroup call it with the same block range and
// xrows.
// (xsh: the x scale exponent of XP = 3; WNT: non-temporal weight loads)
template <class F, int TA, int NW, int NT = SK_THREADS, class XT = _Float16, bool SHORT = false, int GM = 0xFF,
          bool MERGE = false, bool PIN = false, int XB = 1, int XP = 0, bool WNT = false>
__device__ __forceinline__ void skinny_run(const F (&fmt)[NW], const int64_t (&wrow0)[NW],
                                           int64_t nrows, const SkRows<TA, NT> &rows,
                                           const XT *__restrict__ x,
                                           const uint16_t *__restrict__ xs, int b0, int b1,
                                           floatx16 (&acc)[NW][TA], _Float16 *lds, int xrows, int &xsh) {
    if constexpr (TA == 2 && SHORT) {
        if (xrows <= 32) {
            skinny_loop<F, TA, 1, NW, NT, XT, GM, false, false, XB, 0, WNT>(fmt, wrow0, nrows, rows, x, xs, b0, b1,
                                                                           acc, lds, xsh);
            return;
        }
    }
    skinny_loop<F, TA, TA, NW, NT, XT, GM, MERGE, PIN, XB, XP, WNT>(fmt, wrow0, nrows, rows, x, xs, b0, b1, acc,
                                                                   lds, xsh);
}
template <class F, int TA, int NW, int NT = SK_THREADS, class XT = _Float16, bool SHORT = false, int GM = 0xFF,
          bool MERGE = false, bool PIN = false, int XB = 1, int XP = 0, bool WNT = false>
__device__ __forceinline__ void skinny_run(const F (&fmt)[NW], const int64_t (&wrow0)[NW],
                                           int64_t nrows, const SkRows<TA, NT> &rows,
                                           const XT *__restrict__ x,
                                           const uint16_t *__restrict__ xs, int b0, int b1,
                                           floatx16 (&acc)[NW][TA], _Float16 *lds, int xrows) {
    int xsh = 0;
    skinny_run<F, TA, NW, NT, XT, SHORT, GM, MERGE, PIN, XB, XP, WNT>(fmt, wrow0, nrows, rows, x, xs, b0, b1, acc,
                                                                       lds, xrows, xsh);
}
// The rows of `rows` for a tile whose x row r (r < n) is row_of(r) of an
// [*, K] matrix.
template <int TA, int NT = SK_THREADS, class RowOf>
__device__ __forceinline__ SkRows<TA, NT> sk_rows(int n, int K, RowOf row_of) {
    SkRows<TA, NT> r;
    const int tid = sk_tid();
#pragma unroll
    for (int i = 0; i < SkRows<TA, NT>::XC; i++)
        r.x[i] = (int64_t)row_of(min((tid >> 5) + (NT / 32) * i, n - 1)) * K;
    r.s = (int64_t)row_of(min(tid >> 1, min(32 * TA, n) - 1)) * (K / 16);
    return r;
}

// Row of accumulator element i of x tile t for this lane (column = lane % 32).
__device__ __forceinline__ int sk_out_row(int t, int i) {
    const int lane = threadIdx.x & 63;
    return 32 * t + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
}

}  // namespace arfq
