// arfq_gemm_bd.h -- prefill GEMM with the weights going straight from memory
// into the MFMA B operands (no LDS for weights).  Q4_K is described here; the
// Bd* format policies below give Q5_K, Q6_K, Q8_0 and IQ4_XS the same tile.
//
// A workgroup of 8 waves computes 128 x rows by 512 weight rows; wave w owns
// the 64 weight rows [n0 + 64 w, n0 + 64 w + 64) for all 128 x rows, as 4 x 2
// tiles of v_mfma_f32_32x32x16_f16 with f32 accumulators.  Only the f16 x tile
// (and its sub-block sums) goes through LDS: one whole block (128 x 256
// halves, 16-byte row padding), double buffered, so the waves meet at one
// barrier per block and can drift apart within it; all eight waves read it,
// so each x tile is fetched once per 512 weight rows.  A step is 64 k (a
// quarter block).  In step p of block b, lane l serves weight row (l % 32) of
// each of its two 32-row groups and Q4_K sub-block j = 2 p + l / 32: one
// 16-byte load of that sub-block's codes per group gives the B operands of
// the step's 4 MFMA groups (group kk uses dword kk: block elements
// 64 p + 32 (l/32) + 8 kk .. + 7), and the A operands read the x tile with
// the same element map.  Code loads run two steps ahead.  The B operands
// are software-pipelined against the MFMAs: the g = 1 operand of a group is
// built between that group's four g = 0 MFMAs, and the next group's g = 0
// operand between its four g = 1 MFMAs (one MFMA, then three VALU, pinned with
// sched_group_barrier), so a wave's own dequant issues while its MFMAs run
// instead of in a burst after them (C4: 427 -> 414 us).
//
// The B operands are exact: sc_j * q (<= 63 * 15) as f16 integers, made from
// the code bits with v_perm (each nibble under the f16 bit pattern of 1024)
// and one packed f16 FMA per two weights (ggml get_scale_min_k4 for sc_j, m_j:
// crates/arf-ml/src/weight.rs:1353-1365).  The block scale d multiplies the
// whole block, so instead of a second set of accumulators the accumulators run
// in units of the current block's d: before block b they are multiplied by
// d_{b-1} / d_b, and after the last block by d_last (a block with d = 0 uses
// scale 1 and zero weights).  The min term -dmin_b * sum_j m_j * X_j (X_j:
// the x sub-block sums, bf16 hi + lo from xprep) goes in at the start of each
// block with two bf16 MFMAs per tile, its coefficients -dmin * m_j / d_b split
// into bf16 hi + lo.  So y = sum_b (d_b * sum sc*q*x - dmin_b * sum m*X), as
// the reference factorises it (crates/arf-ml/src/matmul.rs:327-358).
//
// Reference behaviour: matmul_mm_q4ks.metal:65-290 (dequantized Q4_K tiles,
// simdgroup MMA with f32 accumulation, half x tiles) and the arithmetic of
// matmul_nt_q4ks (crates/arf-ml/src/matmul.rs:322-400).
#pragma once
#include "arfq_gemm_tile.h"

namespace arfq {

constexpr int BD_BM = 128;         // x rows per workgroup (all waves)
constexpr int BD_WN = 64;          // weight rows per wave
constexpr int BD_NW = 8;           // waves per workgroup
constexpr int BD_BN = BD_NW * BD_WN;  // weight rows per workgroup
constexpr int BD_THREADS = 64 * BD_NW;
constexpr int BD_LD = 256 + 8;     // halves per LDS x row: one block, 16-byte pad

// LDS: x tiles [2][BD_BM][BD_LD] halves, then the x sub-block sums [2][BD_BM][16] bf16,
// then (formats with EXTRA block data) a dword per wave, group, MFMA kk and lane
constexpr size_t BD_EXTRA_DWORDS = (size_t)BD_NW * 2 * 4 * 64;
template <class F>
__host__ __device__ constexpr size_t bd_lds() {
    return (size_t)2 * BD_BM * BD_LD * sizeof(_Float16) + (size_t)2 * BD_BM * 16 * sizeof(uint16_t) +
           (F::EXTRA ? BD_EXTRA_DWORDS * 4 : 0);
}

// workgroup barrier for the x tile: this wave's LDS writes are complete, no
// wait on the (prefetching) global loads
__device__ __forceinline__ void bd_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

__device__ __forceinline__ half8 bd_h8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    return __builtin_bit_cast(half8, u32x4{a, b, c, d});
}

// sc * q of one code dword (8 nibbles of one sub-block, sigma order: byte i
// low nibble = element i, high nibble = element 4 + i), in element order:
// (1024 + q) * sc - 1024 sc and (1024 + 16 q) * (sc / 16) - 64 sc, exact
struct BdScale {
    half2v s1, c1, s16, c16;
};

__device__ __forceinline__ BdScale bd_scale(uint32_t sc) {
    const half2v s1 = h2splat((float)sc);  // sc <= 63: every product below is exact
    return {s1, s1 * (half2v){-1024.f, -1024.f}, s1 * (half2v){0.0625f, 0.0625f},
            s1 * (half2v){-64.f, -64.f}};
}

__device__ __forceinline__ half8 bd_dequant(uint32_t c, const BdScale &k) {
    const uint32_t t01 = __builtin_amdgcn_perm(0x64646464u, c, 0x04010400u);  // b0 64 b1 64
    const uint32_t t23 = __builtin_amdgcn_perm(0x64646464u, c, 0x04030402u);  // b2 64 b3 64
    return bd_h8(pk_fma(t01 & 0x640F640Fu, k.s1, k.c1), pk_fma(t23 & 0x640F640Fu, k.s1, k.c1),
                 pk_fma(t01 & 0x64F064F0u, k.s16, k.c16), pk_fma(t23 & 0x64F064F0u, k.s16, k.c16));
}

// The min-term B operands of one block: (-dmin * m_j / su) for j = 0..7 as
// bf16 hi and lo (every lane all 8, in j order).  Lane half h works out
// j = 4h .. 4h + 3 and v_permlane32_swap hands each half the other's four.
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void bd_mins(const u32x4 hd, float inv_su, int h, bf16x8 &hi, bf16x8 &lo) {
    const float f = -h2f(hd.x >> 16) * inv_su;
    // m_j bytes (ggml get_scale_min_k4): j < 4: scales[4 + j] & 63;
    // j >= 4: (scales[4 + j] >> 4) | ((scales[j] >> 6) << 4)
    const uint32_t mlo = hd.z & 0x3F3F3F3Fu;
    const uint32_t mhi = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
    const uint32_t mb = mlo ^ ((mlo ^ mhi) & (0u - (uint32_t)h));  // branch-free select
    float c[4];
#pragma unroll
    for (int i = 0; i < 4; i++) c[i] = f * (float)((mb >> (8 * i)) & 0xffu);
    uint32_t hv[2], lv[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const bf16x2v hb = {(__bf16)c[2 * i], (__bf16)c[2 * i + 1]};
        const bf16x2v lb = {(__bf16)(c[2 * i] - (float)hb[0]), (__bf16)(c[2 * i + 1] - (float)hb[1])};
        hv[i] = __builtin_bit_cast(uint32_t, hb);
        lv[i] = __builtin_bit_cast(uint32_t, lb);
    }
    // after the swap, .x of every lane holds lane half 0's dword and .y half 1's
    const auto h0 = __builtin_amdgcn_permlane32_swap(hv[0], hv[0], false, false);
    const auto h1 = __builtin_amdgcn_permlane32_swap(hv[1], hv[1], false, false);
    const auto l0 = __builtin_amdgcn_permlane32_swap(lv[0], lv[0], false, false);
    const auto l1 = __builtin_amdgcn_permlane32_swap(lv[1], lv[1], false, false);
    hi = __builtin_bit_cast(bf16x8, u32x4{h0[0], h1[0], h0[1], h1[1]});
    lo = __builtin_bit_cast(bf16x8, u32x4{l0[0], l1[0], l0[1], l1[1]});
}

// ---- formats ------------------------------------------------------------------
// A direct-operand format gives, per lane, the codes of one step (its weight
// row's 32 elements of that step, loaded straight into registers) and, per
// block, the row's header; from those it builds the step's B operands in units
// of the block scale su (UNITS: su = the block's d, so the accumulators are
// moved into each block's unit; otherwise su = 1 and the operands carry their
// whole scale).  MIN: the Q4_K min term (x sub-block sums).  STEP_KK: a
// scale per group, not per step.  LATE: every group reads the block data
// (Blk), so the next block's replaces it only after group 15.  EXTRA: block
// data loaded at group 9 for the next block (LATE formats).  XPERM: the x
// tile is staged in the format's slot order.  VPM: VALU slots
// per MFMA in the pinned schedule (about a quarter of one operand's build).
// a_off(p, kk, h): the block elements a lane's 8 k-slots of MFMA group kk of
// step p hold (the x tile is read with the same map).
// Buffer loads: per-lane 32-bit offsets fixed for the work item plus a
// uniform (SGPR) offset per block and step; the launcher keeps every stream
// below 2 GiB.

// Q4_K (exact): step p, lane half h = sub-block 2p + h; group kk = code dword
// kk (elements 8kk .. 8kk + 7, sigma nibble order).  Operands sc_j * q.
struct BdQ4K {
    static constexpr int XPARTS = 2;
    static constexpr bool EXTRA = false;
    struct Extra {};
    static constexpr bool XPERM = false, LATE = false;
    static constexpr bool UNITS = true, MIN = true, STEP_KK = false, WLO = false;
    static constexpr int VPM = 3;
    using Code = u32x4;
    using Head = u32x4;
    using Blk = uint32_t;  // sc of sub-blocks 2p + h, byte p
    using Step = BdScale;
    const uint4 *hdr, *qs;
    __device__ static int a_off(int p, int kk, int h) { return 64 * p + 32 * h + 8 * kk; }
    struct Lanes {
        __amdgpu_buffer_rsrc_t q, hd;
        uint32_t qv[2], hv[2];
        __device__ Code code(int g, int st) const {
            return __builtin_amdgcn_raw_buffer_load_b128(q, qv[g], (st >> 2) * 128 + 32 * (st & 3), 0);
        }
        __device__ Head head(int g, int blk) const {
            return __builtin_amdgcn_raw_buffer_load_b128(hd, hv[g], blk * 16, 0);
        }
    };
    __device__ Lanes lanes(int n, int nblk, uint32_t wr0, uint32_t wr1, int h) const {
        Lanes l;
        l.q = __builtin_amdgcn_make_buffer_rsrc((void *)qs, (short)0, (int)((uint32_t)n * nblk * 128), 0x00020000);
        l.hd = __builtin_amdgcn_make_buffer_rsrc((void *)hdr, (short)0, (int)((uint32_t)n * nblk * 16), 0x00020000);
        l.qv[0] = wr0 * nblk * 128 + 16 * h;
        l.qv[1] = wr1 * nblk * 128 + 16 * h;
        l.hv[0] = wr0 * nblk * 16;
        l.hv[1] = wr1 * nblk * 16;
        return l;
    }
    __device__ static float unit(const Head &hd) { return h2f(hd.x); }
    __device__ static Blk block(const Head &hd, const Extra &, int h, uint32_t *) {
        uint32_t packed = 0;
#pragma unroll
        for (int p = 0; p < 4; p++) {
            uint32_t sc, mm;
            q4k_scale_min(hd.y, hd.z, hd.w, 2 * p + h, sc, mm);
            packed |= sc << (8 * p);
        }
        return packed;
    }
    __device__ static void kill(Blk &b) { b = 0u; }
    __device__ static Step step(Blk b, int p, int) { return bd_scale((b >> (8 * p)) & 0xffu); }
    __device__ static half8 deq(const Code &c, const Step &k, Blk, int, int kk) {
        return bd_dequant(kk == 0 ? c.x : kk == 1 ? c.y : kk == 2 ? c.z : c.w, k);
    }
    __device__ static void mins(const Head &hd, float inv_su, int h, bf16x8 &hi, bf16x8 &lo) {
        bd_mins(hd, inv_su, h, hi, lo);
    }
};

// Q5_K (exact): ggml's qs pairs sub-blocks 2p (low nibbles) and 2p + 1 (high
// nibbles) byte by byte, so step p, lane half h takes elements 16h .. 16h + 15
// of both: 16 code bytes, and group kk = elements 16h + 4kk .. + 3 of each
// (slots 0..3 sub-block 2p, 4..7 sub-block 2p + 1; the x tile is staged in
// that slot order, XPERM).  The fifth bit of element l of sub-block j is bit j
// of qh[l]: the lane's 16 qh bytes come with the block header.  Operands
// sc_j * q (<= 63 * 31, exact) as Q4_K's, with the fifth bit put into the
// f16 pattern (bit 4 of 1024 + q, bit 8 of 1024 + 16 q).  Same header and
// min term as Q4_K.  (dequant_q5_k, crates/arf-core/src/model/gguf.rs:2053-2090)
struct BdQ5K {
    static constexpr int XPARTS = 4;
    static constexpr bool EXTRA = true;  // the qh bytes come separately, late
    static constexpr bool XPERM = true, LATE = true;
    static constexpr bool UNITS = true, MIN = true, STEP_KK = false, WLO = false;
    static constexpr int VPM = 5;
    using Code = u32x4;
    using Head = u32x4;
    using Extra = u32x4;  // the lane's 16 qh bytes
    struct Blk {
        uint32_t lo, hi;     // sc of sub-blocks 2p, 2p + 1, byte p
        const uint32_t *qh;  // the lane's qh dword of MFMA kk at qh[64 kk] (LDS)
    };
    using Step = BdScale;
    const uint4 *hdr;
    const uint8_t *q;  // qh[32] | qs[128] per block
    __device__ static int a_off(int p, int kk, int h) { return 64 * p + 32 * h + 8 * kk; }
    struct Lanes {
        __amdgpu_buffer_rsrc_t q, hd;
        uint32_t qv[2], hv[2];
        __device__ Code code(int g, int st) const {
            return __builtin_amdgcn_raw_buffer_load_b128(q, qv[g], (st >> 2) * 160 + 32 + 32 * (st & 3), 0);
        }
        __device__ Head head(int g, int blk) const {
            return __builtin_amdgcn_raw_buffer_load_b128(hd, hv[g], blk * 16, 0);
        }
        __device__ Extra extra(int g, int blk) const {
            return __builtin_amdgcn_raw_buffer_load_b128(q, qv[g], blk * 160, 0);
        }
    };
    __device__ Lanes lanes(int n, int nblk, uint32_t wr0, uint32_t wr1, int h) const {
        Lanes l;
        l.q = __builtin_amdgcn_make_buffer_rsrc((void *)q, (short)0, (int)((uint32_t)n * nblk * 160), 0x00020000);
        l.hd = __builtin_amdgcn_make_buffer_rsrc((void *)hdr, (short)0, (int)((uint32_t)n * nblk * 16), 0x00020000);
        l.qv[0] = wr0 * nblk * 160 + 16 * h;
        l.qv[1] = wr1 * nblk * 160 + 16 * h;
        l.hv[0] = wr0 * nblk * 16;
        l.hv[1] = wr1 * nblk * 16;
        return l;
    }
    __device__ static float unit(const Head &hd) { return h2f(hd.x); }
    __device__ static Blk block(const Head &hd, const Extra &qh, int, uint32_t *xl) {
        xl[0] = qh.x;
        xl[64] = qh.y;
        xl[128] = qh.z;
        xl[192] = qh.w;
        Blk b{0u, 0u, xl};
#pragma unroll
        for (int p = 0; p < 4; p++) {
            uint32_t sc, mm;
            q4k_scale_min(hd.y, hd.z, hd.w, 2 * p, sc, mm);
            b.lo |= sc << (8 * p);
            q4k_scale_min(hd.y, hd.z, hd.w, 2 * p + 1, sc, mm);
            b.hi |= sc << (8 * p);
        }
        return b;
    }
    __device__ static void kill(Blk &b) { b.lo = b.hi = 0u; }
    __device__ static Step step(const Blk &b, int p, int) {
        const half2v s1 = h2splat((float)((b.lo >> (8 * p)) & 0xffu));
        const half2v s2 = h2splat((float)((b.hi >> (8 * p)) & 0xffu));
        return {s1, s1 * (half2v){-1024.f, -1024.f}, s2 * (half2v){0.0625f, 0.0625f}, s2 * (half2v){-64.f, -64.f}};
    }
    __device__ static half8 deq(const Code &c, const Step &k, const Blk &b, int p, int kk) {
        const uint32_t w = kk == 0 ? c.x : kk == 1 ? c.y : kk == 2 ? c.z : c.w;
        const uint32_t H = b.qh[64 * kk];
        const uint32_t t01 = __builtin_amdgcn_perm(0x64646464u, w, 0x04010400u);  // b0 64 b1 64
        const uint32_t t23 = __builtin_amdgcn_perm(0x64646464u, w, 0x04030402u);  // b2 64 b3 64
        const uint32_t u01 = __builtin_amdgcn_perm(0u, H, 0x0c010c00u);           // qh b0 0 b1 0
        const uint32_t u23 = __builtin_amdgcn_perm(0u, H, 0x0c030c02u);
        // bit 2p of a qh byte -> bit 4 of the half (+16 on 1024 + q); bit 2p + 1
        // -> bit 8 (+256 on 1024 + 16 q)
        auto lob = [&](uint32_t u) { return (p < 2 ? u << (4 - 2 * p) : u >> (2 * p - 4)) & 0x00100010u; };
        auto hib = [&](uint32_t u) { return (u << (7 - 2 * p)) & 0x01000100u; };
        return bd_h8(pk_fma((t01 & 0x640F640Fu) | lob(u01), k.s1, k.c1),
                     pk_fma((t23 & 0x640F640Fu) | lob(u23), k.s1, k.c1),
                     pk_fma((t01 & 0x64F064F0u) | hib(u01), k.s16, k.c16),
                     pk_fma((t23 & 0x64F064F0u) | hib(u23), k.s16, k.c16));
    }
    __device__ static void mins(const Head &hd, float inv_su, int h, bf16x8 &hi, bf16x8 &lo) {
        bd_mins(hd, inv_su, h, hi, lo);
    }
};

// IQ4_XS (weights rounded to f16): step p, lane half h = sub-block 2p + h,
// whose 16 code bytes hold elements 0..15 in the low nibbles and 16..31 in the
// high ones; group kk = elements 8kk .. 8kk + 7 (nibble kk / 2 of bytes
// 8 (kk % 2) .. + 7).  Operands (ls - 32) * kv in units of d, rounded once to
// f16 (exact while |(ls - 32) kv| <= 2048); kv from the codebook with two
// v_perm.  (dequant_iq4_xs, crates/arf-core/src/model/gguf.rs:1937-1976)
struct BdIQ4XS {
    static constexpr int XPARTS = 2;
    static constexpr bool EXTRA = false;
    struct Extra {};
    static constexpr bool XPERM = false, LATE = false;
    static constexpr bool UNITS = true, MIN = false, STEP_KK = false, WLO = false;
    static constexpr int VPM = 6;
    using Code = u32x4;
    using Head = u32x2;    // d | scales_h << 16, scales_l
    using Blk = uint32_t;  // ls - 32 of sub-blocks 2p + h as int8, byte p
    struct Step {
        half2v s, c;
    };
    const uint2 *hdr;
    const uint4 *qs;
    __device__ static int a_off(int p, int kk, int h) { return 64 * p + 32 * h + 8 * kk; }
    struct Lanes {
        __amdgpu_buffer_rsrc_t q, hd;
        uint32_t qv[2], hv[2];
        __device__ Code code(int g, int st) const {
            return __builtin_amdgcn_raw_buffer_load_b128(q, qv[g], (st >> 2) * 128 + 32 * (st & 3), 0);
        }
        __device__ Head head(int g, int blk) const {
            return __builtin_amdgcn_raw_buffer_load_b64(hd, hv[g], blk * 8, 0);
        }
    };
    __device__ Lanes lanes(int n, int nblk, uint32_t wr0, uint32_t wr1, int h) const {
        Lanes l;
        l.q = __builtin_amdgcn_make_buffer_rsrc((void *)qs, (short)0, (int)((uint32_t)n * nblk * 128), 0x00020000);
        l.hd = __builtin_amdgcn_make_buffer_rsrc((void *)hdr, (short)0, (int)((uint32_t)n * nblk * 8), 0x00020000);
        l.qv[0] = wr0 * nblk * 128 + 16 * h;
        l.qv[1] = wr1 * nblk * 128 + 16 * h;
        l.hv[0] = wr0 * nblk * 8;
        l.hv[1] = wr1 * nblk * 8;
        return l;
    }
    __device__ static float unit(const Head &hd) { return h2f(hd.x); }
    __device__ static Blk block(const Head &hd, const Extra &, int h, uint32_t *) {
        uint32_t packed = 0;
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const int s = 2 * p + h;
            const uint32_t ls = ((hd.y >> (4 * s)) & 0xFu) | (((hd.x >> (16 + 2 * s)) & 3u) << 4);
            packed |= ((ls - 32u) & 0xffu) << (8 * p);
        }
        return packed;
    }
    __device__ static void kill(Blk &b) { b = 0u; }
    __device__ static Step step(Blk b, int p, int) {
        const half2v s = h2splat((float)(int8_t)(b >> (8 * p)));
        return {s, s * (half2v){-1152.f, -1152.f}};  // 1152 |ls - 32| <= 36864: exact
    }
    __device__ static half8 deq(const Code &c, const Step &k, Blk, int, int kk) {
        const uint32_t w[2] = {(kk & 1) ? c.z : c.x, (kk & 1) ? c.w : c.y};
        uint32_t o[4];
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint32_t sel = (kk >> 1) ? (w[j] >> 4) & 0x0F0F0F0Fu : w[j] & 0x0F0F0F0Fu;
            const uint32_t v = iq4nl_lookup<0x80808080u>(sel);  // kv + 128 per byte
            // (1024 + kv + 128) * s - 1152 s = s * kv, one rounding
            o[2 * j] = pk_fma(__builtin_amdgcn_perm(0x64646464u, v, 0x04010400u), k.s, k.c);
            o[2 * j + 1] = pk_fma(__builtin_amdgcn_perm(0x64646464u, v, 0x04030402u), k.s, k.c);
        }
        return bd_h8(o[0], o[1], o[2], o[3]);
    }
};

// Q8_0 (weights d * q exact as two f16 operands, true units): step p of
// block b, lane half h = Q8_0 block 8b + 2p + h (its 32 codes, 32 bytes);
// group kk = elements 8kk .. 8kk + 7.  The header is the 8 block scales d of
// the 256 elements.  d * q has at most 19 significant bits (11 of d, 8 of q):
// hi = d * q rounded to f16 and lo = fma(q, d, -hi), the exact rounding error
// (at most 8 significant bits, a multiple of d's last place), are both exact
// f16 values and hi + lo = d * q, so each group runs its MFMAs twice, once per
// part (WLO).  (dequant_q8_0, crates/arf-core/src/model/gguf.rs)
struct BdQ80 {
    static constexpr int XPARTS = 2;
    static constexpr bool EXTRA = false;
    struct Extra {};
    static constexpr bool XPERM = false, LATE = false;
    static constexpr bool UNITS = false, MIN = false, STEP_KK = false, WLO = true;
    static constexpr int VPM = 4;
    struct Code {
        u32x4 a, b;
    };
    using Head = u32x4;  // d of the 8 Q8_0 blocks
    using Blk = u32x2;   // this lane's d of blocks 2p + h: half p % 2 of dword p / 2
    using Step = half2v;
    const uint4 *qs;
    const uint16_t *dd;
    __device__ static int a_off(int p, int kk, int h) { return 64 * p + 32 * h + 8 * kk; }
    struct Lanes {
        __amdgpu_buffer_rsrc_t q, hd;
        uint32_t qv[2], hv[2];
        __device__ Code code(int g, int st) const {
            const int so = (st >> 2) * 256 + 64 * (st & 3);
            return {__builtin_amdgcn_raw_buffer_load_b128(q, qv[g], so, 0),
                    __builtin_amdgcn_raw_buffer_load_b128(q, qv[g] + 16, so, 0)};
        }
        __device__ Head head(int g, int blk) const {
            return __builtin_amdgcn_raw_buffer_load_b128(hd, hv[g], blk * 16, 0);
        }
    };
    __device__ Lanes lanes(int n, int nblk, uint32_t wr0, uint32_t wr1, int h) const {
        Lanes l;
        l.q = __builtin_amdgcn_make_buffer_rsrc((void *)qs, (short)0, (int)((uint32_t)n * nblk * 256), 0x00020000);
        l.hd = __builtin_amdgcn_make_buffer_rsrc((void *)dd, (short)0, (int)((uint32_t)n * nblk * 16), 0x00020000);
        l.qv[0] = wr0 * nblk * 256 + 32 * h;
        l.qv[1] = wr1 * nblk * 256 + 32 * h;
        l.hv[0] = wr0 * nblk * 16;
        l.hv[1] = wr1 * nblk * 16;
        return l;
    }
    __device__ static float unit(const Head &) { return 1.f; }
    __device__ static Blk block(const Head &hd, const Extra &, int h, uint32_t *) {
        const uint32_t sel = h ? 0x07060302u : 0x05040100u;
        return {__builtin_amdgcn_perm(hd.y, hd.x, sel), __builtin_amdgcn_perm(hd.w, hd.z, sel)};
    }
    __device__ static void kill(Blk &b) { b = u32x2{0u, 0u}; }
    __device__ static Step step(const Blk &b, int p, int) {
        return as_h2(__builtin_amdgcn_perm(0u, (p >> 1) ? b.y : b.x, (p & 1) ? 0x03020302u : 0x01000100u));
    }
    __device__ static void deq2(const Code &c, const Step &d, const Blk &, int, int kk, half8 &hi, half8 &lo) {
        const uint32_t w[2] = {kk == 0 ? c.a.x : kk == 1 ? c.a.z : kk == 2 ? c.b.x : c.b.z,
                               kk == 0 ? c.a.y : kk == 1 ? c.a.w : kk == 2 ? c.b.y : c.b.w};
        const half2v m1152 = {-1152.f, -1152.f};
        uint32_t o[4], l[4];
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint32_t u = w[j] ^ 0x80808080u;  // q + 128 per byte
#pragma unroll
            for (int pr = 0; pr < 2; pr++) {
                // (1024 + q + 128) - 1152 = q exactly; hi = d * q rounded once, lo its error
                const half2v q = as_h2(__builtin_amdgcn_perm(0x64646464u, u, pr ? 0x04030402u : 0x04010400u)) + m1152;
                const half2v hv = q * d;
                o[2 * j + pr] = as_u(hv);
                l[2 * j + pr] = as_u(__builtin_elementwise_fma(q, d, -hv));
            }
        }
        hi = bd_h8(o[0], o[1], o[2], o[3]);
        lo = bd_h8(l[0], l[1], l[2], l[3]);
    }
};

// Q6_K (exact): step p = 48-byte chunk p of the block (ql_a[16] | ql_b[16] |
// qh[16]); lane half h takes bytes 8h .. 8h + 7 of each; group kk = quadrant
// kk: elements 128 (p / 2) + 16 (p % 2) + 32 kk + 8h + 0..7, one 16-element
// sub-block.  Operands sc * (q - 32) in units of d: an integer of magnitude at
// most 128 * 32 = 4096, exact in f16 up to 2048 (|sc| <= 64, the synthetic
// scales and WIDE = false); past 2048 f16 holds only even integers, so with
// WIDE (a tensor with some |sc| > 64) hi = sc * (q - 32) rounded and lo =
// fma(q - 32, sc, -hi) in {-1, 0, 1} run as two MFMAs (WLO).
// (dequant_q6_k, crates/arf-core/src/model/gguf.rs:2092-2131)
template <bool WIDE>
struct BdQ6KT {
    static constexpr int XPARTS = 2;
    static constexpr bool EXTRA = false;
    struct Extra {};
    static constexpr bool XPERM = false, LATE = true;
    static constexpr bool UNITS = true, MIN = false, STEP_KK = true, WLO = WIDE;
    static constexpr int VPM = 7;
    struct Code {
        u32x2 a, b, qh;
    };
    struct Head {
        u32x4 sc;
        uint32_t d;
    };
    using Blk = u32x4;  // the 16 int8 sub-block scales
    using Step = half2v;
    const uint2 *qb8;
    const uint4 *sc16;
    const uint16_t *dd;
    __device__ static int a_off(int p, int kk, int h) { return 128 * (p >> 1) + 16 * (p & 1) + 32 * kk + 8 * h; }
    struct Lanes {
        __amdgpu_buffer_rsrc_t q, s, d;
        uint32_t qv[2], sv[2], dv[2];
        __device__ Code code(int g, int st) const {
            const int so = (st >> 2) * 192 + 48 * (st & 3);
            return {__builtin_amdgcn_raw_buffer_load_b64(q, qv[g], so, 0),
                    __builtin_amdgcn_raw_buffer_load_b64(q, qv[g] + 16, so, 0),
                    __builtin_amdgcn_raw_buffer_load_b64(q, qv[g] + 32, so, 0)};
        }
        __device__ Head head(int g, int blk) const {
            return {__builtin_amdgcn_raw_buffer_load_b128(s, sv[g], blk * 16, 0),
                    (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(d, dv[g], blk * 2, 0)};
        }
    };
    __device__ Lanes lanes(int n, int nblk, uint32_t wr0, uint32_t wr1, int h) const {
        Lanes l;
        l.q = __builtin_amdgcn_make_buffer_rsrc((void *)qb8, (short)0, (int)((uint32_t)n * nblk * 192), 0x00020000);
        l.s = __builtin_amdgcn_make_buffer_rsrc((void *)sc16, (short)0, (int)((uint32_t)n * nblk * 16), 0x00020000);
        l.d = __builtin_amdgcn_make_buffer_rsrc((void *)dd, (short)0, (int)((uint32_t)n * nblk * 2), 0x00020000);
        l.qv[0] = wr0 * nblk * 192 + 8 * h;
        l.qv[1] = wr1 * nblk * 192 + 8 * h;
        l.sv[0] = wr0 * nblk * 16;
        l.sv[1] = wr1 * nblk * 16;
        l.dv[0] = wr0 * nblk * 2;
        l.dv[1] = wr1 * nblk * 2;
        return l;
    }
    __device__ static float unit(const Head &hd) { return h2f(hd.d); }
    __device__ static Blk block(const Head &hd, const Extra &, int, uint32_t *) { return hd.sc; }
    __device__ static void kill(Blk &b) { b = u32x4{0u, 0u, 0u, 0u}; }
    __device__ static Step step(const Blk &b, int p, int kk) {
        const int si = 8 * (p >> 1) + (p & 1) + 2 * kk;
        const uint32_t w = (si >> 2) == 0 ? b.x : (si >> 2) == 1 ? b.y : (si >> 2) == 2 ? b.z : b.w;
        return h2splat((float)(int8_t)(w >> (8 * (si & 3))));
    }
    // q as the f16 1024 + q (v_perm puts 0x64 above each code byte; the two
    // qh bits go to bits 4-5), minus 1056 (exact), times sc (one rounding,
    // none while |sc| <= 64); LO: the rounding error as a second operand
    template <bool LO>
    __device__ static void deq_t(const Code &c, const Step &sc, int kk, half8 &hi, half8 &lo) {
        const half2v m1056 = {-1056.f, -1056.f};
        const u32x2 ql = (kk & 1) ? c.b : c.a;
        uint32_t o[4], e[4];
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            const uint32_t l = (kk & 2) ? ((hh ? ql.y : ql.x) >> 4) : (hh ? ql.y : ql.x);
            const uint32_t qw = hh ? c.qh.y : c.qh.x;
#pragma unroll
            for (int pr = 0; pr < 2; pr++) {
                const uint32_t lp = __builtin_amdgcn_perm(0x64646464u, l, pr ? 0x04030402u : 0x04010400u);
                const uint32_t hp = __builtin_amdgcn_perm(0u, qw, pr ? 0x0c030c02u : 0x0c010c00u);
                const uint32_t top = 2 * kk <= 4 ? (hp << (4 - 2 * kk)) : (hp >> (2 * kk - 4));
                const uint32_t q = (lp & 0x640F640Fu) | (top & 0x00300030u);
                const half2v qm = as_h2(q) + m1056;
                const half2v hv = qm * sc;
                o[2 * hh + pr] = as_u(hv);
                if constexpr (LO) e[2 * hh + pr] = as_u(__builtin_elementwise_fma(qm, sc, -hv));
            }
        }
        hi = bd_h8(o[0], o[1], o[2], o[3]);
        if constexpr (LO) lo = bd_h8(e[0], e[1], e[2], e[3]);
    }
    __device__ static half8 deq(const Code &c, const Step &sc, const Blk &, int, int kk) {
        half8 hi, lo;
        deq_t<false>(c, sc, kk, hi, lo);
        return hi;
    }
    __device__ static void deq2(const Code &c, const Step &sc, const Blk &, int, int kk, half8 &hi, half8 &lo) {
        deq_t<true>(c, sc, kk, hi, lo);
    }
};
using BdQ6K = BdQ6KT<false>;   // every |sc| <= 64: one exact operand
using BdQ6KW = BdQ6KT<true>;   // some |sc| > 64: hi + lo operands

// Work items: the first `full` items are whole tiles (in XCD order when
// xcd_order); the remaining tiles are each split into `chunks` K ranges of
// whole blocks, one item per range, whose partial tiles go to part[item -
// full][BD_BM][BD_BN] and are added in chunk order by bd_reduce_kernel.  This
// fills the last round of workgroups when the tiles do not divide the CUs.
// PX (an f32 x as f16 hi + lo): x holds the m hi rows, then the m lo rows
// (and xs their sub-block sums in the same order).  A tile then covers 64
// rows: its staged rows 0..63 are the hi rows, 64..127 the same rows' lo
// parts, and the MFMAs of x row groups 2 and 3 accumulate onto groups 0 and 1
// (x = hi + lo, ~22 bits), at twice the MFMAs per output.
template <class F, bool PX = false>
__global__ __launch_bounds__(BD_THREADS, 1) void gemm_bd(
    F fmt, const _Float16 *__restrict__ x, const uint16_t *__restrict__ xs, const float *__restrict__ rs,
    float *__restrict__ y, float *__restrict__ part, int m, int n, int k, int mt, int xcd_order, int full,
    int chunks) {
    constexpr int RM = PX ? BD_BM / 2 : BD_BM;  // output rows per tile
    constexpr int MG = RM / 32;                 // accumulator row groups
    auto ai = [](int mg) { return PX ? mg & 1 : mg; };  // the accumulators x row group mg adds to
    extern __shared__ __attribute__((aligned(16))) _Float16 sx[];  // [2][BD_BM][BD_LD]
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int nblk = k / 256;

    // tile and block range of this work item (XCD x keeps a fixed set of x
    // tiles when the M tiles divide by 8; the dispatcher places workgroup b on
    // XCD b % 8)
    const int item = blockIdx.x;
    int tile, kb0 = 0, kb1 = nblk;
    const bool split = item >= full;
    if (!split) {
        if (xcd_order) {
            const int xcd = item & 7, q = item >> 3, per = mt >> 3;
            tile = (q / per) * mt + xcd * per + q % per;
        } else {
            tile = item;
        }
    } else {
        const int li = item - full, ch = li % chunks;
        tile = full + li / chunks;
        kb0 = (int)((int64_t)ch * nblk / chunks);
        kb1 = (int)((int64_t)(ch + 1) * nblk / chunks);
    }
    const int tm = tile % mt, tn = tile / mt;
    const int m0 = tm * RM, n0 = tn * BD_BN + wave * BD_WN;
    const int st0 = 4 * kb0, st1 = 4 * kb1;  // this item's steps

    const int col = lane & 31, h = lane >> 5;
    const uint32_t wr0 = min(n0 + col, n - 1), wr1 = min(n0 + 32 + col, n - 1);
    const typename F::Lanes ld = fmt.lanes(n, nblk, wr0, wr1, h);
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
        (void *)x, (short)0, (int)((uint32_t)(PX ? 2 : 1) * m * k * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(
        (void *)xs, (short)0, (int)((uint32_t)(PX ? 2 : 1) * m * (k / 16) * 2), 0x00020000);

    // x tile staging: thread t copies row t / 4.  The next block's x moves in
    // XP parts of 256 / XP halves of the row (two or four; fewer registers
    // held with four), each loaded during the current block and stored into
    // the other buffer a few groups later: thread (t % 4) takes 2 x 16 bytes
    // per 64 halves.
    constexpr int XP = F::XPARTS, XS = 4 / XP;  // parts, steps per part
    const int xr = tid >> 2, xo = (tid & 3) * 16;
    // the x row staged as tile row xr (with PX, rows 64.. are lo rows M + r)
    const uint32_t gxr = PX ? (xr < RM ? min(m0 + xr, m - 1) : m + min(m0 + xr - RM, m - 1)) : min(m0 + xr, m - 1);
    const uint32_t xv = gxr * k * 2 + xo * 2;  // bytes
    u32x4 xa[2 * XS];
    auto xload = [&](int blk, int part) {
#pragma unroll
        for (int j = 0; j < XS; j++) {
            const int so = blk * 512 + 128 * (XS * part + j);
            xa[2 * j] = __builtin_amdgcn_raw_buffer_load_b128(xrs, xv, so, 0);
            xa[2 * j + 1] = __builtin_amdgcn_raw_buffer_load_b128(xrs, xv + 16, so, 0);
        }
    };
    // x sub-block sums of the next block (min term): thread t moves 4 of row
    // t / 4's 16
    const uint32_t sv = gxr * (k / 16) * 2 + (tid & 3) * 8;  // bytes
    uint16_t *sxs = reinterpret_cast<uint16_t *>(sx + 2 * BD_BM * BD_LD);  // [2][BD_BM][16]
    // EXTRA block data: this wave's [2][4][64] dwords, at this lane
    uint32_t *exl = reinterpret_cast<uint32_t *>(sxs + 2 * BD_BM * 16) + (size_t)wave * 512 + lane;
    u32x2 xsa;
    auto xsload = [&](int blk) {
        if constexpr (F::MIN) xsa = __builtin_amdgcn_raw_buffer_load_b64(srs, sv, blk * 32, 0);
    };
    auto xsstore = [&](int buf) {
        if constexpr (F::MIN)
            *reinterpret_cast<u32x2 *>(sxs + ((size_t)buf * BD_BM + xr) * 16 + (tid & 3) * 4) = xsa;
    };
    auto xstore = [&](int buf, int part) {
#pragma unroll
        for (int j = 0; j < XS; j++) {
            _Float16 *row = sx + ((size_t)buf * BD_BM + xr) * BD_LD + 64 * (XS * part + j);
            if constexpr (F::XPERM) {
                // element e = 32 s + 16 hh + 4 kk + i of a step goes to slot
                // 32 hh + 8 kk + 4 s + i (s = sub-block parity); this thread's
                // 16 elements of each step have s = (t % 4) / 2, hh = t % 2
                const int base = 32 * (tid & 1) + 4 * ((tid >> 1) & 1);
#pragma unroll
                for (int kk = 0; kk < 4; kk++) {
                    const u32x4 &v = xa[2 * j + (kk >> 1)];
                    *reinterpret_cast<u32x2 *>(row + base + 8 * kk) = (kk & 1) ? u32x2{v.z, v.w} : u32x2{v.x, v.y};
                }
            } else {
                u32x4 *dst = reinterpret_cast<u32x4 *>(row + xo);
                dst[0] = xa[2 * j];
                dst[1] = xa[2 * j + 1];
            }
        }
    };
    // the groups that load and store x part q of the next block
    // (loads at the top of a group, stores at its end; with four parts one
    // part's registers are reused by the next)
    auto xload_at = [](int i, int q) { return XP == 2 ? i == 3 + 6 * q : i == 4 * q + 1; };
    auto xstore_at = [](int i, int q) { return XP == 2 ? i == (q == 0 ? 8 : 15) : i == (q == 3 ? 15 : 4 * q + 4); };

    // code ring: slot s % 2 holds step s (both groups' codes); it is refilled
    // with step s + 2 as soon as its last operand is built
    typename F::Code cq[2][2];
    auto cload = [&](int u, int st) {
        st = min(st, st1 - 1);  // past the end: reload the last step (unused)
        cq[u][0] = ld.code(0, st);
        cq[u][1] = ld.code(1, st);
    };
    // block headers of the two rows, one block ahead; a format's EXTRA block
    // data, from group 9 of the block before
    typename F::Head hdn[2];
    auto hload = [&](int blk) {
        blk = min(blk, kb1 - 1);
        hdn[0] = ld.head(0, blk);
        hdn[1] = ld.head(1, blk);
    };
    typename F::Extra ext[2];
    auto eload = [&](int blk) {
        if constexpr (F::EXTRA) {
            blk = min(blk, kb1 - 1);
            ext[0] = ld.extra(0, blk);
            ext[1] = ld.extra(1, blk);
        }
    };

    floatx16 acc[MG][2];
#pragma unroll
    for (int i = 0; i < MG; i++)
#pragma unroll
        for (int g = 0; g < 2; g++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][g][e] = 0.f;

    // prologue: the first block's x tile, the first headers and code steps
#pragma unroll
    for (int q = 0; q < XP; q++) {
        xload(kb0, q);
        xstore(0, q);
    }
    xsload(kb0);
    xsstore(0);
    hload(kb0);
    eload(kb0);
#pragma unroll
    for (int u = 0; u < 2; u++) cload(u, st0 + u);
    bd_barrier();

    // block scale state of the current block: scd (the step scales), inv =
    // 1 / su and ratio = su_prev / su, the factor that moves the accumulators
    // into this block's unit su (= d, or 1 when d = 0: zero weights); hdc
    // holds the block's headers for the min term
    typename F::Blk scd[2];
    float inv[2], ratio[2], sprev[2] = {1.f, 1.f};
    typename F::Head hdc[2];
    auto block_scales = [&]() {
#pragma unroll
        for (int g = 0; g < 2; g++) {
            hdc[g] = hdn[g];
            const float d = F::unit(hdc[g]);
            const bool live = d != 0.f;
            const float su = live ? d : 1.f;
            scd[g] = F::block(hdc[g], ext[g], h, exl + 256 * g);
            if (!live) F::kill(scd[g]);
            inv[g] = __builtin_amdgcn_rcpf(su);
            ratio[g] = sprev[g] * inv[g];
            sprev[g] = su;
        }
    };
    block_scales();
    hload(kb0 + 1);

    for (int blk = kb0; blk < kb1; blk++) {
        const int buf = (blk - kb0) & 1;
        const int nb = min(blk + 1, kb1 - 1);  // next block (past the end: unused copy)
        const _Float16 *xt0 = sx + ((size_t)buf * BD_BM + col) * BD_LD;

        // 16 MFMA groups per block: group i = (step p = i / 4, kk = i % 4) of
        // 8 MFMAs, g-major.  Operand registers are refilled as soon as their
        // last use has issued: b[1] between group i's four g = 0 MFMAs, b[0] of
        // group i + 1 between its four g = 1 MFMAs, a[mg] (x from LDS) after
        // MFMA (mg, g = 1).  Around them:
        //  - the accumulators move into this block's unit: g = 1 here, g = 0
        //    at the end of the previous block (behind its last MFMAs);
        //  - min term: groups 0, 1 work out its operands and group 2 adds
        //    -dmin * sum_j m_j X_j (units of d: two bf16 MFMAs per tile
        //    against the x sub-block sums, lane half h reading the hi / lo
        //    half of row (32 mg + l % 32)'s 16);
        //  - group 13 takes the next block's headers (scales, ratio; the last
        //    read of this block's scales is group 12's b[1]) and issues the
        //    loads of the one after; where every group's operands read the
        //    block data (LATE), group 15 does, after its b[1].
        half8 a[4], b[2], bw[2];  // bw: the weights' lo operands (WLO)
        typename F::Step ks[2];
        bf16x8 bh[2], bl[2], am[4];
        auto xread = [&](int i, int mg) {
            a[mg] = *reinterpret_cast<const half8 *>(xt0 + (size_t)mg * 32 * BD_LD + F::a_off(i >> 2, i & 3, h));
        };
        auto deq = [&](int i, int g) {
            const int p = i >> 2, kk = i & 3;
            if (F::STEP_KK || kk == 0) ks[g] = F::step(scd[g], p, kk);
            if constexpr (F::WLO)
                F::deq2(cq[p & 1][g], ks[g], scd[g], p, kk, b[g], bw[g]);
            else
                b[g] = F::deq(cq[p & 1][g], ks[g], scd[g], p, kk);
        };
#pragma unroll
        for (int mg = 0; mg < 4; mg++) xread(0, mg);
        deq(0, 0);
        if constexpr (F::UNITS) {
#pragma unroll
            for (int mg = 0; mg < MG; mg++)
#pragma unroll
                for (int e = 0; e < 16; e++) acc[mg][1][e] *= ratio[1];
        }
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int p = i >> 2, kk = i & 3;
            const bool more = i < 15;
            const bool mgroup = F::MIN && i == 2;  // the min-term group
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int q = 0; q < XP; q++)
                if (xload_at(i, q)) xload(nb, q);
            if (i == 3) xsload(nb);
            if (i == 9) eload(blk + 1);
            if (!F::LATE && i == 13) {
                block_scales();  // the next block's (scd of this one is used up)
                hload(blk + 2);
            }
            if constexpr (F::MIN) {
                if (i < 2) F::mins(hdc[i], inv[i], h, bh[i], bl[i]);
                if (i == 1) {
#pragma unroll
                    for (int mg = 0; mg < 4; mg++)
                        am[mg] = *reinterpret_cast<const bf16x8 *>(sxs + ((size_t)buf * BD_BM + 32 * mg + col) * 16 + 8 * h);
                }
            }
#pragma unroll
            for (int mg = 0; mg < 4; mg++) {
                acc[ai(mg)][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[mg], b[0], acc[ai(mg)][0], 0, 0, 0);
                if constexpr (F::WLO)
                    acc[ai(mg)][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[mg], bw[0], acc[ai(mg)][0], 0, 0, 0);
                if (mgroup) {
#pragma unroll
                    for (int g = 0; g < 2; g++) {
                        acc[ai(mg)][g] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(am[mg], bh[g], acc[ai(mg)][g], 0, 0, 0);
                        acc[ai(mg)][g] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(am[mg], bl[g], acc[ai(mg)][g], 0, 0, 0);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            deq(i, 1);  // this group's second B operand, under its first four MFMAs
            if (!mgroup) {
#pragma unroll
                for (int mg = 0; mg < 4; mg++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, F::WLO ? 2 : 1, 0);  // one MFMA (per part)
                    __builtin_amdgcn_sched_group_barrier(0x002, F::VPM, 0);           // VALU
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            if (F::LATE && i == 15) {
                block_scales();  // block data read by every group: the last read is above
                hload(blk + 2);
            }
            if (F::UNITS && i == 15) {
                // group 0's accumulators into the next block's unit (the last
                // block keeps its unit)
                const float r0 = blk + 1 < kb1 ? ratio[0] : 1.f;
#pragma unroll
                for (int mg = 0; mg < MG; mg++)
#pragma unroll
                    for (int e = 0; e < 16; e++) acc[mg][0][e] *= r0;
            }
#pragma unroll
            for (int mg = 0; mg < 4; mg++) {
                acc[ai(mg)][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[mg], b[1], acc[ai(mg)][1], 0, 0, 0);
                if constexpr (F::WLO)
                    acc[ai(mg)][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[mg], bw[1], acc[ai(mg)][1], 0, 0, 0);
                if (more) xread(i + 1, mg);
            }
            if (more) deq(i + 1, 0);  // the next group's first B operand, under these MFMAs
#pragma unroll
            for (int mg = 0; mg < 4; mg++) {
                __builtin_amdgcn_sched_group_barrier(0x008, F::WLO ? 2 : 1, 0);  // one MFMA (per part)
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                // its x read
                __builtin_amdgcn_sched_group_barrier(0x002, F::VPM, 0);           // VALU
            }
            __builtin_amdgcn_sched_barrier(0);
            if (kk == 3) cload(p & 1, 4 * blk + p + 2);  // the slot is free: step + 2
#pragma unroll
            for (int q = 0; q < XP; q++)
                if (xstore_at(i, q)) xstore(buf ^ 1, q);
            if (i == 8) xsstore(buf ^ 1);
        }
        bd_barrier();
    }
    if constexpr (F::UNITS) {
        // back to true units
#pragma unroll
        for (int g = 0; g < 2; g++)
#pragma unroll
            for (int mg = 0; mg < MG; mg++)
#pragma unroll
                for (int e = 0; e < 16; e++) acc[mg][g][e] *= sprev[g];
    }

    // C layout of a 32x32 tile: lane l, value i -> row 8 (i/4) + 4 (l/32) + i%4, column l % 32
    float *pt = split ? part + (size_t)(item - full) * BD_BM * BD_BN : nullptr;
#pragma unroll
    for (int mg = 0; mg < MG; mg++) {
#pragma unroll
        for (int g = 0; g < 2; g++) {
            const int cl = wave * BD_WN + 32 * g + col;  // column within the tile
            const int cn = n0 + 32 * g + col;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int rl = 32 * mg + 8 * (i >> 2) + 4 * h + (i & 3);
                if (split) {
                    pt[(size_t)rl * BD_BN + cl] = acc[mg][g][i];
                } else if (cn < n && m0 + rl < m) {
                    y[(int64_t)(m0 + rl) * n + cn] = rs ? acc[mg][g][i] * rs[m0 + rl] : acc[mg][g][i];
                }
            }
        }
    }
}

// y of the split tiles: the chunks' partial tiles added in chunk order.
// A thread per 4 consecutive outputs of a tile row (16-byte partial loads,
// up to 8 chunks' loads in flight at once); grid (rm * BD_BN / 1024, split
// tiles), rm the output rows per tile (BD_BM, or half with an x of two parts).
__global__ __launch_bounds__(256) void bd_reduce_kernel(const float *__restrict__ part,
                                                        const float *__restrict__ rs,
                                                        float *__restrict__ y, int m, int n,
                                                        int mt, int full, int chunks, int rm) {
    const int lt = blockIdx.y;
    const int e = (blockIdx.x * 256 + threadIdx.x) * 4;
    const int rl = e / BD_BN, cl = e - rl * BD_BN;
    const int tile = full + lt;
    const int r = (tile % mt) * rm + rl, c = (tile / mt) * BD_BN + cl;  // rm rows per tile
    if (rl >= rm || r >= m || c >= n) return;
    const float4 *pp = reinterpret_cast<const float4 *>(part + (size_t)lt * chunks * BD_BM * BD_BN + e);
    constexpr size_t CS = (size_t)BD_BM * BD_BN / 4;  // one chunk's tile, in float4
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int j0 = 0; j0 < chunks; j0 += 8) {
        float4 t[8];
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (j0 + j < chunks) t[j] = pp[(size_t)(j0 + j) * CS];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            if (j0 + j < chunks) {
                v.x += t[j].x;
                v.y += t[j].y;
                v.z += t[j].z;
                v.w += t[j].w;
            }
        }
    }
    const float sr = rs ? rs[r] : 1.f;
    float *yr = y + (int64_t)r * n + c;
    const float o[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; i++)
        if (c + i < n) yr[i] = rs ? o[i] * sr : o[i];
}

}  // namespace arfq
