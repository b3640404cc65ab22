// arfq_common.h -- device-side layout of the repacked GGUF blocks and the
// per-format dequant helpers shared by every kernel (GEMV, GEMM, MoE, and the
// arfq_dequant_f32 parity hook).
//
// Device layouts (all lossless permutations of ggml's bytes; each stream is a
// separate 256-B aligned allocation; blocks are ordered expert-major, then row,
// then along k):
//   Q4_K  hdr[nblk] 16 B  = d(f16) | dmin(f16) | scales[12]   (ggml bytes 0..15)
//         qs [nblk] 128 B = the 256 nibbles regrouped per sub-block: dword 4j+w
//                           holds elements 32j+8w .. 32j+8w+7 of sub-block j; its
//                           byte i (0..3) holds element 32j+8w+i in the low nibble
//                           and element 32j+8w+4+i in the high nibble (nibble
//                           position p <-> element 8w + q4k_sigma(p)).  The order
//                           matches how the GEMV packs x digits with v_perm.
//                           ggml stores element 32j+i in byte 32*(j/2)+i, low
//                           nibble for even j, high for odd j.
//   Q8_0  qs [nblk] 32 B  = the 32 i8 codes;   d[nblk] f16
//   Q6_K  qb [nblk] 192 B = 4 chunks of 48 B; chunk c (n2 = c/2, l0 = 16*(c%2)):
//                           ql[64n2+l0 .. +16] | ql[64n2+32+l0 .. +16] | qh[32n2+l0 .. +16]
//         sc [nblk] 16 B  = the 16 i8 sub-block scales;  d[nblk] f16
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "../../include/arfq.h"

namespace arfq {

constexpr int QK_K = 256;
constexpr int WAVE = 64;

// f16 bits -> f32.  v_cvt_f32_f16 is exact for every f16 value, subnormals
// included (f16 denormals are not flushed in the default gfx950 FP mode); the
// exhaustive 65536-pattern test pins this against the reference's
// f16_to_f32 (crates/arf-ml/src/dtype.rs:41-70).
__device__ __forceinline__ float h2f(uint32_t bits16) {
    return __half2float(__ushort_as_half((unsigned short)(bits16 & 0xffffu)));
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// two f32 -> f16 (round to nearest even, as a scalar (_Float16) cast) packed
// low | high << 16
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
    const f16x2 h = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, h);
}

// Workgroup barrier that orders LDS accesses only.  __syncthreads() also waits
// for every outstanding global load of the wave (s_waitcnt vmcnt(0)); this one
// leaves weight loads issued before it in flight.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// 16-byte streaming load (non-temporal hint: each weight byte is read once).
__device__ __forceinline__ uint4 ld_nt(const uint4 *p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// nibble position p (0..7) of a Q4_K code dword -> element offset within its
// 8-element group; and the inverse
__host__ __device__ constexpr int q4k_sigma(int p) { return (p & 1) ? 4 + (p >> 1) : (p >> 1); }
__host__ __device__ constexpr int q4k_sigma_inv(int t) { return t < 4 ? 2 * t : 2 * (t - 4) + 1; }

__device__ __forceinline__ uint32_t byte_of(uint32_t w, int i) { return (w >> (8 * i)) & 0xffu; }

// Bit s (0..7) of every byte of w, moved to bit 4 of its byte (the fifth bit of
// a Q5_K code): one rotate (v_alignbit_b32) and a mask.
__device__ __forceinline__ uint32_t bit_to4(uint32_t w, int s) {
    return __builtin_amdgcn_alignbit(w, w, (uint32_t)(s - 4) & 31u) & 0x10101010u;
}

// The IQ4_NL codebook value (ggml's kvalues_iq4nl, gguf.rs:1908-1914) xor X of
// four 4-bit codes, one per byte of sel: two v_perm over the table's 8-entry
// halves (entries 0..7 and 8..15 as little-endian bytes), and a third that
// takes each byte from the half its code's bit 3 names (selector i or i + 4).
template <uint32_t X>
__device__ __forceinline__ uint32_t iq4nl_lookup(uint32_t sel) {
    constexpr uint32_t T0lo = 0xBFAD9881u ^ X, T0hi = 0xF6EADDCFu ^ X;
    constexpr uint32_t T1lo = 0x26190D01u ^ X, T1hi = 0x71594535u ^ X;
    const uint32_t s7 = sel & 0x07070707u;
    const uint32_t v0 = __builtin_amdgcn_perm(T0hi, T0lo, s7);
    const uint32_t v1 = __builtin_amdgcn_perm(T1hi, T1lo, s7);
    return __builtin_amdgcn_perm(v1, v0, ((sel >> 1) & 0x04040404u) | 0x03020100u);
}

// 6-bit scale / min of Q4_K sub-block j (0..7) from the header dwords
// s0 = scales[0..3], s1 = scales[4..7], s2 = scales[8..11]  (ggml
// get_scale_min_k4; crates/arf-ml/src/weight.rs:1353-1365).
__device__ __forceinline__ void q4k_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int j,
                                              uint32_t &sc, uint32_t &m) {
    if (j < 4) {
        sc = byte_of(s0, j) & 63u;
        m = byte_of(s1, j) & 63u;
    } else {
        const int i = j - 4;
        sc = (byte_of(s2, i) & 0xFu) | ((byte_of(s0, i) >> 6) << 4);
        m = (byte_of(s2, i) >> 4) | ((byte_of(s1, i) >> 6) << 4);
    }
}

// Q4_K weight:  (d*sc)*q - (dmin*m), three separately rounded f32 operations
// (crates/arf-core/src/model/gguf.rs:2022-2031).  Contraction into an FMA would
// change the last bit, so it is switched off here.
__device__ __forceinline__ float q4k_weight(float d1, float m1, uint32_t q) {
#pragma clang fp contract(off)
    return d1 * (float)q - m1;
}
__device__ __forceinline__ float q4k_d1(float d, uint32_t sc) {
#pragma clang fp contract(off)
    return d * (float)sc;
}

// Q8_0 weight: d * q (crates/arf-core/src/model/gguf.rs:1645).
__device__ __forceinline__ float q80_weight(float d, int q) {
#pragma clang fp contract(off)
    return d * (float)q;
}

// Q6_K weight: (d * sc) * (q - 32), left to right (gguf.rs:2120-2123).
__device__ __forceinline__ float q6k_weight(float d, int sc, int q) {
#pragma clang fp contract(off)
    return d * (float)sc * (float)(q - 32);
}

// Extract the 6-bit code q_{t+1} (t = quadrant 0..3) of element i (0..15) of a
// Q6_K 48-byte chunk, given the chunk as 12 dwords w[0..11]:
//   t=0: ql_a low nibble | qh bits 0-1;  t=1: ql_b low | qh bits 2-3;
//   t=2: ql_a high       | qh bits 4-5;  t=3: ql_b high | qh bits 6-7.
// (crates/arf-core/src/model/gguf.rs:2110-2117)
__device__ __forceinline__ int q6k_code(const uint32_t *w, int t, int i) {
    const uint32_t qla = byte_of(w[i >> 2], i & 3);
    const uint32_t qlb = byte_of(w[4 + (i >> 2)], i & 3);
    const uint32_t qh = byte_of(w[8 + (i >> 2)], i & 3);
    const uint32_t lo = (t & 1) ? qlb : qla;
    const uint32_t nib = (t & 2) ? (lo >> 4) : (lo & 0xFu);
    return (int)(nib | (((qh >> (2 * t)) & 3u) << 4));
}

// ---- gated FFN activations: h = act(g) * u ---------------------------------
// act 0, SwiGLU: silu(g) = g / (1 + exp(-g)) (crates/arf-ml/src/lib.rs:160-162,
// mlp.rs:20-24).  act 1, GeGLU: gelu_tanh(g) = 0.5 g (1 + tanh(inner)),
// inner = sqrt(2/pi) (g + 0.044715 g^3) clamped to [-15, 15] before the tanh
// (shaders/metal/decode_ops_msl.metal:15-27; CPU oracle
// gpu/metal/selftest.rs:6091-6095), the gate activation of GateAct::GeluTanh
// models (crates/arf-core/src/config.rs:58).  Evaluated left to right without
// contraction, as the reference writes them.
constexpr int ACT_SILU = ARFQ_ACT_SILU, ACT_GELU_TANH = ARFQ_ACT_GELU_TANH;
template <int ACT>
__device__ __forceinline__ float glu(float g, float u) {
#pragma clang fp contract(off)
    if constexpr (ACT == ACT_GELU_TANH) {
        const float inner = fminf(fmaxf(0.7978845608028654f * (g + 0.044715f * g * g * g), -15.0f), 15.0f);
        return 0.5f * g * (1.0f + tanhf(inner)) * u;
    } else {
        return g / (1.0f + expf(-g)) * u;
    }
}

}  // namespace arfq
