/*
 * arfq_oracle.c -- CPU restatement of Arf's reference arithmetic for the GGUF
 * quantized-matmul path (Q8_0 / Q4_K / Q6_K dequant, the Q4_K_S transcode, the
 * quantized and f32 CPU matmuls, top-k softmax routing and the SwiGLU MoE block).
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the HIP library is held
 * against; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it.  The product (arf_amd/, libarfq.so) never links or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the joydle/Arf source tree).  The reference is Rust; Rust never contracts
 * a*b+c into an FMA, so this file is built with -ffp-contract=off and every
 * expression keeps the reference's evaluation order.
 *
 * Pinning status (what checks each function beyond re-reading the formula):
 *   f16_to_f32          all 65536 bit patterns vs numpy float16 (IEEE) + known values
 *   q4k_get_scale_min   reference known answers + exhaustive bit-level model
 *   dequant_q4_k        reference known block (19.0 / -5.0) + LCG bit-exact gate
 *   q4ks transcode      bit-exact vs dequant_q4_k on the reference's LCG gate
 *   dequant_q6_k        reference known block (-44.0) + closed-form per-quadrant blocks
 *   dequant_q8_0        closed form y = d*q, exhaustive over q
 *   matmul_nt*          quantized == dequant + double-precision matmul; integer exactness
 *   top_k_softmax       reference route cases (ties, 128-expert LCG cases)
 *   moe_forward         closed forms (one-hot router, identity-like experts)
 * The last-ULP order of `wide` 1.7.1's f32x8 reduce_add inside matmul_nt and
 * Rust's f32::exp are not reproducible without the Rust toolchain; both are far
 * below the 2e-3 matmul gate ("last-ULP unpinned").
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#define QK_K 256
#define QK8 32

/* f32 matmul (a9), defined below; the dequant-then-matmul oracles above it use it */
void arfo_matmul_nt(const float *a, int64_t m, int64_t k, const float *b, int64_t n, float *out);

/* ---- a1: f16 -> f32.  crates/arf-ml/src/dtype.rs:41-70 ------------------- */
float arfo_f16_to_f32(uint16_t h) {
    uint32_t sign = (h >> 15) & 1u;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu;
    uint32_t f;
    if (exp == 0) {
        if (mant == 0) {
            f = sign << 31;
        } else {
            /* subnormal: shift the mantissa up until the implicit bit appears */
            int32_t e = -14;
            uint32_t m = mant;
            while ((m & 0x400u) == 0) {
                m <<= 1;
                e -= 1;
            }
            m &= 0x3ffu;
            f = (sign << 31) | ((uint32_t)(e + 127) << 23) | (m << 13);
        }
    } else if (exp == 0x1f) {
        f = (sign << 31) | (0xffu << 23) | (mant << 13);
    } else {
        f = (sign << 31) | ((exp + 112u) << 23) | (mant << 13);
    }
    float out;
    memcpy(&out, &f, 4);
    return out;
}

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* ---- a3: 6-bit scale/min unpack.  crates/arf-ml/src/weight.rs:1353-1365 --- */
void arfo_q4k_get_scale_min(const uint8_t *s, int j, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* ---- a2: Q8_0 dequant.  crates/arf-core/src/model/gguf.rs:1633-1649 ------- */
void arfo_dequant_q8_0(const uint8_t *bytes, int64_t n, float *out) {
    int64_t nblocks = n / QK8;
    for (int64_t b = 0; b < nblocks; b++) {
        const uint8_t *p = bytes + b * 34;
        float d = arfo_f16_to_f32(rd16(p));
        const uint8_t *qs = p + 2;
        for (int k = 0; k < 32; k++) out[b * 32 + k] = d * (float)(int8_t)qs[k];
    }
}

/* ---- a4: Q4_K dequant.  crates/arf-core/src/model/gguf.rs:2004-2035 ------- */
void arfo_dequant_q4_k(const uint8_t *bytes, int64_t n, float *out) {
    int64_t nblocks = n / QK_K;
    for (int64_t b = 0; b < nblocks; b++) {
        const uint8_t *p = bytes + b * 144;
        float d = arfo_f16_to_f32(rd16(p));
        float dmin = arfo_f16_to_f32(rd16(p + 2));
        const uint8_t *scales = p + 4;
        const uint8_t *qs = p + 16;
        float *o = out + b * QK_K;
        for (int j = 0; j < 8; j++) {
            uint8_t sc, m;
            arfo_q4k_get_scale_min(scales, j, &sc, &m);
            float d1 = d * (float)sc;
            float m1 = dmin * (float)m;
            int qbase = (j / 2) * 32;
            int shift = (j % 2 == 0) ? 0 : 4;
            for (int i = 0; i < 32; i++) {
                float q = (float)((qs[qbase + i] >> shift) & 0xF);
                o[j * 32 + i] = d1 * q - m1;
            }
        }
    }
}

/* ---- a5: Q6_K dequant.  crates/arf-core/src/model/gguf.rs:2092-2131 ------- */
void arfo_dequant_q6_k(const uint8_t *bytes, int64_t n, float *out) {
    int64_t nblocks = n / QK_K;
    for (int64_t b = 0; b < nblocks; b++) {
        const uint8_t *p = bytes + b * 210;
        const uint8_t *ql = p;
        const uint8_t *qh = p + 128;
        const int8_t *scales = (const int8_t *)(p + 192);
        float d = arfo_f16_to_f32(rd16(p + 208));
        float *o = out + b * QK_K;
        for (int n2 = 0; n2 < 2; n2++) {
            int bql = n2 * 64, bqh = n2 * 32, bsc = n2 * 8, bo = n2 * 128;
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                int q1 = (ql[bql + l] & 0xF) | ((qh[bqh + l] & 3) << 4);
                int q2 = (ql[bql + l + 32] & 0xF) | (((qh[bqh + l] >> 2) & 3) << 4);
                int q3 = ((ql[bql + l] >> 4) & 0xF) | (((qh[bqh + l] >> 4) & 3) << 4);
                int q4 = ((ql[bql + l + 32] >> 4) & 0xF) | (((qh[bqh + l] >> 6) & 3) << 4);
                /* `d * sc as f32 * (q - 32) as f32` evaluates left to right */
                o[bo + l] = d * (float)scales[bsc + is] * (float)(q1 - 32);
                o[bo + l + 32] = d * (float)scales[bsc + is + 2] * (float)(q2 - 32);
                o[bo + l + 64] = d * (float)scales[bsc + is + 4] * (float)(q3 - 32);
                o[bo + l + 96] = d * (float)scales[bsc + is + 6] * (float)(q4 - 32);
            }
        }
    }
}

/* ---- next row f2: Q5_K dequant.  crates/arf-core/src/model/gguf.rs:2053-2090.
 * Block = 176 B: f16 d, f16 dmin, scales[12] (Q4_K packing), qh[32] (the 5th bit),
 * qs[128] (low nibbles).  Group g (64 weights): sub-blocks 2g (low nibbles of
 * qs[32g + l], 5th bit qh[l] & (1 << 2g)) and 2g + 1 (high nibbles, 5th bit
 * qh[l] & (2 << 2g)); y = d1 * q - m1 with d1 = d * sc, m1 = dmin * m. */
void arfo_dequant_q5_k(const uint8_t *bytes, int64_t n, float *out) {
    int64_t nblocks = n / QK_K;
    for (int64_t b = 0; b < nblocks; b++) {
        const uint8_t *p = bytes + b * 176;
        float d = arfo_f16_to_f32(rd16(p));
        float dmin = arfo_f16_to_f32(rd16(p + 2));
        const uint8_t *scales = p + 4, *qh = p + 16, *qs = p + 48;
        float *o = out + b * QK_K;
        for (int g = 0; g < 4; g++) {
            uint8_t sc1, m1, sc2, m2;
            arfo_q4k_get_scale_min(scales, 2 * g, &sc1, &m1);
            arfo_q4k_get_scale_min(scales, 2 * g + 1, &sc2, &m2);
            float d1 = d * (float)sc1, mm1 = dmin * (float)m1;
            float d2 = d * (float)sc2, mm2 = dmin * (float)m2;
            uint8_t u1 = (uint8_t)(1u << (2 * g)), u2 = (uint8_t)(2u << (2 * g));
            for (int l = 0; l < 32; l++) {
                float q = (float)(qs[32 * g + l] & 0xF) + ((qh[l] & u1) ? 16.0f : 0.0f);
                o[64 * g + l] = d1 * q - mm1;
            }
            for (int l = 0; l < 32; l++) {
                float q = (float)(qs[32 * g + l] >> 4) + ((qh[l] & u2) ? 16.0f : 0.0f);
                o[64 * g + 32 + l] = d2 * q - mm2;
            }
        }
    }
}

/* ---- next row f2: IQ4_XS dequant.  crates/arf-core/src/model/gguf.rs:1908-1976.
 * Block = 136 B: f16 d, u16 scales_h, scales_l[4], qs[128].  Sub-block j (32
 * weights): ls = ((scales_l[j/2] >> 4 (j%2)) & 15) | (((scales_h >> 2j) & 3) << 4),
 * dl = d * (ls - 32); weight 32j + i = dl * kvalues[qs[16j + i] & 15] (i < 16),
 * dl * kvalues[qs[16j + i - 16] >> 4] (i >= 16), kvalues the non-linear IQ4 codebook. */
static const int8_t IQ4_KVALUES[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                       1,    13,   25,  38,  53,  69,  89,  113};
void arfo_dequant_iq4_xs(const uint8_t *bytes, int64_t n, float *out) {
    int64_t nblocks = n / QK_K;
    for (int64_t b = 0; b < nblocks; b++) {
        const uint8_t *p = bytes + b * 136;
        float d = arfo_f16_to_f32(rd16(p));
        uint16_t scales_h = rd16(p + 2);
        const uint8_t *scales_l = p + 4, *qs = p + 8;
        float *o = out + b * QK_K;
        for (int j = 0; j < 8; j++) {
            int lo = (scales_l[j / 2] >> (4 * (j % 2))) & 0xF;
            int hi = (scales_h >> (2 * j)) & 3;
            float dl = d * (float)(((hi << 4) | lo) - 32);
            for (int i = 0; i < 16; i++) {
                o[32 * j + i] = dl * (float)IQ4_KVALUES[qs[16 * j + i] & 0xF];
                o[32 * j + i + 16] = dl * (float)IQ4_KVALUES[qs[16 * j + i] >> 4];
            }
        }
    }
}

/* IQ4_XS reference matmul: dequant then matmul_nt (the CPU path reads IQ4_XS
 * through its f32 dequant; gguf.rs:1937-1976 then matmul.rs:84-99). */
void arfo_matmul_nt_iq4_xs(const float *a, int64_t m, int64_t k, const uint8_t *blocks, int64_t n,
                           float *out) {
    float *w = (float *)malloc((size_t)(n * k) * 4);
    arfo_dequant_iq4_xs(blocks, n * k, w);
    arfo_matmul_nt(a, m, k, w, n, out);
    free(w);
}

/* Q5KSMatrix::from_ggml_q5k (crates/arf-ml/src/weight.rs:551-632): low nibbles 8 per
 * u32 in element order, the 5th bit 32 per u32 (bit 1 << ss of qh[i] for sub-block
 * ss, element i), sub-block scales u8, mins -m as i8, d / dmin widened to f32. */
void arfo_q5ks_from_ggml(const uint8_t *blocks, int64_t rows, int64_t cols, uint32_t *codes_lo,
                         uint32_t *codes_hi, uint8_t *scales, int8_t *mins, float *d, float *dmin) {
    int64_t spr = cols / 32, bpr = cols / QK_K;
    memset(codes_lo, 0, (size_t)(rows * cols / 8) * 4);
    memset(codes_hi, 0, (size_t)(rows * cols / 32) * 4);
    for (int64_t r = 0; r < rows; r++)
        for (int64_t sb = 0; sb < bpr; sb++) {
            const uint8_t *p = blocks + (r * bpr + sb) * 176;
            d[r * bpr + sb] = arfo_f16_to_f32(rd16(p));
            dmin[r * bpr + sb] = arfo_f16_to_f32(rd16(p + 2));
            const uint8_t *qh = p + 16, *qs = p + 48;
            for (int ss = 0; ss < 8; ss++) {
                uint8_t sc, m;
                arfo_q4k_get_scale_min(p + 4, ss, &sc, &m);
                scales[r * spr + sb * 8 + ss] = sc;
                mins[r * spr + sb * 8 + ss] = (int8_t)(-(int)m);
                int shift = (ss % 2) ? 4 : 0;
                for (int i = 0; i < 32; i++) {
                    uint32_t lo = (uint32_t)((qs[(ss / 2) * 32 + i] >> shift) & 0xF);
                    uint32_t hi = (qh[i] >> ss) & 1u;
                    int64_t pos = r * cols + sb * QK_K + ss * 32 + i;
                    codes_lo[pos / 8] |= lo << ((pos % 8) * 4);
                    codes_hi[pos / 32] |= hi << (pos % 32);
                }
            }
        }
}

/* ---- a6: lossless ggml Q4_K -> Q4_K_S transcode.
 *      crates/arf-ml/src/weight.rs:1000-1080 (from_ggml_q4k) ---------------- */
void arfo_q4ks_from_ggml(const uint8_t *blocks, int64_t rows, int64_t cols, uint32_t *codes,
                         uint8_t *scales, int8_t *mins, float *d, float *dmin) {
    int64_t subs_per_row = cols / 32, supers_per_row = cols / QK_K;
    memset(codes, 0, (size_t)(rows * cols / 8) * sizeof(uint32_t));
    for (int64_t r = 0; r < rows; r++) {
        for (int64_t sblk = 0; sblk < supers_per_row; sblk++) {
            int64_t b = r * supers_per_row + sblk;
            const uint8_t *p = blocks + b * 144;
            d[b] = arfo_f16_to_f32(rd16(p));
            dmin[b] = arfo_f16_to_f32(rd16(p + 2));
            const uint8_t *sb12 = p + 4, *qs = p + 16;
            for (int ss = 0; ss < 8; ss++) {
                int half = ss / 2, shift = (ss % 2 == 0) ? 0 : 4;
                uint8_t sc, m;
                arfo_q4k_get_scale_min(sb12, ss, &sc, &m);
                int64_t sb = r * subs_per_row + sblk * 8 + ss;
                scales[sb] = sc;
                mins[sb] = (int8_t)(-(int)m);
                for (int i = 0; i < 32; i++) {
                    uint32_t code = (uint32_t)((qs[half * 32 + i] >> shift) & 0xF);
                    int64_t pos = r * cols + sblk * QK_K + ss * 32 + i;
                    codes[pos / 8] |= code << ((pos % 8) * 4);
                }
            }
        }
    }
}

/* Q4_K_S dequant.  crates/arf-ml/src/weight.rs:1110-1136 (to_f32) */
void arfo_q4ks_to_f32(const uint32_t *codes, const uint8_t *scales, const int8_t *mins,
                      const float *d, const float *dmin, int64_t rows, int64_t cols, float *out) {
    int64_t subs_per_row = cols / 32, supers_per_row = cols / QK_K;
    for (int64_t r = 0; r < rows; r++) {
        for (int64_t sblk = 0; sblk < supers_per_row; sblk++) {
            int64_t sidx = r * supers_per_row + sblk;
            float dq = d[sidx], dmq = dmin[sidx];
            for (int ss = 0; ss < 8; ss++) {
                int64_t sb = r * subs_per_row + sblk * 8 + ss;
                float s = dq * (float)scales[sb];
                float lo = dmq * (float)mins[sb];
                int64_t base = r * cols + (sblk * 8 + ss) * 32;
                for (int j = 0; j < 32; j++) {
                    uint32_t code = (codes[(base + j) / 8] >> (((base + j) % 8) * 4)) & 0xF;
                    out[base + j] = (float)code * s + lo;
                }
            }
        }
    }
}

/* ---- par_rows: crates/arf-ml/src/matmul.rs:16-45.  Output rows (the M
 * activation rows) are split over `threads` workers; serial when threads <= 1,
 * n_rows < 2 or row_len*n_rows < 2^14. ------------------------------------- */
typedef void (*row_fn)(void *ctx, int64_t i, float *row);
typedef struct {
    row_fn f;
    void *ctx;
    float *out;
    int64_t row_len, lo, hi;
} par_job;

static void *par_worker(void *arg) {
    par_job *j = (par_job *)arg;
    for (int64_t i = j->lo; i < j->hi; i++) j->f(j->ctx, i, j->out + i * j->row_len);
    return NULL;
}

static int g_threads = 0; /* 0 -> hardware concurrency */

void arfo_set_threads(int t) { g_threads = t; }

int arfo_threads(void) {
    if (g_threads > 0) return g_threads;
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    return n > 0 ? (int)n : 1;
}

static void par_rows(float *out, int64_t row_len, int64_t n_rows, row_fn f, void *ctx) {
    int threads = arfo_threads();
    if (threads <= 1 || n_rows < 2 || row_len * n_rows < (1 << 14)) {
        for (int64_t i = 0; i < n_rows; i++) f(ctx, i, out + i * row_len);
        return;
    }
    int64_t rows_per = (n_rows + threads - 1) / threads;
    int64_t nt = (n_rows + rows_per - 1) / rows_per;
    pthread_t *tid = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)nt);
    par_job *jobs = (par_job *)malloc(sizeof(par_job) * (size_t)nt);
    for (int64_t t = 0; t < nt; t++) {
        jobs[t].f = f;
        jobs[t].ctx = ctx;
        jobs[t].out = out;
        jobs[t].row_len = row_len;
        jobs[t].lo = t * rows_per;
        jobs[t].hi = (t + 1) * rows_per < n_rows ? (t + 1) * rows_per : n_rows;
        pthread_create(&tid[t], NULL, par_worker, &jobs[t]);
    }
    for (int64_t t = 0; t < nt; t++) pthread_join(tid[t], NULL);
    free(tid);
    free(jobs);
}

/* ---- a9: f32 matmul_nt + SIMD dot.  crates/arf-ml/src/matmul.rs:47-64,84-99.
 * `wide::f32x8` lanes: lane l accumulates a[8c+l]*b[8c+l]; the default x86-64
 * target has no FMA feature, so mul_add is a multiply then an add.  The lanes
 * are then summed (reduce_add) and the scalar tail added in order. ---------- */
static float dot8(const float *a, const float *b, int64_t len) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int64_t c = 0;
    for (; c + 8 <= len; c += 8)
        for (int l = 0; l < 8; l++) acc[l] = a[c + l] * b[c + l] + acc[l];
    /* reduce_add: pairwise halves (order is last-ULP unpinned) */
    float s4[4], s2[2];
    for (int l = 0; l < 4; l++) s4[l] = acc[l] + acc[l + 4];
    for (int l = 0; l < 2; l++) s2[l] = s4[l] + s4[l + 2];
    float sum = s2[0] + s2[1];
    for (; c < len; c++) sum += a[c] * b[c];
    return sum;
}

typedef struct {
    const float *a, *b;
    int64_t k, n;
} nt_ctx;

static void nt_row(void *vctx, int64_t i, float *row) {
    nt_ctx *c = (nt_ctx *)vctx;
    const float *ar = c->a + i * c->k;
    for (int64_t j = 0; j < c->n; j++) row[j] = dot8(ar, c->b + j * c->k, c->k);
}

void arfo_matmul_nt(const float *a, int64_t m, int64_t k, const float *b, int64_t n, float *out) {
    nt_ctx c = {a, b, k, n};
    par_rows(out, n, m, nt_row, &c);
}

/* ---- a8: Q8_0 matmul.  crates/arf-ml/src/matmul.rs:174-204 ---------------- */
typedef struct {
    const float *a;
    const uint8_t *blocks;
    int64_t k, n;
} q8_ctx;

static void q8_row(void *vctx, int64_t i, float *row) {
    q8_ctx *c = (q8_ctx *)vctx;
    int64_t bpr = c->k / 32;
    const float *ar = c->a + i * c->k;
    for (int64_t j = 0; j < c->n; j++) {
        float acc = 0.0f;
        for (int64_t blk = 0; blk < bpr; blk++) {
            const uint8_t *p = c->blocks + (j * bpr + blk) * 34;
            float d = arfo_f16_to_f32(rd16(p));
            const uint8_t *qs = p + 2;
            int64_t xb = blk * 32;
            float bsum = 0.0f;
            for (int t = 0; t < 32; t++) bsum += ar[xb + t] * (float)(int8_t)qs[t];
            acc += d * bsum;
        }
        row[j] = acc;
    }
}

void arfo_matmul_nt_q8_0(const float *a, int64_t m, int64_t k, const uint8_t *blocks, int64_t n,
                         float *out) {
    q8_ctx c = {a, blocks, k, n};
    par_rows(out, n, m, q8_row, &c);
}

/* ---- a7: Q4_K_S matmul.  crates/arf-ml/src/matmul.rs:322-400 -------------- */
typedef struct {
    const float *a;
    const uint32_t *codes;
    const uint8_t *scales;
    const int8_t *mins;
    const float *d, *dmin;
    int64_t k, n;
} q4ks_ctx;

static float dot_q4ks(const float *x, const uint32_t *codes, const uint8_t *scales,
                      const int8_t *mins, const float *d, const float *dmin, int64_t k) {
    int64_t subs = k / 32;
    float sum = 0.0f;
    for (int64_t sb = 0; sb < subs; sb++) {
        int64_t sblk = sb / 8;
        float s = d[sblk] * (float)scales[sb];
        float lo = dmin[sblk] * (float)mins[sb];
        float code_sum = 0.0f, x_sum = 0.0f;
        for (int w = 0; w < 4; w++) {
            uint32_t word = codes[sb * 4 + w];
            int64_t xb = sb * 32 + w * 8;
            for (int j = 0; j < 8; j++) {
                float code = (float)((word >> (j * 4)) & 0xF);
                float xv = x[xb + j];
                code_sum += xv * code;
                x_sum += xv;
            }
        }
        sum += s * code_sum + lo * x_sum;
    }
    return sum;
}

static void q4ks_row(void *vctx, int64_t i, float *row) {
    q4ks_ctx *c = (q4ks_ctx *)vctx;
    int64_t wpr = c->k / 8, spr = c->k / 32, ppr = c->k / QK_K;
    const float *ar = c->a + i * c->k;
    for (int64_t j = 0; j < c->n; j++)
        row[j] = dot_q4ks(ar, c->codes + j * wpr, c->scales + j * spr, c->mins + j * spr,
                          c->d + j * ppr, c->dmin + j * ppr, c->k);
}

void arfo_matmul_nt_q4ks(const float *a, int64_t m, int64_t k, const uint32_t *codes,
                         const uint8_t *scales, const int8_t *mins, const float *d,
                         const float *dmin, int64_t n, float *out) {
    q4ks_ctx c = {a, codes, scales, mins, d, dmin, k, n};
    par_rows(out, n, m, q4ks_row, &c);
}

/* Convenience used by the tests: ggml Q4_K blocks -> transcode -> matmul_nt_q4ks,
 * which is the reference's Linear::forward on a Q4_K GGUF tensor
 * (crates/arf-core/src/model/weights.rs:478-500 then nn.rs:22-32). */
void arfo_matmul_nt_q4_k(const float *a, int64_t m, int64_t k, const uint8_t *blocks, int64_t n,
                        float *out) {
    int64_t subs = n * (k / 32), supers = n * (k / QK_K);
    uint32_t *codes = (uint32_t *)malloc((size_t)(n * k / 8) * 4);
    uint8_t *scales = (uint8_t *)malloc((size_t)subs);
    int8_t *mins = (int8_t *)malloc((size_t)subs);
    float *d = (float *)malloc((size_t)supers * 4);
    float *dmin = (float *)malloc((size_t)supers * 4);
    arfo_q4ks_from_ggml(blocks, n, k, codes, scales, mins, d, dmin);
    arfo_matmul_nt_q4ks(a, m, k, codes, scales, mins, d, dmin, n, out);
    free(codes);
    free(scales);
    free(mins);
    free(d);
    free(dmin);
}

/* Q6_K reference matmul: dequant_q6_k then matmul_nt (the reference has no native
 * Q6_K matmul; crates/arf-core/src/model/gguf.rs:2092-2131 then matmul.rs:84-99). */
void arfo_matmul_nt_q6_k(const float *a, int64_t m, int64_t k, const uint8_t *blocks, int64_t n,
                         float *out) {
    float *w = (float *)malloc((size_t)(n * k) * 4);
    arfo_dequant_q6_k(blocks, n * k, w);
    arfo_matmul_nt(a, m, k, w, n, out);
    free(w);
}

/* Q5_K reference matmul: dequant_q5_k then matmul_nt (the CPU path reads a Q5_K
 * tensor through its f32 dequant; crates/arf-core/src/model/gguf.rs:2053-2090 then
 * matmul.rs:84-99). */
void arfo_matmul_nt_q5_k(const float *a, int64_t m, int64_t k, const uint8_t *blocks, int64_t n,
                         float *out) {
    float *w = (float *)malloc((size_t)(n * k) * 4);
    arfo_dequant_q5_k(blocks, n * k, w);
    arfo_matmul_nt(a, m, k, w, n, out);
    free(w);
}

/* ---- a10: top-k softmax routing.  crates/arf-core/src/model/moe.rs:89-121.
 * Full softmax, stable sort by probability (descending, ties -> lower index),
 * truncate to k, optional renormalisation (only when the sum is > 0). ------ */
void arfo_top_k_softmax(const float *logits, int n, int top_k, int norm_topk, int32_t *ids,
                        float *weights) {
    int k = top_k < n ? top_k : n;
    float mx = -INFINITY;
    for (int i = 0; i < n; i++) mx = fmaxf(mx, logits[i]);
    float *probs = (float *)malloc(sizeof(float) * (size_t)n);
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        probs[i] = expf(logits[i] - mx);
    }
    for (int i = 0; i < n; i++) sum += probs[i];
    for (int i = 0; i < n; i++) probs[i] = probs[i] / sum;
    /* selection of the k best in (prob desc, index asc) order == stable sort + truncate */
    char *taken = (char *)calloc((size_t)n, 1);
    for (int t = 0; t < k; t++) {
        int best = -1;
        for (int i = 0; i < n; i++) {
            if (taken[i]) continue;
            if (best < 0 || probs[i] > probs[best]) best = i;
        }
        taken[best] = 1;
        ids[t] = best;
        weights[t] = probs[best];
    }
    if (norm_topk) {
        float s = 0.0f;
        for (int t = 0; t < k; t++) s += weights[t];
        if (s > 0.0f)
            for (int t = 0; t < k; t++) weights[t] /= s;
    }
    free(taken);
    free(probs);
}

/* silu: crates/arf-ml/src/lib.rs:160-162  x / (1 + exp(-x)) */
static float silu(float x) { return x / (1.0f + expf(-x)); }

/* gelu_tanh with the inner clamp: crates/arf-gpu/src/shaders/metal/decode_ops_msl.metal:15-27,
 * the same expression as its CPU oracle crates/arf-gpu/src/gpu/metal/selftest.rs:6091-6095
 * (inner = (C * (x + 0.044715 x^3)).clamp(-15, 15), 0.5 x (1 + tanh(inner))).  Rust's
 * f32::clamp keeps a NaN; so do the comparisons below. */
static float gelu_tanh(float x) {
    const float C = 0.7978845608028654f; /* sqrt(2/pi); the selftest's 0.797_884_6 is the same f32 */
    float inner = C * (x + 0.044715f * x * x * x);
    if (inner < -15.0f) inner = -15.0f;
    if (inner > 15.0f) inner = 15.0f;
    return 0.5f * x * (1.0f + tanhf(inner));
}

/* The gated FFN activation h = act(g) * u over n elements: act 0 SwiGLU
 * (mlp.rs:20-24 with silu above), act 1 GeGLU (decode_ops_msl.metal:15-27). */
void arfo_glu(const float *g, const float *u, int64_t n, int act, float *out) {
    for (int64_t i = 0; i < n; i++) out[i] = (act ? gelu_tanh(g[i]) : silu(g[i])) * u[i];
}

/* ---- a11/a12: SwiGLU expert + MoE block.  crates/arf-core/src/model/mlp.rs:20-24,
 * crates/arf-core/src/model/moe.rs:53-86.  Experts are Q4_K (transcoded to
 * Q4_K_S, so every projection is matmul_nt_q4ks).  The router Linear is replaced
 * by the given logits.  Tokens run serially; each selected expert runs on the
 * single token row (m = 1); `out[t] += w_j * expert_j(x_t)` in top-k order.
 * gate/up: [n_experts][inter rows][hidden] Q4_K blocks; down: [n_experts][hidden
 * rows][inter] Q4_K blocks. ---------------------------------------------------- */
void arfo_moe_forward(const float *x, int64_t tokens, int64_t hidden, int64_t inter,
                      const uint8_t *gate, const uint8_t *up, const uint8_t *down,
                      int n_experts, const float *logits, int top_k, int norm_topk, int accumulate,
                      float *out) {
    int64_t gu_bytes = inter * (hidden / QK_K) * 144;  /* one expert's gate (or up) */
    int64_t dn_bytes = hidden * (inter / QK_K) * 144;  /* one expert's down */
    float *g = (float *)malloc(sizeof(float) * (size_t)inter);
    float *u = (float *)malloc(sizeof(float) * (size_t)inter);
    float *y = (float *)malloc(sizeof(float) * (size_t)hidden);
    int32_t *ids = (int32_t *)malloc(sizeof(int32_t) * (size_t)top_k);
    float *wts = (float *)malloc(sizeof(float) * (size_t)top_k);
    /* out starts at 0; with accumulate it holds the shared experts' sum, which the
     * reference adds first (moe.rs:62-67; 0 + s == s exactly) */
    if (!accumulate) memset(out, 0, sizeof(float) * (size_t)(tokens * hidden));
    for (int64_t t = 0; t < tokens; t++) {
        arfo_top_k_softmax(logits + t * n_experts, n_experts, top_k, norm_topk, ids, wts);
        int k = top_k < n_experts ? top_k : n_experts;
        const float *xt = x + t * hidden;
        for (int j = 0; j < k; j++) {
            int e = ids[j];
            arfo_matmul_nt_q4_k(xt, 1, hidden, gate + e * gu_bytes, inter, g);
            arfo_matmul_nt_q4_k(xt, 1, hidden, up + e * gu_bytes, inter, u);
            for (int64_t i = 0; i < inter; i++) g[i] = silu(g[i]) * u[i];
            arfo_matmul_nt_q4_k(g, 1, inter, down + e * dn_bytes, hidden, y);
            float *dst = out + t * hidden;
            for (int64_t i = 0; i < hidden; i++) dst[i] += wts[j] * y[i];
        }
    }
    free(g);
    free(u);
    free(y);
    free(ids);
    free(wts);
}
