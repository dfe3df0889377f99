/*
 * sgo — CPU oracle for the super-gemma quantized compute core.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is a plain-C restatement of the
 * reference's CPU ground truth (Rust, not buildable here: no rustc/cargo in
 * the image).  It exists so that tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py can CHECK the HIP library; the product path
 * (libsgq) never links, loads or calls it.
 *
 * Every function names the reference file:line it restates.  Pinning (what
 * checks each function against something other than itself) lives in
 * tests/test_oracle.py; a function with no such check would be marked
 * "parity unpinned" here — currently there is none.
 *
 * Conventions: f16 values travel as raw uint16_t bits; Q4_0 weights are the
 * GGUF byte stream (18-byte blocks: f16 d, 16 nibble bytes); Q8_0 is the
 * structure-of-arrays page format (f16 scales[nblk], int8 quants[n]).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define QK 32
#define Q4_BLOCK_BYTES 18

/* ------------------------------------------------------------------------ */
/* RNG: xorshift64* — crates/sg-gpu/tests/reference/mod.rs:7-32             */
/* ------------------------------------------------------------------------ */

uint64_t sgo_rng_seed(uint64_t seed) { return seed ? seed : 1; } /* seed.max(1) */

uint64_t sgo_rng_next(uint64_t *s) {
    uint64_t x = *s;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *s = x;
    return x * 0x2545F4914F6CDD1DULL;
}

/* Uniform in [-2, 2): (next >> 40) / 2^24 * 4 - 2, each step in f32. */
float sgo_rng_f32(uint64_t *s) {
    float a = (float)(sgo_rng_next(s) >> 40);
    float v = a / 16777216.0f;
    v = v * 4.0f;
    return v - 2.0f;
}

/* Fills n values; returns the advanced state (mod.rs:28-30 f32_vec). */
uint64_t sgo_rng_f32_vec(uint64_t state, float *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = sgo_rng_f32(&state);
    return state;
}

uint64_t sgo_rng_u64_vec(uint64_t state, uint64_t *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = sgo_rng_next(&state);
    return state;
}

/* ------------------------------------------------------------------------ */
/* IEEE binary16 with round-to-nearest-even (the `half` crate 2.7.1 used by  */
/* mod.rs:36-52 through_f16 / to_f16_bits / from_f16_bits).                 */
/* ------------------------------------------------------------------------ */

uint16_t sgo_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) { /* inf / nan */
        if (ax == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    }
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 → inf */
    if (ax < 0x38800000u) {                                      /* below 2^-14 */
        if (ax < 0x33000000u) return (uint16_t)sign;             /* <= 2^-25 → 0 */
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - e; /* units of 2^-24 */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (ax >> 23) - 127u + 15u;
    uint32_t m = ax & 0x7fffffu;
    uint32_t q = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

float sgo_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t out;
    if (e == 0) {
        if (m == 0) {
            out = sign;
        } else { /* subnormal: m * 2^-24 */
            float v = (float)m * (1.0f / 16777216.0f);
            memcpy(&out, &v, 4);
            out |= sign;
        }
    } else if (e == 31) {
        out = sign | 0x7f800000u | (m << 13);
    } else {
        out = sign | ((e - 15u + 127u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &out, 4);
    return f;
}

void sgo_f32_to_f16_vec(const float *x, uint16_t *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = sgo_f32_to_f16(x[i]);
}

void sgo_f16_to_f32_vec(const uint16_t *x, float *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = sgo_f16_to_f32(x[i]);
}

/* through_f16 (mod.rs:36-40) in place. */
void sgo_through_f16(float *x, size_t n) {
    for (size_t i = 0; i < n; i++) x[i] = sgo_f16_to_f32(sgo_f32_to_f16(x[i]));
}

/* ------------------------------------------------------------------------ */
/* Q4_0 — crates/sg-gguf/src/q4_0.rs:31-42                                  */
/* ------------------------------------------------------------------------ */

/* w[j] = d*((qs[j]&15)-8), w[j+16] = d*((qs[j]>>4)-8); d is f16 widened to
 * f32, the product is a single f32 multiply (exact: 11-bit × 4-bit). */
void sgo_q4_0_dequant_block(const uint8_t *blk, float *out) {
    uint16_t dbits = (uint16_t)(blk[0] | (blk[1] << 8));
    float d = sgo_f16_to_f32(dbits);
    const uint8_t *qs = blk + 2;
    for (int j = 0; j < 16; j++) {
        int lo = (qs[j] & 0x0f) - 8;
        int hi = (qs[j] >> 4) - 8;
        out[j] = d * (float)lo;
        out[j + 16] = d * (float)hi;
    }
}

/* dequant_row (crates/sg-model/src/reference.rs:447-462, the Q4_0 arm). */
void sgo_q4_0_dequant_rows(const uint8_t *w, size_t n_rows, size_t k, float *out) {
    size_t nb = k / QK;
    for (size_t r = 0; r < n_rows; r++)
        for (size_t b = 0; b < nb; b++)
            sgo_q4_0_dequant_block(w + (r * nb + b) * Q4_BLOCK_BYTES, out + r * k + b * QK);
}

/* random_q4_0 (crates/sg-gpu/tests/parity_gemv.rs:23-33): per block
 * d = f16(rng.f32()*0.05), then 16 bytes of next_u64() & 0xFF. */
uint64_t sgo_random_q4_0(uint64_t state, uint8_t *out, size_t n_blocks) {
    for (size_t b = 0; b < n_blocks; b++) {
        float v = sgo_rng_f32(&state) * 0.05f;
        uint16_t d = sgo_f32_to_f16(v);
        uint8_t *blk = out + b * Q4_BLOCK_BYTES;
        blk[0] = (uint8_t)(d & 0xff);
        blk[1] = (uint8_t)(d >> 8);
        for (int j = 0; j < 16; j++) blk[2 + j] = (uint8_t)(sgo_rng_next(&state) & 0xff);
    }
    return state;
}

/* ------------------------------------------------------------------------ */
/* Q6_K — crates/sg-gguf/src/q6_k.rs:41-62 (ggml dequantize_row_q6_K)       */
/* block: ql[128] low nibbles, qh[64] 2-bit highs, int8 scales[16], f16 d   */
/* ------------------------------------------------------------------------ */

#define Q6K_BLOCK_BYTES 210
#define Q6K_WEIGHTS 256

/* w = d * scale[sub] * (q - 32), one f32 product chain d*sc*q as in the
 * reference (d widened to f32, sc and q converted to f32). */
void sgo_q6_k_dequant_block(const uint8_t *blk, float *out) {
    const uint8_t *ql0 = blk, *qh0 = blk + 128;
    const int8_t *sc0 = (const int8_t *)(blk + 192);
    const float d = sgo_f16_to_f32((uint16_t)(blk[208] | (blk[209] << 8)));
    for (int half = 0; half < 2; half++) {
        const uint8_t *ql = ql0 + half * 64, *qh = qh0 + half * 32;
        const int8_t *sc = sc0 + half * 8;
        float *y = out + half * 128;
        for (int l = 0; l < 32; l++) {
            const int is = l / 16;
            const int q1 = ((ql[l] & 0x0F) | ((qh[l] & 0x03) << 4)) - 32;
            const int q2 = ((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 0x03) << 4)) - 32;
            const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 0x03) << 4)) - 32;
            const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 0x03) << 4)) - 32;
            y[l] = d * (float)sc[is] * (float)q1;
            y[l + 32] = d * (float)sc[is + 2] * (float)q2;
            y[l + 64] = d * (float)sc[is + 4] * (float)q3;
            y[l + 96] = d * (float)sc[is + 6] * (float)q4;
        }
    }
}

/* Rows of k/256 blocks at a byte stride (the GPU layout pads rows). */
void sgo_q6_k_dequant_rows(const uint8_t *w, size_t row_stride, size_t n_rows, size_t k,
                           float *out) {
    const size_t nb = k / Q6K_WEIGHTS;
    for (size_t r = 0; r < n_rows; r++)
        for (size_t b = 0; b < nb; b++)
            sgo_q6_k_dequant_block(w + r * row_stride + b * Q6K_BLOCK_BYTES,
                                   out + r * k + b * Q6K_WEIGHTS);
}

/* random_q6k_rows (crates/sg-gpu/tests/parity_logits.rs:31-51): every byte
 * of a row's blocks = next_u64() & 0xFF; then per block the 16 sub-scales
 * become (s & 0x0F) - 8 and d = f16(f32() * 1e-3).  Padding stays 0. */
uint64_t sgo_random_q6_k_rows(uint64_t state, uint8_t *out, size_t n_rows, size_t k,
                              size_t row_stride) {
    const size_t nb = k / Q6K_WEIGHTS, row_bytes = nb * Q6K_BLOCK_BYTES;
    memset(out, 0, n_rows * row_stride);
    for (size_t r = 0; r < n_rows; r++) {
        uint8_t *row = out + r * row_stride;
        for (size_t i = 0; i < row_bytes; i++) row[i] = (uint8_t)(sgo_rng_next(&state) & 0xff);
        for (size_t b = 0; b < nb; b++) {
            uint8_t *blk = row + b * Q6K_BLOCK_BYTES;
            for (int s = 192; s < 208; s++) blk[s] = (uint8_t)(int8_t)((int)(blk[s] & 0x0F) - 8);
            const uint16_t d = sgo_f32_to_f16(sgo_rng_f32(&state) * 1e-3f);
            blk[208] = (uint8_t)(d & 0xff);
            blk[209] = (uint8_t)(d >> 8);
        }
    }
    return state;
}

/* gemv_q6_k_logits reference (crates/sg-gpu/tests/parity_logits.rs:84-98):
 * f64 dot of each dequantized row with x, then softcap*tanh(dot/softcap)
 * (softcap <= 0: the raw dot). */
void sgo_gemv_q6_k_logits(const uint8_t *w, size_t row_stride, const float *x, size_t n,
                          size_t k, double softcap, float *y) {
    const size_t nb = k / Q6K_WEIGHTS;
    float deq[Q6K_WEIGHTS];
    for (size_t r = 0; r < n; r++) {
        double dot = 0.0;
        for (size_t b = 0; b < nb; b++) {
            sgo_q6_k_dequant_block(w + r * row_stride + b * Q6K_BLOCK_BYTES, deq);
            for (int j = 0; j < Q6K_WEIGHTS; j++) dot += (double)deq[j] * (double)x[b * Q6K_WEIGHTS + j];
        }
        y[r] = (float)(softcap > 0.0 ? softcap * tanh(dot / softcap) : dot);
    }
}

/* ------------------------------------------------------------------------ */
/* GEMV oracle: f64 dot over dequantized rows                               */
/* (crates/sg-gpu/tests/parity_gemv.rs:37-55 reference_rows)                */
/* ------------------------------------------------------------------------ */

void sgo_gemv_q4_0_rows(const uint8_t *w, const float *x, size_t k, const int64_t *rows,
                        size_t n_rows, float *y) {
    size_t nb = k / QK;
    float deq[QK];
    for (size_t i = 0; i < n_rows; i++) {
        const uint8_t *row = w + (size_t)rows[i] * nb * Q4_BLOCK_BYTES;
        double acc = 0.0;
        for (size_t b = 0; b < nb; b++) {
            sgo_q4_0_dequant_block(row + b * Q4_BLOCK_BYTES, deq);
            for (int j = 0; j < QK; j++) acc += (double)deq[j] * (double)x[b * QK + j];
        }
        y[i] = (float)acc;
    }
}

/* ------------------------------------------------------------------------ */
/* CPU baseline: CpuModel matmul (crates/sg-model/src/reference.rs:402-444) */
/* dequant_row, then dot_f64 with 8 independent f64 lanes merged in fixed    */
/* order, plus a sequential tail; row-parallel (rayon there, pthreads here). */
/* ------------------------------------------------------------------------ */

double sgo_dot_f64(const float *a, const float *b, size_t n) {
    double acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t n8 = n / 8 * 8;
    for (size_t i = 0; i < n8; i += 8)
        for (int j = 0; j < 8; j++) acc[j] += (double)a[i + j] * (double)b[i + j];
    double sum = 0.0;
    for (int j = 0; j < 8; j++) sum += acc[j]; /* acc.iter().sum(): left fold from 0 */
    for (size_t i = n8; i < n; i++) sum += (double)a[i] * (double)b[i];
    return sum;
}

typedef struct {
    const uint8_t *w;
    const float *x;
    float *y;
    size_t n_tokens, n_out, n_in;
    size_t r0, r1;
} mm_job;

static void *mm_worker(void *arg) {
    mm_job *j = (mm_job *)arg;
    float *row = (float *)malloc(j->n_in * sizeof(float));
    size_t nb = j->n_in / QK;
    for (size_t r = j->r0; r < j->r1; r++) {
        sgo_q4_0_dequant_rows(j->w + r * nb * Q4_BLOCK_BYTES, 1, j->n_in, row);
        for (size_t t = 0; t < j->n_tokens; t++)
            j->y[t * j->n_out + r] = (float)sgo_dot_f64(row, j->x + t * j->n_in, j->n_in);
    }
    free(row);
    return NULL;
}

/* y[t][r] = dot_f64(dequant_row(W, r), x[t]); rows split over `threads`. */
void sgo_matmul_q4_0(const uint8_t *w, const float *x, size_t n_tokens, size_t n_out,
                     size_t n_in, float *y, int threads) {
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    pthread_t tid[256];
    mm_job jobs[256];
    size_t per = (n_out + (size_t)threads - 1) / (size_t)threads;
    int started = 0;
    for (int t = 0; t < threads; t++) {
        size_t r0 = (size_t)t * per, r1 = r0 + per;
        if (r0 >= n_out) break;
        if (r1 > n_out) r1 = n_out;
        jobs[t] = (mm_job){w, x, y, n_tokens, n_out, n_in, r0, r1};
        if (threads == 1) {
            mm_worker(&jobs[t]);
        } else {
            pthread_create(&tid[t], NULL, mm_worker, &jobs[t]);
            started++;
        }
    }
    for (int t = 0; t < started; t++) pthread_join(tid[t], NULL);
}

/* ------------------------------------------------------------------------ */
/* Q8_0                                                                     */
/* ------------------------------------------------------------------------ */

/* quant_q8_0 (mod.rs:272-286), the GPU kv_quant_q8 semantics
 * (shaders/kv_quant_q8.wgsl:41-56): per 32-block amax; d = amax*(1/127) in
 * f32; id = d>0 ? 1/d : 0 (from the UNROUNDED d); scale = f16(d) RTNE;
 * q = round_ties_even(x*id) as i8 (Rust's saturating cast). */
void sgo_quant_q8_0(const float *x, size_t n, uint16_t *scales, int8_t *quants) {
    const float inv127 = 1.0f / 127.0f;
    for (size_t b = 0; b < n / QK; b++) {
        const float *blk = x + b * QK;
        float amax = 0.0f;
        for (int i = 0; i < QK; i++) {
            float a = fabsf(blk[i]);
            amax = a > amax ? a : amax; /* f32::max; inputs are finite */
        }
        float d = amax * inv127;
        float id = d > 0.0f ? 1.0f / d : 0.0f;
        scales[b] = sgo_f32_to_f16(d);
        for (int i = 0; i < QK; i++) {
            float r = rintf(blk[i] * id); /* default FE_TONEAREST: ties-even */
            if (r > 127.0f) r = 127.0f;
            if (r < -128.0f) r = -128.0f;
            quants[b * QK + i] = (int8_t)r;
        }
    }
}

/* q8_quant (mod.rs:58-79): the division-scale variant with an explicit
 * clamp, plus the dequant through the f16-rounded scale. */
void sgo_q8_quant_div(const float *x, size_t n, uint16_t *scales, int8_t *quants, float *deq) {
    for (size_t b = 0; b < n / QK; b++) {
        const float *blk = x + b * QK;
        float amax = 0.0f;
        for (int i = 0; i < QK; i++) {
            float a = fabsf(blk[i]);
            amax = a > amax ? a : amax;
        }
        float d = amax / 127.0f;
        float id = d > 0.0f ? 1.0f / d : 0.0f;
        uint16_t d16 = sgo_f32_to_f16(d);
        scales[b] = d16;
        float dd = sgo_f16_to_f32(d16);
        for (int i = 0; i < QK; i++) {
            float r = rintf(blk[i] * id);
            int q = (int)r;
            if (q < -128) q = -128;
            if (q > 127) q = 127;
            quants[b * QK + i] = (int8_t)q;
            deq[b * QK + i] = dd * (float)q;
        }
    }
}

/* q8_quant_v (mod.rs:98-134): V quantized in 32-KEY blocks per (head, col);
 * quants keep the [keys × heads × hd] layout, scales are
 * [ceil(keys/32) × heads × hd]; a short final block covers the live keys. */
void sgo_q8_quant_v(const float *v, size_t keys, size_t n_kv_heads, size_t head_dim,
                    int8_t *quants, uint16_t *scales, float *deq) {
    size_t row = n_kv_heads * head_dim;
    size_t kblk = (keys + 31) / 32;
    for (size_t h = 0; h < n_kv_heads; h++)
        for (size_t c = 0; c < head_dim; c++)
            for (size_t kb = 0; kb < kblk; kb++) {
                size_t k0 = kb * 32, k1 = k0 + 32 < keys ? k0 + 32 : keys;
                float amax = 0.0f;
                for (size_t key = k0; key < k1; key++) {
                    float a = fabsf(v[(key * n_kv_heads + h) * head_dim + c]);
                    amax = a > amax ? a : amax;
                }
                float d = amax / 127.0f;
                float id = d > 0.0f ? 1.0f / d : 0.0f;
                uint16_t d16 = sgo_f32_to_f16(d);
                scales[(kb * n_kv_heads + h) * head_dim + c] = d16;
                float dd = sgo_f16_to_f32(d16);
                for (size_t key = k0; key < k1; key++) {
                    size_t idx = (key * n_kv_heads + h) * head_dim + c;
                    int q = (int)rintf(v[idx] * id);
                    if (q < -128) q = -128;
                    if (q > 127) q = 127;
                    quants[idx] = (int8_t)q;
                    deq[idx] = dd * (float)q;
                }
            }
    (void)row;
}

/* dequant_q8_0 (mod.rs:291-299): x = f16(f16_d * q). */
void sgo_dequant_q8_0_f16(const uint16_t *scales, const int8_t *quants, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) {
        float d = sgo_f16_to_f32(scales[i / QK]);
        out[i] = sgo_f16_to_f32(sgo_f32_to_f16(d * (float)quants[i]));
    }
}

/* Plain Q8_0 dequant in f32: x = f32(d) * q (exact: 11-bit × 8-bit). */
void sgo_dequant_q8_0(const uint16_t *scales, const int8_t *quants, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) out[i] = sgo_f16_to_f32(scales[i / QK]) * (float)quants[i];
}

/* ------------------------------------------------------------------------ */
/* int8 MMQ — mmq_q4_0_q8 (mod.rs:311-340)                                  */
/* ------------------------------------------------------------------------ */

/* Exact i32 dot of one Q4_0 block with one Q8_0 block (mod.rs:327-335):
 * weight j<16 is lo nibble of qs[j], j>=16 the hi nibble of qs[j-16]. */
int32_t sgo_block_dot_q4_q8(const uint8_t *wblk, const int8_t *xq) {
    const uint8_t *qs = wblk + 2;
    int32_t dot = 0;
    for (int j = 0; j < 32; j++) {
        int wq = j < 16 ? (qs[j] & 0x0f) - 8 : (qs[j - 16] >> 4) - 8;
        dot += (int32_t)xq[j] * wq;
    }
    return dot;
}

/* Y[m][n] = sum_b f64(d_a)*f64(d_w)*dot, evaluated for the listed (m, n)
 * pairs only, from PRE-quantized activations (xq [M×K], xs [M×K/32]). */
void sgo_mmq_pairs(const uint8_t *w, const int8_t *xq, const uint16_t *xs, size_t k,
                   const int64_t *ms, const int64_t *ns, size_t n_pairs, float *y) {
    size_t nb = k / QK;
    for (size_t p = 0; p < n_pairs; p++) {
        size_t mi = (size_t)ms[p], ni = (size_t)ns[p];
        const uint8_t *row = w + ni * nb * Q4_BLOCK_BYTES;
        double acc = 0.0;
        for (size_t b = 0; b < nb; b++) {
            const uint8_t *blk = row + b * Q4_BLOCK_BYTES;
            double da = (double)sgo_f16_to_f32(xs[mi * nb + b]);
            double dw = (double)sgo_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
            int32_t dot = sgo_block_dot_q4_q8(blk, xq + mi * k + b * QK);
            acc += da * dw * (double)dot;
        }
        y[p] = (float)acc;
    }
}

/* Full mmq_q4_0_q8: quantizes each X row with quant_q8_0, then the above. */
void sgo_mmq_q4_0_q8(const uint8_t *w, const float *x, size_t m, size_t k, size_t n, float *y) {
    size_t nb = k / QK;
    int8_t *xq = (int8_t *)malloc(m * k);
    uint16_t *xs = (uint16_t *)malloc(m * nb * sizeof(uint16_t));
    sgo_quant_q8_0(x, m * k, xs, xq);
    for (size_t mi = 0; mi < m; mi++)
        for (size_t ni = 0; ni < n; ni++) {
            int64_t a = (int64_t)mi, b = (int64_t)ni;
            sgo_mmq_pairs(w, xq, xs, k, &a, &b, 1, y + mi * n + ni);
        }
    free(xq);
    free(xs);
}

/* Per-block i32 dots for one (m, n) pair: out[b] for b < K/32. */
void sgo_mmq_block_dots(const uint8_t *w, const int8_t *xq, size_t k, size_t mi, size_t ni,
                        int32_t *out) {
    size_t nb = k / QK;
    const uint8_t *row = w + ni * nb * Q4_BLOCK_BYTES;
    for (size_t b = 0; b < nb; b++)
        out[b] = sgo_block_dot_q4_q8(row + b * Q4_BLOCK_BYTES, xq + mi * k + b * QK);
}

/* ------------------------------------------------------------------------ */
/* Elementwise ops                                                          */
/* ------------------------------------------------------------------------ */

/* rmsnorm (mod.rs:156-172): f64 sum of squares, inv = 1/sqrt(ss/len+eps),
 * out = f32(v*inv*weight) in f64; w == NULL is the weightless V-norm
 * (crates/sg-model/src/reference.rs:367-383). */
void sgo_rmsnorm(const float *x, const float *w, size_t rows, size_t row_len, double eps,
                 int plus_one, float *out) {
    for (size_t r = 0; r < rows; r++) {
        const float *row = x + r * row_len;
        double ss = 0.0;
        for (size_t i = 0; i < row_len; i++) ss += (double)row[i] * (double)row[i];
        double inv = 1.0 / sqrt(ss / (double)row_len + eps);
        for (size_t i = 0; i < row_len; i++) {
            double weight = w ? (plus_one ? 1.0 + (double)w[i] : (double)w[i]) : 1.0;
            out[r * row_len + i] = (float)((double)row[i] * inv * weight);
        }
    }
}

/* cos_sin_table (crates/sg-model/src/rope.rs:27-48): angle in f64 =
 * pos * theta^(-2i/head_dim) / factor[i]; stored (cos, sin) as f32,
 * [position × head_dim/2 × 2]. factors == NULL means all 1. */
void sgo_cos_sin_table(const uint32_t *positions, size_t n_pos, size_t head_dim, float theta,
                       const float *factors, float *out) {
    size_t half = head_dim / 2;
    for (size_t p = 0; p < n_pos; p++)
        for (size_t i = 0; i < half; i++) {
            double freq = pow((double)theta, -2.0 * (double)i / (double)head_dim);
            double factor = factors ? (double)factors[i] : 1.0;
            double angle = (double)positions[p] * freq / factor;
            out[(p * half + i) * 2] = (float)cos(angle);
            out[(p * half + i) * 2 + 1] = (float)sin(angle);
        }
}

/* rope (mod.rs:198-216): NEOX pairing over the full head, pair i couples
 * (i, i+head_dim/2), first rot_dims/2 pairs live; f64 math per element;
 * table [token × rot_dims/2 × 2]; rows [token × n_heads × head_dim]. */
void sgo_rope(float *x, size_t n_rows, size_t head_dim, size_t rot_dims, size_t n_heads,
              const float *cos_sin) {
    size_t live = rot_dims / 2, partner = head_dim / 2;
    for (size_t r = 0; r < n_rows; r++) {
        float *row = x + r * head_dim;
        size_t token = r / n_heads;
        for (size_t p = 0; p < live; p++) {
            double c = cos_sin[(token * live + p) * 2];
            double s = cos_sin[(token * live + p) * 2 + 1];
            double a = row[p], b = row[p + partner];
            row[p] = (float)(a * c - b * s);
            row[p + partner] = (float)(b * c + a * s);
        }
    }
}

/* apply_rope (crates/sg-model/src/rope.rs:54-64): the f32 form. */
void sgo_apply_rope_f32(float *row, size_t head_dim, const float *cs) {
    size_t half = head_dim / 2;
    for (size_t i = 0; i < half; i++) {
        float c = cs[2 * i], s = cs[2 * i + 1];
        float a = row[i], b = row[i + half];
        row[i] = a * c - b * s;
        row[i + half] = b * c + a * s;
    }
}

/* gelu_tanh (crates/sg-model/src/reference.rs:533-537). */
float sgo_gelu_tanh(float xf) {
    const double k = 0.7978845608028654;
    double x = xf;
    return (float)(0.5 * x * (1.0 + tanh(k * (x + 0.044715 * x * x * x))));
}

/* geglu (mod.rs:343-352): gelu_tanh(g)*u, f64. */
void sgo_geglu(const float *g, const float *u, size_t n, float *out) {
    const double k = 0.7978845608028654; /* (2/pi)^0.5 */
    for (size_t i = 0; i < n; i++) {
        double x = g[i];
        double inner = k * (x + 0.044715 * x * x * x);
        out[i] = (float)(0.5 * x * (1.0 + tanh(inner)) * (double)u[i]);
    }
}

/* add_scaled (crates/sg-gpu/shaders/add_scaled.wgsl:21-27): (a+b)*s in f32. */
void sgo_add_scaled(const float *a, const float *b, size_t n, float s, float *out) {
    for (size_t i = 0; i < n; i++) out[i] = (a[i] + b[i]) * s;
}

/* ------------------------------------------------------------------------ */
/* Attention                                                                */
/* ------------------------------------------------------------------------ */

/* attention_head (mod.rs:224-263): full softmax over keys [t0, t1], f64;
 * GQA kv head = qh / (n_q/n_kv); q [m × n_q × hd], k/v [L × n_kv × hd]. */
void sgo_attention_head(const float *q, const float *k, const float *v, size_t i, size_t qh,
                        size_t n_q_heads, size_t n_kv_heads, size_t head_dim, double scale,
                        size_t t0, size_t t1, float *out) {
    size_t kvh = qh / (n_q_heads / n_kv_heads);
    const float *qrow = q + (i * n_q_heads + qh) * head_dim;
    size_t n = t1 - t0 + 1;
    double *sc = (double *)malloc(n * sizeof(double));
    double mx = -INFINITY;
    for (size_t t = t0; t <= t1; t++) {
        const float *krow = k + (t * n_kv_heads + kvh) * head_dim;
        double dot = 0.0;
        for (size_t d = 0; d < head_dim; d++) dot += (double)qrow[d] * (double)krow[d];
        sc[t - t0] = dot * scale;
        if (sc[t - t0] > mx) mx = sc[t - t0];
    }
    double denom = 0.0;
    for (size_t j = 0; j < n; j++) {
        sc[j] = exp(sc[j] - mx);
        denom += sc[j];
    }
    for (size_t d = 0; d < head_dim; d++) {
        double acc = 0.0;
        for (size_t t = t0; t <= t1; t++)
            acc += sc[t - t0] * (double)v[(t * n_kv_heads + kvh) * head_dim + d];
        out[d] = (float)(acc / denom);
    }
    free(sc);
}

/* attention_head with the int8-PV quantization of
 * attn_prefill_global_flash_sp_ipv.wgsl:134-181: P = exp(s - max) is
 * quantized per 32-KEY block (blocks of absolute key index t/32, restricted
 * to [t0, t1]): d = amax*(1/127) in f32, id = 1/d, scale f16(d),
 * q = clamp(round(p*id)), p~ = f16(d)*q; the denominator sums the
 * dequantized p~ as the numerator does (ipv.wgsl:157-177); V is the
 * dequantized key-blocked V the kernel multiplies. */
void sgo_attention_head_ipv(const float *q, const float *k, const float *v, size_t i, size_t qh,
                            size_t n_q_heads, size_t n_kv_heads, size_t head_dim, double scale,
                            size_t t0, size_t t1, float *out) {
    size_t kvh = qh / (n_q_heads / n_kv_heads);
    const float *qrow = q + (i * n_q_heads + qh) * head_dim;
    size_t n = t1 - t0 + 1;
    double *sc = (double *)malloc(n * sizeof(double));
    double mx = -INFINITY;
    for (size_t t = t0; t <= t1; t++) {
        const float *krow = k + (t * n_kv_heads + kvh) * head_dim;
        double dot = 0.0;
        for (size_t d = 0; d < head_dim; d++) dot += (double)qrow[d] * (double)krow[d];
        sc[t - t0] = dot * scale;
        if (sc[t - t0] > mx) mx = sc[t - t0];
    }
    for (size_t j = 0; j < n; j++) sc[j] = (double)(float)exp(sc[j] - mx);
    const float inv127 = 1.0f / 127.0f;
    for (size_t b0 = t0 / 32 * 32; b0 <= t1; b0 += 32) {
        size_t lo = b0 > t0 ? b0 : t0, hi = b0 + 31 < t1 ? b0 + 31 : t1;
        float amax = 0.0f;
        for (size_t t = lo; t <= hi; t++) {
            float p = (float)sc[t - t0];
            amax = p > amax ? p : amax;
        }
        float d = amax * inv127;
        float id = d > 0.0f ? 1.0f / d : 0.0f;
        float dd = sgo_f16_to_f32(sgo_f32_to_f16(d));
        for (size_t t = lo; t <= hi; t++) {
            int qi = (int)rintf((float)sc[t - t0] * id);
            if (qi < -128) qi = -128;
            if (qi > 127) qi = 127;
            sc[t - t0] = (double)dd * (double)qi;
        }
    }
    double denom = 0.0;
    for (size_t j = 0; j < n; j++) denom += sc[j];
    for (size_t d = 0; d < head_dim; d++) {
        double acc = 0.0;
        for (size_t t = t0; t <= t1; t++)
            acc += sc[t - t0] * (double)v[(t * n_kv_heads + kvh) * head_dim + d];
        out[d] = denom > 0.0 ? (float)(acc / denom) : 0.0f;
    }
    free(sc);
}

/* kv_append_global_v_q8.wgsl:32-75: append n_tok rows of V (fp32 [n_tok x
 * row], row = n_kv*hd) at positions pos.. (pos a multiple of 32) quantized
 * in 32-KEY blocks per column: global key block kb = pos/32 + t/32, one f16
 * scale per (kb, col) into scales[kb*row + col] (d = amax*(1/127), id = 1/d
 * of the unrounded d, round half to even), quants at [(pos+t)*row + col].
 * A short final block is quantized over its live rows. */
void sgo_kv_append_v_q8(const float *src, size_t n_tok, size_t row, size_t pos, int8_t *quants,
                        uint16_t *scales) {
    const float inv127 = 1.0f / 127.0f;
    for (size_t tb = 0; tb * 32 < n_tok; tb++) {
        size_t k0 = tb * 32, k1 = k0 + 32 < n_tok ? k0 + 32 : n_tok;
        size_t kb = pos / 32 + tb;
        for (size_t c = 0; c < row; c++) {
            float amax = 0.0f;
            for (size_t t = k0; t < k1; t++) {
                float a = fabsf(src[t * row + c]);
                amax = a > amax ? a : amax;
            }
            float d = amax * inv127;
            float id = d > 0.0f ? 1.0f / d : 0.0f;
            scales[kb * row + c] = sgo_f32_to_f16(d);
            for (size_t t = k0; t < k1; t++)
                quants[(pos + t) * row + c] = (int8_t)(int)rintf(src[t * row + c] * id);
        }
    }
}

/* attention (crates/sg-model/src/reference.rs:482-530): causal, optionally
 * windowed GQA over a linear cache; query t sits at q0+t and sees keys
 * [max(0, q0+t+1-window), q0+t]. window == 0 means no window. */
void sgo_attention(const float *q, const float *ck, const float *cv, size_t n, size_t q0,
                   size_t n_q_heads, size_t n_kv, size_t hd, size_t window, float scale,
                   float *out) {
    for (size_t t = 0; t < n; t++)
        for (size_t h = 0; h < n_q_heads; h++) {
            size_t qpos = q0 + t;
            size_t lo = window ? (qpos + 1 > window ? qpos + 1 - window : 0) : 0;
            sgo_attention_head(q, ck, cv, t, h, n_q_heads, n_kv, hd, (double)scale, lo, qpos,
                               out + (t * n_q_heads + h) * hd);
        }
}
