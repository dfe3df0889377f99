// Decode-step driver: the caller side of the hot path at the BASELINE shape
// (a random-init Gemma-4-style decoder, Q4_0 linears, Q8_0 KV cache).
//
// Semantics follow the reference's CPU model forward pass
// (crates/sg-model/src/reference.rs:157-316) and its GPU graph
// (crates/sg-model/src/graph.rs:478-756, record_layer / record_logits):
//   x = embed(token)·√hidden
//   per layer: xn = rmsnorm(x, attn_norm); q,k,v = Wq/Wk/Wv·xn;
//     q = rope(rmsnorm(q_h, q_norm)); k = rope(rmsnorm(k_h, k_norm));
//     v = rmsnorm(v_h) (weightless); append Q8_0(k), Q8_0(v) at the slot;
//     a = softmax(scale·q·kᵀ)·v over the window (sliding) or all (global);
//     x += rmsnorm(Wo·a, post_attention_norm);
//     f = Wd·(gelu_tanh(Wg·fn)·Wu·fn) with fn = rmsnorm(x, ffn_norm);
//     x = (x + rmsnorm(f, post_ffw_norm))·layer_output_scale
//   logits = softcap·tanh((E·rmsnorm(x, output_norm))/softcap), E tied.
// Shape deviations from the real checkpoint follow the benchmark's decoder:
// every layer has 32 q / 16 kv heads of dim 128, K and V pages are both
// Q8_0, and the tied head is Q4_0.  Global layers take V from the K
// projection (attention_k_eq_v, reference.rs:214-222) unless
// global_k_eq_v is 0.
//
// Every per-token input lives on the device (token, position and the two
// kv lengths in a step buffer; RoPE angles are computed on the device in
// f64 from the position), so one decode step can be captured into a hipGraph
// once and replayed — the reference records its graph once and rewrites the
// step buffer (graph.rs:462-476, 1485-1529).
//
// Kernels per layer: norm/embed row kernel -> QKV GEMV (one launch, three
// matrices) -> q/k/v post (norms, RoPE, Q8 append) -> split-K attention ->
// limb quant -> O GEMV -> post-attention row kernel -> gate/up GEMV (one
// launch) -> GeGLU+limbs -> down GEMV -> post-FFN row kernel (fused with the
// next layer's input norm).  Row kernels write the next GEMV's x limb table.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "limbs.h"
#include "q8.h"

struct sgq_model;

namespace sgq {
namespace {

constexpr int kRowWG = 1024;
constexpr int kHeadDim = 128;

__device__ __forceinline__ float gelu_tanh(float x) {
    const float k = 0.7978845608028654f;
    return 0.5f * x * (1.f + tanhf(k * (x + 0.044715f * x * x * x)));
}

// Sum over the workgroup in a fixed tree order (deterministic).  `red` holds
// one float per wave; the caller separates reuses with a barrier.
__device__ __forceinline__ float wg_sum(float v, float *red) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float r = 0.f;
    for (int w = 0; w < kRowWG / kWave; w++) r += red[w];
    return r;
}

__device__ __forceinline__ float sumsq4(float4 a) {
    return a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
}

// Row kernels: one workgroup of kRowWG threads, thread t owns the float4s
// t, t + kRowWG, ... (at most kRowV of them) in registers; the limb table of
// the result is written by 8-lane groups (float4 index i -> block i/8).
constexpr int kRowV = 4;  // hidden <= 4 * 4 * kRowWG = 16384

// x = dequant(E[token])·scale; xl = limbs(rmsnorm(x, w))
__global__ __launch_bounds__(kRowWG) void embed_norm_kernel(const uint8_t *__restrict__ E,
                                                             const uint32_t *__restrict__ step,
                                                             int hidden, float scale,
                                                             const float *__restrict__ w, float eps,
                                                             float *__restrict__ x,
                                                             BlockLimbs *__restrict__ xl) {
    __shared__ float red[kRowWG / kWave];
    const int n4 = hidden / 4, t = threadIdx.x;
    const uint8_t *er = E + (size_t)step[4] * (hidden / 32) * 18;
    float4 v[kRowV];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < kRowV; k++) {
        const int i = t + k * kRowWG;
        if (i < n4) {
            const uint8_t *blk = er + (i >> 3) * 18;
            const float d = f16_bits_to_f32(blk[0] | (blk[1] << 8));
            const int j0 = 4 * (i & 7);
            const int sh = j0 < 16 ? 0 : 4;
            const uint8_t *qs = blk + 2 + (j0 & 15);
            float e[4];
#pragma unroll
            for (int u = 0; u < 4; u++) e[u] = d * (float)(((qs[u] >> sh) & 15) - 8) * scale;
            v[k] = make_float4(e[0], e[1], e[2], e[3]);
            reinterpret_cast<float4 *>(x)[i] = v[k];
            ss += sumsq4(v[k]);
        }
    }
    ss = wg_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)hidden + eps);
#pragma unroll
    for (int k = 0; k < kRowV; k++) {
        const int i = t + k * kRowWG;
        if (i < n4) {
            const float4 wv = reinterpret_cast<const float4 *>(w)[i];
            const float4 y = make_float4(v[k].x * inv * wv.x, v[k].y * inv * wv.y,
                                         v[k].z * inv * wv.z, v[k].w * inv * wv.w);
            limbs_block8(y, i & 7, &xl[i >> 3]);
        }
    }
}

// The same with a Q6_K embedding row at a byte stride (q6_k.rs:41-62: value
// 128h + 32w + l of a 256-weight block is d·sc[l/16 + 2w + 8h]·q, q the
// 6-bit quant from ql's low (w even) or high (w odd) nibble of byte
// 64h + l (+32 for w = 1, 3) and 2 bits of qh[32h + l], minus 32).
// Values j0..j0+3 (j0 % 4 == 0) of a Q6_K row (q6_k.rs:41-62: 256-value
// super-blocks of ql[128], qh[64], int8 scales[16], f16 d), times `scale`.
__device__ __forceinline__ float4 q6k_quad(const uint8_t *__restrict__ er, int j0, float scale) {
    const uint8_t *blk = er + (j0 / 256) * 210;
    const int j = j0 % 256, h = j / 128, r = j % 128, wq = r / 32, l0 = r % 32;
    const float d = f16_bits_to_f32(blk[208] | (blk[209] << 8));
    const float ds = d * (float)(int8_t)blk[192 + 8 * h + l0 / 16 + 2 * wq];
    const uint8_t *ql = blk + 64 * h + (wq & 1) * 32;
    const uint8_t *qh = blk + 128 + 32 * h;
    float e[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int l = l0 + u;
        const int lo = wq < 2 ? (ql[l] & 15) : (ql[l] >> 4);
        const int q = (lo | (((qh[l] >> (2 * wq)) & 3) << 4)) - 32;
        e[u] = ds * (float)q * scale;
    }
    return make_float4(e[0], e[1], e[2], e[3]);
}

__global__ __launch_bounds__(kRowWG) void embed_q6k_norm_kernel(
    const uint8_t *__restrict__ E, uint64_t row_stride, const uint32_t *__restrict__ step,
    int hidden, float scale, const float *__restrict__ w, float eps, float *__restrict__ x,
    BlockLimbs *__restrict__ xl) {
    __shared__ float red[kRowWG / kWave];
    const int n4 = hidden / 4, t = threadIdx.x;
    const uint8_t *er = E + (size_t)step[4] * row_stride;
    float4 v[kRowV];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < kRowV; k++) {
        const int i = t + k * kRowWG;
        if (i < n4) {
            const float4 e4 = q6k_quad(er, 4 * i, scale);
            const float e[4] = {e4.x, e4.y, e4.z, e4.w};
            v[k] = make_float4(e[0], e[1], e[2], e[3]);
            reinterpret_cast<float4 *>(x)[i] = v[k];
            ss += sumsq4(v[k]);
        }
    }
    ss = wg_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)hidden + eps);
#pragma unroll
    for (int k = 0; k < kRowV; k++) {
        const int i = t + k * kRowWG;
        if (i < n4) {
            const float4 wv = reinterpret_cast<const float4 *>(w)[i];
            const float4 y = make_float4(v[k].x * inv * wv.x, v[k].y * inv * wv.y,
                                         v[k].z * inv * wv.z, v[k].w * inv * wv.w);
            limbs_block8(y, i & 7, &xl[i >> 3]);
        }
    }
}

// RoPE tables of the step's position for both layer kinds at their own
// head_dim (rope.rs:27-48 with f64 angles): [sliding: hd_s/2 pairs][global:
// hd_g/2 pairs] of (cos, sin); global pairs past live_g use divisor 1e30.
// The fused step's norm of the residual from a kEpiResid launch's partial
// sums (the GEMV's kProNorm prologue, written out for a head that is not a
// Q4_0 GEMV): with P = Σ of the np partials (Σo², Σx·u, Σu², Σx²),
// ra = 1/sqrt(P0/H + eps), rb = 1/sqrt(s²(P3 + 2·ra·P1 + ra²·P2)/H + eps),
// y = (A + ra·B)·rb·s with A = x·w_next, B = u·w_next the GEMV's rows.
__global__ __launch_bounds__(kRowWG) void norm_from_partials_kernel(
    const float4 *__restrict__ part, int np, const float *__restrict__ A,
    const float *__restrict__ B, const float *__restrict__ scale, int hidden, float eps,
    float *__restrict__ y) {
    __shared__ float red[kRowWG / kWave];
    const int t = threadIdx.x;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int i = t; i < np; i += kRowWG)
        acc.x += part[i].x, acc.y += part[i].y, acc.z += part[i].z, acc.w += part[i].w;
    float P[4] = {acc.x, acc.y, acc.z, acc.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
        P[k] = wg_sum(P[k], red);
        __syncthreads();  // red is reused by the next sum
    }
    const float P0 = P[0], P1 = P[1], P2 = P[2], P3 = P[3];
    const float s = scale ? *scale : 1.f, K = (float)hidden;
    const float ra = 1.0f / sqrtf(P0 / K + eps);
    const float rb = 1.0f / sqrtf(s * s * (P3 + 2.f * ra * P1 + ra * ra * P2) / K + eps);
    const float rs = rb * s;
    for (int i = t; i < hidden; i += kRowWG) y[i] = (A[i] + ra * B[i]) * rs;
}

__global__ void rope_table_generic_kernel(const uint32_t *__restrict__ step,
                                          float *__restrict__ cs, int hd_s, int hd_g,
                                          float theta_s, float theta_g, int live_g) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    const int ps = hd_s / 2, pg = hd_g / 2;
    if (t >= ps + pg) return;
    const bool glob = t >= ps;
    const int i = glob ? t - ps : t;
    const int hd = glob ? hd_g : hd_s;
    const double theta = glob ? (double)theta_g : (double)theta_s;
    const double factor = glob && i >= live_g ? 1e30 : 1.0;
    const double ang = (double)step[0] * pow(theta, -2.0 * (double)i / (double)hd) / factor;
    cs[2 * t] = (float)cos(ang);
    cs[2 * t + 1] = (float)sin(ang);
}

// post-attention: x += rmsnorm(o, w_post);            xl = limbs(rmsnorm(x, w_next))
// post-FFN:       x = (x + rmsnorm(o, w_post))·scale;  xl = limbs(rmsnorm(x, w_next))
// o arrives as n_parts K-slice partials (o = Σ_s o[s·hidden + i], s in order).
// Every input is loaded up front (one memory round trip); NP = K-slice
// partials of o, added in order.
template <int NP>
__global__ __launch_bounds__(kRowWG) void residual_norm_kernel(
    const float *__restrict__ o, const float *__restrict__ w_post, float *__restrict__ x,
    const float *__restrict__ scale_ptr, const float *__restrict__ w_next, int hidden, float eps,
    BlockLimbs *__restrict__ xl) {
    __shared__ float red[2][kRowWG / kWave];
    const int n4 = hidden / 4, t = threadIdx.x;
    float4 ov[kRowV][NP], xv[kRowV], wp[kRowV], wn[kRowV];
#pragma unroll
    for (int k = 0; k < kRowV; k++) {
        const int i = t + k * kRowWG;
        if (i < n4) {
#pragma unroll
            for (int p = 0; p < NP; p++)
                ov[k][p] = reinterpret_cast<const float4 *>(o + (size_t)p * hidden)[i];
            xv[k] = reinterpret_cast<const float4 *>(x)[i];
            wp[k] = reinterpret_cast<const float4 *>(w_post)[i];
            wn[k] = reinterpret_cast<const float4 *>(w_next)[i];
        }
    }
    const float s = scale_ptr ? *scale_ptr : 1.f;
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < kRowV; k++) {
        const int i = t + k * kRowWG;
        if (i < n4) {
            float4 a = ov[k][0];
#pragma unroll
            for (int p = 1; p < NP; p++)
                a.x += ov[k][p].x, a.y += ov[k][p].y, a.z += ov[k][p].z, a.w += ov[k][p].w;
            ov[k][0] = a;
            ss += sumsq4(a);
        }
    }
    ss = wg_sum(ss, red[0]);
    const float inv = 1.0f / sqrtf(ss / (float)hidden + eps);
    float ss2 = 0.f;
#pragma unroll
    for (int k = 0; k < kRowV; k++) {
        const int i = t + k * kRowWG;
        if (i < n4) {
            const float4 a = ov[k][0];
            float4 r;
            r.x = (xv[k].x + a.x * inv * wp[k].x) * s;
            r.y = (xv[k].y + a.y * inv * wp[k].y) * s;
            r.z = (xv[k].z + a.z * inv * wp[k].z) * s;
            r.w = (xv[k].w + a.w * inv * wp[k].w) * s;
            xv[k] = r;
            reinterpret_cast<float4 *>(x)[i] = r;
            ss2 += sumsq4(r);
        }
    }
    ss2 = wg_sum(ss2, red[1]);
    const float inv2 = 1.0f / sqrtf(ss2 / (float)hidden + eps);
#pragma unroll
    for (int k = 0; k < kRowV; k++) {
        const int i = t + k * kRowWG;
        if (i < n4) {
            const float4 y = make_float4(xv[k].x * inv2 * wn[k].x, xv[k].y * inv2 * wn[k].y,
                                         xv[k].z * inv2 * wn[k].z, xv[k].w * inv2 * wn[k].w);
            limbs_block8(y, i & 7, &xl[i >> 3]);
        }
    }
}

// h = gelu_tanh(g)·u, then its limb table; one float4 per thread.
__global__ __launch_bounds__(256) void geglu_limbs_kernel(const float *__restrict__ g,
                                                          const float *__restrict__ u, int n,
                                                          BlockLimbs *__restrict__ xl) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n / 4) return;  // n % 32 == 0: whole 8-lane groups exit together
    const float4 gv = reinterpret_cast<const float4 *>(g)[i];
    const float4 uv = reinterpret_cast<const float4 *>(u)[i];
    const float4 h = make_float4(gelu_tanh(gv.x) * uv.x, gelu_tanh(gv.y) * uv.y,
                                 gelu_tanh(gv.z) * uv.z, gelu_tanh(gv.w) * uv.w);
    limbs_block8(h, i & 7, &xl[i >> 3]);
}

// step words [pos, kv_len_sliding, kv_len_global, q0, token], and the RoPE
// (cos, sin) tables of position `a` for both layer kinds, angles in f64
// (crates/sg-model/src/rope.rs:27-48): pair i of 64 turns by
// pos·theta^(-2i/128)/factor_i; global layers use the divisor factors
// [1 × live, 1e30 × rest] (rope.rs:13-16), so pairs past `live` barely move.
__global__ void model_step_kernel(uint32_t *step, uint32_t a, uint32_t b, uint32_t c, uint32_t d,
                                  uint32_t e, float *rope_cs, float theta_s, float theta_g,
                                  int live_g) {
    const uint32_t t = threadIdx.x;
    if (t < 5) step[t] = t == 0 ? a : t == 1 ? b : t == 2 ? c : t == 3 ? d : e;
    if (t < kHeadDim) {
        const int kind = t / (kHeadDim / 2), i = t % (kHeadDim / 2);
        const double theta = kind ? (double)theta_g : (double)theta_s;
        const double factor = kind && i >= live_g ? 1e30 : 1.0;
        const double freq = pow(theta, -2.0 * (double)i / (double)kHeadDim);
        const double ang = (double)a * freq / factor;
        rope_cs[t * 2] = (float)cos(ang);
        rope_cs[t * 2 + 1] = (float)sin(ang);
    }
}

// ---- prefill row kernels (one chunk of M tokens) ------------------------

// RoPE tables of positions q0..q0+M-1 for both layer kinds, f64 angles as
// in model_step_kernel; layout [kind][token][pair][cos, sin].
__global__ void pf_rope_table_kernel(float *__restrict__ cs, int q0, int M, int hd_s, int hd_g,
                                     float theta_s, float theta_g, int live_g) {
    // sliding table [M][hd_s/2] (cos, sin), then the global one [M][hd_g/2]
    const int t = blockIdx.x * 256 + threadIdx.x;
    const int hs = hd_s / 2, hg = hd_g / 2;
    if (t >= M * (hs + hg)) return;
    const int kind = t >= M * hs;
    const int r = kind ? t - M * hs : t, half = kind ? hg : hs;
    const int tok = r / half, i = r % half;
    const double theta = kind ? (double)theta_g : (double)theta_s;
    const double factor = kind && i >= live_g ? 1e30 : 1.0;
    const double ang =
        (double)(q0 + tok) * pow(theta, -2.0 * (double)i / (double)(kind ? hd_g : hd_s)) / factor;
    cs[2 * t] = (float)cos(ang);
    cs[2 * t + 1] = (float)sin(ang);
}

constexpr int kPfWG = 256;

__device__ __forceinline__ float block_sum256(float v, float *red) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    const float r = red[0] + red[1] + red[2] + red[3];
    __syncthreads();
    return r;
}

// x[row] = dequant(E[token])·scale; Q8_0 of rmsnorm(x[row], w).  One
// workgroup per row; thread t owns float4s t, t+256, ... (8-lane groups =
// one Q8 block, as n4 % 8 == 0).
__global__ __launch_bounds__(kPfWG) void pf_embed_norm_q8_kernel(
    const uint8_t *__restrict__ E, const uint32_t *__restrict__ tokens, int H, float scale,
    const float *__restrict__ w, float eps, float *__restrict__ x, int8_t *__restrict__ xq,
    uint16_t *__restrict__ xs) {
    __shared__ float red[4];
    const int row = blockIdx.x, t = threadIdx.x, n4 = H / 4;
    const uint8_t *er = E + (size_t)tokens[row] * (H / 32) * 18;
    float4 *xr = reinterpret_cast<float4 *>(x + (size_t)row * H);
    float ss = 0.f;
    for (int i = t; i < n4; i += kPfWG) {
        const uint8_t *blk = er + (i >> 3) * 18;
        const float d = f16_bits_to_f32(blk[0] | (blk[1] << 8));
        const int j0 = 4 * (i & 7);
        const int sh = j0 < 16 ? 0 : 4;
        const uint8_t *qs = blk + 2 + (j0 & 15);
        float e[4];
#pragma unroll
        for (int u = 0; u < 4; u++) e[u] = d * (float)(((qs[u] >> sh) & 15) - 8) * scale;
        const float4 v = make_float4(e[0], e[1], e[2], e[3]);
        xr[i] = v;
        ss += e[0] * e[0] + e[1] * e[1] + e[2] * e[2] + e[3] * e[3];
    }
    const float inv = 1.0f / sqrtf(block_sum256(ss, red) / (float)H + eps);
    int *qr = reinterpret_cast<int *>(xq + (size_t)row * H);
    for (int i = t; i < n4; i += kPfWG) {
        const float4 v = xr[i], wv = reinterpret_cast<const float4 *>(w)[i];
        const float4 y = make_float4(v.x * inv * wv.x, v.y * inv * wv.y, v.z * inv * wv.z,
                                     v.w * inv * wv.w);
        int q;
        quant_lane(y, i & 7, &xs[(size_t)row * (H / 32) + (i >> 3)], &q);
        qr[i] = q;
    }
}

// The same for a Q6_K embedding (rows at the device's padded stride).
__global__ __launch_bounds__(kPfWG) void pf_embed_q6k_norm_q8_kernel(
    const uint8_t *__restrict__ E, uint64_t row_stride, const uint32_t *__restrict__ tokens, int H,
    float scale, const float *__restrict__ w, float eps, float *__restrict__ x,
    int8_t *__restrict__ xq, uint16_t *__restrict__ xs) {
    __shared__ float red[4];
    const int row = blockIdx.x, t = threadIdx.x, n4 = H / 4;
    const uint8_t *er = E + (size_t)tokens[row] * row_stride;
    float4 *xr = reinterpret_cast<float4 *>(x + (size_t)row * H);
    float ss = 0.f;
    for (int i = t; i < n4; i += kPfWG) {
        const float4 v = q6k_quad(er, 4 * i, scale);
        xr[i] = v;
        ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
    const float inv = 1.0f / sqrtf(block_sum256(ss, red) / (float)H + eps);
    int *qr = reinterpret_cast<int *>(xq + (size_t)row * H);
    for (int i = t; i < n4; i += kPfWG) {
        const float4 v = xr[i], wv = reinterpret_cast<const float4 *>(w)[i];
        const float4 y = make_float4(v.x * inv * wv.x, v.y * inv * wv.y, v.z * inv * wv.z,
                                     v.w * inv * wv.w);
        int q;
        quant_lane(y, i & 7, &xs[(size_t)row * (H / 32) + (i >> 3)], &q);
        qr[i] = q;
    }
}

// post-attention: x += rmsnorm(o, w_post);            Q8_0 of rmsnorm(x, w_next)
// post-FFN:       x = (x + rmsnorm(o, w_post))·scale;  Q8_0 of rmsnorm(x, w_next)
__global__ __launch_bounds__(kPfWG) void pf_residual_norm_q8_kernel(
    const float *__restrict__ o, const float *__restrict__ w_post, float *__restrict__ x,
    const float *__restrict__ scale_ptr, const float *__restrict__ w_next, int H, float eps,
    int8_t *__restrict__ xq, uint16_t *__restrict__ xs) {
    __shared__ float red[4];
    const int row = blockIdx.x, t = threadIdx.x, n4 = H / 4;
    const float4 *orow = reinterpret_cast<const float4 *>(o + (size_t)row * H);
    float4 *xr = reinterpret_cast<float4 *>(x + (size_t)row * H);
    float ss = 0.f;
    for (int i = t; i < n4; i += kPfWG) {
        const float4 v = orow[i];
        ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
    const float inv = 1.0f / sqrtf(block_sum256(ss, red) / (float)H + eps);
    const float s = scale_ptr ? *scale_ptr : 1.f;
    float ss2 = 0.f;
    for (int i = t; i < n4; i += kPfWG) {
        const float4 v = orow[i], xv = xr[i], wp = reinterpret_cast<const float4 *>(w_post)[i];
        float4 r;
        r.x = (xv.x + v.x * inv * wp.x) * s;
        r.y = (xv.y + v.y * inv * wp.y) * s;
        r.z = (xv.z + v.z * inv * wp.z) * s;
        r.w = (xv.w + v.w * inv * wp.w) * s;
        xr[i] = r;
        ss2 += r.x * r.x + r.y * r.y + r.z * r.z + r.w * r.w;
    }
    const float inv2 = 1.0f / sqrtf(block_sum256(ss2, red) / (float)H + eps);
    int *qr = reinterpret_cast<int *>(xq + (size_t)row * H);
    for (int i = t; i < n4; i += kPfWG) {
        const float4 v = xr[i], wv = reinterpret_cast<const float4 *>(w_next)[i];
        const float4 y = make_float4(v.x * inv2 * wv.x, v.y * inv2 * wv.y, v.z * inv2 * wv.z,
                                     v.w * inv2 * wv.w);
        int q;
        quant_lane(y, i & 7, &xs[(size_t)row * (H / 32) + (i >> 3)], &q);
        qr[i] = q;
    }
}

// h = gelu_tanh(g)·u as Q8_0, one float4 per thread.
__global__ __launch_bounds__(256) void pf_geglu_q8_kernel(const float4 *__restrict__ g,
                                                          const float4 *__restrict__ u,
                                                          uint64_t n4, int *__restrict__ hq,
                                                          uint16_t *__restrict__ hs) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;  // n4 % 8 == 0: whole 8-lane groups exit together
    const float4 a = g[i], b = u[i];
    const float4 h = make_float4(gelu_tanh(a.x) * b.x, gelu_tanh(a.y) * b.y, gelu_tanh(a.z) * b.z,
                                 gelu_tanh(a.w) * b.w);
    int q;
    quant_lane(h, (int)(i & 7), &hs[i >> 3], &q);
    hq[i] = q;
}


// Per (token, head): q -> rmsnorm(q_norm) + RoPE (fp32 out); k -> rmsnorm
// (k_norm) + RoPE -> Q8_0 into the chunk's K pages; v -> weightless rmsnorm
// -> Q8_0 into the chunk's V pages.
// At head_dim 128 / 256 / 512: LPR = min(64, head_dim/4)
// lanes per (token, head row) (half a wave at 128, a whole wave at 256 and
// 512), lane j holding float4 j (and j + 64 at 512), the NEOX partner
// float4 j ± HD/8 a lane shuffle within the row's lanes (128, 256) or the
// lane's other float4 (512), and the Q8_0 quantization of 8-lane groups
// (quant_lane): 4·(64/LPR) rows per 256-thread workgroup, no barriers.
template <int HD>
__global__ __launch_bounds__(256) void pf_qkv_post_wide_kernel(
    const float *__restrict__ q_raw, const float *__restrict__ k_raw,
    const float *__restrict__ v_src, const float *__restrict__ wq_norm,
    const float *__restrict__ wk_norm, const float *__restrict__ cs, int n_q, int n_kv, int M,
    float eps, float *__restrict__ q_out, int8_t *__restrict__ ckq, uint16_t *__restrict__ cks,
    int8_t *__restrict__ cvq, uint16_t *__restrict__ cvs) {
    constexpr int NF = HD / 4;                  // float4s per row
    constexpr int LPR = NF < 64 ? NF : 64;      // lanes per row
    constexpr int RPW = 64 / LPR;               // rows per wave
    constexpr int NV = NF / LPR;                // float4s per lane
    static_assert(NV == 1 || NV == 2, "head_dim 128, 256 or 512");
    const int lane = threadIdx.x & 63, sub = lane % LPR;
    const int R = n_q + 2 * n_kv;
    const long rid = ((long)blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW + lane / LPR;
    if (rid >= (long)M * R) return;  // whole rows (a row's lanes share a wave)
    const int tok = (int)(rid / R), h = (int)(rid % R);
    const int kind = h < n_q ? 0 : (h < n_q + n_kv ? 1 : 2);
    const int head = kind == 0 ? h : (kind == 1 ? h - n_q : h - n_q - n_kv);
    const int QD = n_q * HD, KD = n_kv * HD;
    const float *src = (kind == 0 ? q_raw + (size_t)tok * QD
                                  : (kind == 1 ? k_raw : v_src) + (size_t)tok * KD) +
                       (size_t)head * HD;
    const float *w = kind == 0 ? wq_norm : (kind == 1 ? wk_norm : nullptr);
    float4 x[NV];
    float ss = 0.f;
#pragma unroll
    for (int v = 0; v < NV; v++) {
        x[v] = reinterpret_cast<const float4 *>(src)[sub + LPR * v];
        ss += x[v].x * x[v].x + x[v].y * x[v].y + x[v].z * x[v].z + x[v].w * x[v].w;
    }
    for (int o = LPR / 2; o > 0; o >>= 1) ss += __shfl_xor(ss, o, kWave);
    const float inv = 1.0f / sqrtf(ss / (float)HD + eps);
#pragma unroll
    for (int v = 0; v < NV; v++) {
        const float4 wt = w ? reinterpret_cast<const float4 *>(w)[sub + LPR * v]
                            : make_float4(1.f, 1.f, 1.f, 1.f);
        x[v] = make_float4(x[v].x * inv * wt.x, x[v].y * inv * wt.y, x[v].z * inv * wt.z,
                           x[v].w * inv * wt.w);
    }
    if (kind < 2) {
        float4 pr[NV];
        if (NV == 1) {
            const int pl = lane ^ (NF / 2);  // float4 j ± NF/2, within the row's lanes
            pr[0] = make_float4(__shfl(x[0].x, pl, kWave), __shfl(x[0].y, pl, kWave),
                                __shfl(x[0].z, pl, kWave), __shfl(x[0].w, pl, kWave));
        } else {
#pragma unroll
            for (int v = 0; v < NV; v++) pr[v] = x[NV - 1 - v];
        }
        const float2 *tc = reinterpret_cast<const float2 *>(cs) + (size_t)tok * (HD / 2);
#pragma unroll
        for (int v = 0; v < NV; v++) {
            const int j = sub + LPR * v;
            const bool lo = j < NF / 2;
            const int i0 = (lo ? j : j - NF / 2) * 4;
            const float sg = lo ? -1.f : 1.f;
            const float2 c0 = tc[i0], c1 = tc[i0 + 1], c2 = tc[i0 + 2], c3 = tc[i0 + 3];
            x[v] = make_float4(x[v].x * c0.x + sg * pr[v].x * c0.y,
                               x[v].y * c1.x + sg * pr[v].y * c1.y,
                               x[v].z * c2.x + sg * pr[v].z * c2.y,
                               x[v].w * c3.x + sg * pr[v].w * c3.y);
        }
    }
    if (kind == 0) {
#pragma unroll
        for (int v = 0; v < NV; v++)
            reinterpret_cast<float4 *>(q_out + (size_t)tok * QD + (size_t)head * HD)[sub + LPR * v] = x[v];
        return;
    }
    const size_t e0 = ((size_t)tok * n_kv + head) * HD;
    int *qt = reinterpret_cast<int *>(kind == 1 ? ckq : cvq);
    uint16_t *sc = kind == 1 ? cks : cvs;
#pragma unroll
    for (int v = 0; v < NV; v++) {
        const int j = sub + LPR * v;
        int qv;
        quant_lane(x[v], j & 7, &sc[(e0 + 4 * j) / 32], &qv);
        qt[(e0 + 4 * j) / 4] = qv;
    }
}

// Append the chunk's K/V pages (rows i = position - q0) to a cache: slot
// q0+i, or (q0+i) mod ring — then only the last `ring` rows, so no two
// threads write one slot.  Thread = one 16-byte quant chunk of a row (and one
// scale where the row has one).
__global__ void pf_kv_append_kernel(const int8_t *__restrict__ ckq, const uint16_t *__restrict__ cks,
                                    const int8_t *__restrict__ cvq, const uint16_t *__restrict__ cvs,
                                    int8_t *__restrict__ kq, uint16_t *__restrict__ ks,
                                    int8_t *__restrict__ vq, uint16_t *__restrict__ vs, int M,
                                    int q0, int ring, int KD) {
    const int per_row = KD / 16;
    const int i0 = ring && M > ring ? M - ring : 0;
    const long g = (long)blockIdx.x * 256 + threadIdx.x;
    if (g >= (long)(M - i0) * per_row) return;
    const int i = i0 + (int)(g / per_row), c = (int)(g % per_row);
    const int pos = q0 + i;
    const size_t slot = ring ? (size_t)(pos % ring) : (size_t)pos;
    typedef int i4v __attribute__((ext_vector_type(4)));
    reinterpret_cast<i4v *>(kq + slot * KD)[c] = reinterpret_cast<const i4v *>(ckq + (size_t)i * KD)[c];
    reinterpret_cast<i4v *>(vq + slot * KD)[c] = reinterpret_cast<const i4v *>(cvq + (size_t)i * KD)[c];
    if (c < KD / 32) {
        ks[slot * (KD / 32) + c] = cks[(size_t)i * (KD / 32) + c];
        vs[slot * (KD / 32) + c] = cvs[(size_t)i * (KD / 32) + c];
    }
}

}  // namespace
}  // namespace sgq

using namespace sgq;

struct LayerW {
    void *wq = nullptr, *wk = nullptr, *wv = nullptr, *wo = nullptr, *wg = nullptr,
         *wu = nullptr, *wd = nullptr;  // Q4_0 (wv null: V from the K projection)
    float *attn_norm, *q_norm, *k_norm, *post_attn_norm, *ffn_norm, *post_ffw_norm;
    float *out_scale;  // 1 float
    bool global;
    int8_t *kq, *vq;
    uint16_t *ks, *vs;
    uint32_t slots;
    uint32_t hd, n_kv;  // this layer kind's head_dim and kv heads
};

// The split merge of the fused decode runs as its own launch: queued behind
// the split kernel it costs little, and measured 1.7% faster per step than
// the last split of each kv head merging inside the split kernel (which
// adds a store drain and a counter to every workgroup).

// Decode attention splits per kv head: 16 for a 1024-slot ring (64 slots
// per split; with the merge as its own launch, 16 and 32 measured equal and
// 0.6% faster per step than 8, 4 was 2.3% slower), about 512 slots per
// workgroup for a linear cache (measured best at 8K against 256 and 1024).
#ifndef SGQ_SLIDING_SPLITS
#define SGQ_SLIDING_SPLITS 16
#endif
#ifndef SGQ_GLOBAL_SLOTS_PER_SPLIT
#define SGQ_GLOBAL_SLOTS_PER_SPLIT 512
#endif
static int decode_splits(const LayerW &L) {
    return L.global ? (int)std::min(64u, std::max(8u, L.slots / SGQ_GLOBAL_SLOTS_PER_SPLIT))
                    : SGQ_SLIDING_SPLITS;
}

struct sgq_model {
    sgq_ctx *ctx;
    sgq_model_config cfg;
    std::vector<LayerW> layers;
    void *embd = nullptr;
    float *out_norm = nullptr;
    std::vector<void *> allocs;
    // activations
    float *x, *q_raw, *k_raw, *v_raw, *q, *attn, *o, *g, *u, *f;
    void *xl;  // limb table (largest K)
    uint32_t *step;
    float *rope_cs;  // [2 kinds][head_dim/2][cos, sin] of the current position
    // mode 3 (any geometry): per-kind RoPE tables [hd_s/2 + hd_g/2][cos, sin],
    // post-norm k and v rows, attention split partials, the final-normed x
    // for a Q6_K head; embd_stride = bytes per embedding row (Q6_K rows are
    // padded to 16 bytes, as the reference uploads them)
    bool generic = false;
    uint64_t embd_stride = 0;
    float *rope_g = nullptr, *kx = nullptr, *vx = nullptr, *part_g = nullptr, *xf = nullptr;
    float *logits_tmp = nullptr;
    uint32_t pos = 0;
    sgq_graph *graph = nullptr;
    float *graph_logits = nullptr;
    // fused decode (mode 2): the residual in two buffers (xa: entering a
    // layer, xb: after attention), the residual epilogue's u/A/B rows and
    // per-workgroup partial sums, and the limb tables of the attention
    // output and of the GeGLU output
    struct {
        float *xb, *u, *a, *b;
        float4 *part;
        void *xl_o, *hl;
    } fx{};
    int mode = 0;  // 0 kernel per operator, 2 fused, 3 any geometry
    // prefill chunk buffers (allocated at the first prefill, `chunk` rows)
    struct {
        uint32_t chunk = 0;
        uint32_t *tok;
        float *rope;                      // [2 kinds][chunk][64][cos, sin]
        float *x, *q_raw, *k_raw, *v_raw, *q, *attn, *o, *g, *u, *f, *part, *head_in;
        int8_t *xq, *aq, *hq, *ckq, *cvq;  // Q8_0 quants
        uint16_t *xs, *as, *hs, *cks, *cvs;  // and their f16 scales
    } pf;
};

namespace {

int alloc(sgq_model *m, size_t bytes, void **p) {
    SGQ_HIP(hipMalloc(p, bytes ? bytes : 256));
    m->allocs.push_back(*p);
    return SGQ_OK;
}

uint64_t mix(uint64_t a, uint64_t b) { return (a + 0x9E3779B97F4A7C15ull) * 0xBF58476D1CE4E5B9ull ^ b; }

int q4_tensor(sgq_model *m, size_t rows, size_t cols, uint64_t seed, void **p) {
    int rc = alloc(m, rows * (cols / 32) * 18, p);
    if (rc) return rc;
    return launch_fill_q4_0(ctx_stream(m->ctx), *p, rows * (cols / 32), seed, m->cfg.weight_sigma);
}

int f32_tensor(sgq_model *m, size_t n, uint64_t seed, float mean, float sigma, float **p) {
    int rc = alloc(m, n * 4, reinterpret_cast<void **>(p));
    if (rc) return rc;
    return launch_fill_normal(ctx_stream(m->ctx), *p, n, seed, mean, sigma);
}

int record_step(sgq_model *m, float *logits) {
    const sgq_model_config &c = m->cfg;
    hipStream_t st = ctx_stream(m->ctx);
    const int H = (int)c.hidden, F = (int)c.ffn, QD = (int)(c.n_q_heads * kHeadDim),
              KD = (int)(c.n_kv_heads * kHeadDim);
    BlockLimbs *xl = static_cast<BlockLimbs *>(m->xl);
    int rc;
    hipLaunchKernelGGL(embed_norm_kernel, dim3(1), dim3(kRowWG), 0, st,
                       static_cast<const uint8_t *>(m->embd), m->step, H, sqrtf((float)H),
                       m->layers[0].attn_norm, c.eps, m->x, xl);
    SGQ_HIP(hipGetLastError());
    for (size_t li = 0; li < m->layers.size(); li++) {
        const LayerW &L = m->layers[li];
        GemvTargets qkv{};
        qkv.w[0] = L.wq, qkv.w[1] = L.wk, qkv.w[2] = L.wv;
        qkv.y[0] = m->q_raw, qkv.y[1] = m->k_raw, qkv.y[2] = m->v_raw;
        qkv.end[0] = QD, qkv.end[1] = QD + KD, qkv.end[2] = QD + 2 * KD;
        qkv.count = L.wv ? 3 : 2;
        const float *v_src = L.wv ? m->v_raw : m->k_raw;
        if ((rc = launch_gemv_limbs(st, qkv, xl, H))) return rc;
        const int n_splits = decode_splits(L);
        if ((rc = launch_attn_decode_fused(
                 st, m->q_raw, m->k_raw, v_src, L.q_norm, L.k_norm,
                 m->rope_cs + (L.global ? kHeadDim : 0), c.eps, m->step, L.global ? 2 : 1,
                 L.global ? 0u : L.slots, L.kq, L.ks, L.vq, L.vs, (int)c.n_q_heads,
                 (int)c.n_kv_heads, n_splits, c.attn_scale, m->attn, ctx_workspace(m->ctx),
                 kWorkspaceBytes, xl)))
            return rc;
        GemvTargets ot{};
        ot.w[0] = L.wo, ot.y[0] = m->o, ot.end[0] = H, ot.count = 1;
        if ((rc = launch_gemv_limbs(st, ot, xl, QD))) return rc;
        hipLaunchKernelGGL(residual_norm_kernel<1>, dim3(1), dim3(kRowWG), 0, st, m->o,
                           L.post_attn_norm, m->x, (const float *)nullptr, L.ffn_norm, H, c.eps, xl);
        SGQ_HIP(hipGetLastError());
        GemvTargets gu{};
        gu.w[0] = L.wg, gu.w[1] = L.wu, gu.y[0] = m->g, gu.y[1] = m->u;
        gu.end[0] = F, gu.end[1] = 2 * F, gu.count = 2;
        if ((rc = launch_gemv_limbs(st, gu, xl, H))) return rc;
        hipLaunchKernelGGL(geglu_limbs_kernel, dim3((F / 4 + 255) / 256), dim3(256), 0, st, m->g,
                           m->u, F, xl);
        SGQ_HIP(hipGetLastError());
        GemvTargets dt{};
        dt.w[0] = L.wd, dt.y[0] = m->f, dt.end[0] = H, dt.count = 1;
        dt.split_out = gemv_slices(F) > 1;
        const int f_parts = dt.split_out ? gemv_slices(F) : 1;
        if ((rc = launch_gemv_limbs(st, dt, xl, F))) return rc;
        const float *w_next =
            li + 1 < m->layers.size() ? m->layers[li + 1].attn_norm : m->out_norm;
        if (f_parts == 4)
            hipLaunchKernelGGL(residual_norm_kernel<4>, dim3(1), dim3(kRowWG), 0, st, m->f,
                               L.post_ffw_norm, m->x, L.out_scale, w_next, H, c.eps, xl);
        else if (f_parts == 2)
            hipLaunchKernelGGL(residual_norm_kernel<2>, dim3(1), dim3(kRowWG), 0, st, m->f,
                               L.post_ffw_norm, m->x, L.out_scale, w_next, H, c.eps, xl);
        else
            hipLaunchKernelGGL(residual_norm_kernel<1>, dim3(1), dim3(kRowWG), 0, st, m->f,
                               L.post_ffw_norm, m->x, L.out_scale, w_next, H, c.eps, xl);
        SGQ_HIP(hipGetLastError());
    }
    GemvTargets head{};
    head.w[0] = m->embd, head.y[0] = logits, head.end[0] = (int)c.vocab, head.count = 1;
    head.softcap = c.final_softcap;
    return launch_gemv_limbs(st, head, xl, H);
}

// Decode step at any supported geometry (mode 3): the kernel-per-operator
// sequence of record_step with each layer kind's own head_dim and kv heads
// (the real checkpoint: sliding 16 × 256, global 4 × 512 under 32 query
// heads, desc.rs:66-93), the q/k/v post-projection as separate norm, RoPE
// and Q8_0-append launches, the VALU split-K attention (attn_generic.hip),
// and a Q4_0 or Q6_K tied head.  `head` false skips the logits (prefill's
// inner tokens).
int record_step_generic(sgq_model *m, float *logits, bool head) {
    const sgq_model_config &c = m->cfg;
    hipStream_t st = ctx_stream(m->ctx);
    const int H = (int)c.hidden, F = (int)c.ffn, nq = (int)c.n_q_heads;
    const int hd_s = (int)c.head_dim;
    BlockLimbs *xl = static_cast<BlockLimbs *>(m->xl);
    int rc;
    if (c.embed_q6k)
        hipLaunchKernelGGL(embed_q6k_norm_kernel, dim3(1), dim3(kRowWG), 0, st,
                           static_cast<const uint8_t *>(m->embd), m->embd_stride, m->step, H,
                           sqrtf((float)H), m->layers[0].attn_norm, c.eps, m->x, xl);
    else
        hipLaunchKernelGGL(embed_norm_kernel, dim3(1), dim3(kRowWG), 0, st,
                           static_cast<const uint8_t *>(m->embd), m->step, H, sqrtf((float)H),
                           m->layers[0].attn_norm, c.eps, m->x, xl);
    SGQ_HIP(hipGetLastError());
    for (size_t li = 0; li < m->layers.size(); li++) {
        const LayerW &L = m->layers[li];
        const int hd = (int)L.hd, nkv = (int)L.n_kv, QD = nq * hd, KD = nkv * hd;
        GemvTargets qkv{};
        qkv.w[0] = L.wq, qkv.w[1] = L.wk, qkv.w[2] = L.wv;
        qkv.y[0] = m->q_raw, qkv.y[1] = m->k_raw, qkv.y[2] = m->v_raw;
        qkv.end[0] = QD, qkv.end[1] = QD + KD, qkv.end[2] = QD + 2 * KD;
        qkv.count = L.wv ? 3 : 2;
        if ((rc = launch_gemv_limbs(st, qkv, xl, H))) return rc;
        const float *v_src = L.wv ? m->v_raw : m->k_raw;
        // attention with the post-projection fused in (q/k norms with
        // weights, weightless v norm, NEOX RoPE, Q8_0 append), merged into
        // the O projection's limbs
        const float *cs = m->rope_g + (L.global ? hd_s : 0);
        const GenericPost post{m->q_raw, m->k_raw, v_src, L.q_norm, L.k_norm, (const float2 *)cs,
                               c.eps, L.global ? 0u : L.slots, L.kq, L.vq, L.ks, L.vs};
        if ((rc = launch_attn_decode_generic(st, nullptr, L.kq, L.ks, L.vq, L.vs, m->step,
                                             L.global ? 2 : 1, nq, nkv, hd,
                                             attn_generic_splits(L.slots), c.attn_scale,
                                             m->part_g, m->attn, xl, &post)))
            return rc;
        GemvTargets ot{};
        ot.w[0] = L.wo, ot.y[0] = m->o, ot.end[0] = H, ot.count = 1;
        if ((rc = launch_gemv_limbs(st, ot, xl, QD))) return rc;
        hipLaunchKernelGGL(residual_norm_kernel<1>, dim3(1), dim3(kRowWG), 0, st, m->o,
                           L.post_attn_norm, m->x, (const float *)nullptr, L.ffn_norm, H, c.eps, xl);
        SGQ_HIP(hipGetLastError());
        GemvTargets gu{};
        gu.w[0] = L.wg, gu.w[1] = L.wu, gu.y[0] = m->g, gu.y[1] = m->u;
        gu.end[0] = F, gu.end[1] = 2 * F, gu.count = 2;
        if ((rc = launch_gemv_limbs(st, gu, xl, H))) return rc;
        hipLaunchKernelGGL(geglu_limbs_kernel, dim3((F / 4 + 255) / 256), dim3(256), 0, st, m->g,
                           m->u, F, xl);
        SGQ_HIP(hipGetLastError());
        GemvTargets dt{};
        dt.w[0] = L.wd, dt.y[0] = m->f, dt.end[0] = H, dt.count = 1;
        if ((rc = launch_gemv_limbs(st, dt, xl, F))) return rc;
        const float *w_next =
            li + 1 < m->layers.size() ? m->layers[li + 1].attn_norm : m->out_norm;
        hipLaunchKernelGGL(residual_norm_kernel<1>, dim3(1), dim3(kRowWG), 0, st, m->f,
                           L.post_ffw_norm, m->x, L.out_scale, w_next, H, c.eps, xl);
        SGQ_HIP(hipGetLastError());
    }
    if (!head) return SGQ_OK;
    if (c.embed_q6k) {
        if ((rc = launch_rmsnorm(st, m->x, m->out_norm, m->xf, 1, (uint32_t)H, 0, c.eps))) return rc;
        return launch_gemv_q6_k(st, m->embd, m->embd_stride, m->xf, logits, c.vocab, (uint32_t)H,
                                c.final_softcap);
    }
    GemvTargets hd_t{};
    hd_t.w[0] = m->embd, hd_t.y[0] = logits, hd_t.end[0] = (int)c.vocab, hd_t.count = 1;
    hd_t.softcap = c.final_softcap;
    return launch_gemv_limbs(st, hd_t, xl, H);
}

// Fused decode step (mode 2): six launches per layer.
//   QKV GEMV       prologue: the previous layer's post-FFN residual update and
//                  this layer's input RMSNorm, from the down GEMV's partial
//                  sums (layer 0: the embedding row); writes x (xa)
//   attention      fused q/k/v post-projection and K/V append
//   merge          the splits in split order -> the O GEMV's limbs
//   O GEMV         epilogue: u/A/B rows and partial sums for the post-
//                  attention residual and the FFN norm
//   gate/up GEMV   prologue: the post-attention residual (writes xb) and the
//                  FFN norm; epilogue: GeGLU of 32-unit blocks -> limbs
//   down GEMV      epilogue: u/A/B rows and partial sums for the post-FFN
//                  residual and the next layer's (or the head's) norm
// The tied head's GEMV takes the last layer's update in its prologue.
// Norm statistics come from sums of per-row terms:
//   Σ(x + r·u)² = Σx² + 2r·Σx·u + r²·Σu²,  r = 1/sqrt(Σo²/H + eps).
int record_step_fused(sgq_model *m, float *logits) {
    const sgq_model_config &c = m->cfg;
    hipStream_t st = ctx_stream(m->ctx);
    const int H = (int)c.hidden, F = (int)c.ffn, nq = (int)c.n_q_heads;
    // the down projection's four K-slices of the GeGLU limb table (672
    // entries, 53.8 KB) go to LDS once per workgroup, instead of each wave
    // loading its slice's entries into registers: 234.7 -> 237.6 tok/s
    // (three interleaved pairs in one call)
    const int pro_d = kProTableLds;
    const int np_d = gemv_fused_grid((uint32_t)H, (uint32_t)F, kEpiResid, pro_d);
    SGQ_CHECK(np_d > 0 && np_d <= kGemvMaxPartials, "model (fused): partial sums %d", np_d);
    float *xa = m->x, *xb = m->fx.xb;
    int rc;
    const size_t nl = m->layers.size();
    for (size_t li = 0; li < nl; li++) {
        const LayerW &L = m->layers[li];
        const int hd = (int)L.hd, nkv = (int)L.n_kv, QD = nq * hd, KD = nkv * hd;
        // O's limb table into LDS once per workgroup when it is one K-slice
        const int pro_o = gemv_slices((uint32_t)QD) == 1 ? kProTableLds : kProTable;
        const int np_o = gemv_fused_grid((uint32_t)H, (uint32_t)QD, kEpiResid, pro_o);
        SGQ_CHECK(np_o > 0 && np_o <= kGemvMaxPartials, "model (fused): partial sums %d", np_o);
        GemvTargets qkv{};
        qkv.w[0] = L.wq, qkv.w[1] = L.wk, qkv.w[2] = L.wv;
        qkv.y[0] = m->q_raw, qkv.y[1] = m->k_raw, qkv.y[2] = m->v_raw;
        qkv.end[0] = QD, qkv.end[1] = QD + KD, qkv.end[2] = QD + 2 * KD;
        qkv.count = L.wv ? 3 : 2;
        GemvFuse pre{};
        pre.eps = c.eps;
        pre.x_out = xa;
        int pro;
        const void *qkv_xl = nullptr;
        if (li == 0 && c.embed_q6k) {
            // Q6_K embedding row: its own launch writes x and the norm's limbs
            hipLaunchKernelGGL(embed_q6k_norm_kernel, dim3(1), dim3(kRowWG), 0, st,
                               static_cast<const uint8_t *>(m->embd), m->embd_stride, m->step, H,
                               sqrtf((float)H), L.attn_norm, c.eps, xa,
                               static_cast<BlockLimbs *>(m->xl));
            SGQ_HIP(hipGetLastError());
            pro = kProTable;
            qkv_xl = m->xl;
            pre = GemvFuse{};
        } else if (li == 0) {
            pro = kProEmbed;
            pre.embd = static_cast<const uint8_t *>(m->embd);
            pre.step = m->step;
            pre.embed_scale = sqrtf((float)H);
            pre.w = L.attn_norm;
        } else {
            pro = kProNorm;
            pre.part = m->fx.part, pre.np = np_d;
            pre.A = m->fx.a, pre.B = m->fx.b, pre.u = m->fx.u, pre.x_in = xb;
            pre.scale = m->layers[li - 1].out_scale;
        }
        if ((rc = launch_gemv_fused(st, qkv, qkv_xl, (uint32_t)H, pro, kEpiRows, pre))) return rc;
        const float *v_src = L.wv ? m->v_raw : m->k_raw;
        if (m->generic) {
            const float *cs = m->rope_g + (L.global ? c.head_dim : 0);
            const GenericPost post{m->q_raw, m->k_raw, v_src, L.q_norm, L.k_norm,
                                   (const float2 *)cs, c.eps, L.global ? 0u : L.slots,
                                   L.kq, L.vq, L.ks, L.vs};
            if ((rc = launch_attn_decode_generic(st, nullptr, L.kq, L.ks, L.vq, L.vs, m->step,
                                                 L.global ? 2 : 1, nq, nkv, hd,
                                                 attn_generic_splits(L.slots), c.attn_scale,
                                                 m->part_g, nullptr, m->fx.xl_o, &post)))
                return rc;
        } else if ((rc = launch_attn_decode_fused(
                        st, m->q_raw, m->k_raw, v_src, L.q_norm, L.k_norm,
                        m->rope_cs + (L.global ? kHeadDim : 0), c.eps, m->step, L.global ? 2 : 1,
                        L.global ? 0u : L.slots, L.kq, L.ks, L.vq, L.vs, nq, nkv,
                        decode_splits(L), c.attn_scale, nullptr, ctx_workspace(m->ctx),
                        kWorkspaceBytes, m->fx.xl_o))) {
            return rc;
        }
        GemvTargets ot{};
        ot.w[0] = L.wo, ot.y[0] = m->o, ot.end[0] = H, ot.count = 1;
        GemvFuse eo{};
        eo.x_res = xa, eo.w_post = L.post_attn_norm, eo.w_next = L.ffn_norm;
        eo.u_out = m->fx.u, eo.A_out = m->fx.a, eo.B_out = m->fx.b, eo.part_out = m->fx.part;
        if ((rc = launch_gemv_fused(st, ot, m->fx.xl_o, (uint32_t)QD, pro_o, kEpiResid, eo)))
            return rc;
        GemvTargets gu{};
        gu.w[0] = L.wg, gu.w[1] = L.wu, gu.y[0] = m->g, gu.y[1] = m->u;
        gu.end[0] = F, gu.end[1] = 2 * F, gu.count = 2;
        GemvFuse pg{};
        pg.eps = c.eps;
        pg.part = m->fx.part, pg.np = np_o;
        pg.A = m->fx.a, pg.B = m->fx.b, pg.u = m->fx.u, pg.x_in = xa, pg.x_out = xb;
        pg.hl = static_cast<BlockLimbs *>(m->fx.hl);
        if ((rc = launch_gemv_fused(st, gu, nullptr, (uint32_t)H, kProNorm, kEpiGeglu, pg)))
            return rc;
        GemvTargets dt{};
        dt.w[0] = L.wd, dt.y[0] = m->f, dt.end[0] = H, dt.count = 1;
        GemvFuse ed{};
        ed.x_res = xb, ed.w_post = L.post_ffw_norm;
        ed.w_next = li + 1 < nl ? m->layers[li + 1].attn_norm : m->out_norm;
        ed.u_out = m->fx.u, ed.A_out = m->fx.a, ed.B_out = m->fx.b, ed.part_out = m->fx.part;
        if ((rc = launch_gemv_fused(st, dt, m->fx.hl, (uint32_t)F, pro_d, kEpiResid, ed)))
            return rc;
    }
    if (c.embed_q6k) {
        // the last layer's residual update and the output norm from the down
        // GEMV's partial sums, then the Q6_K head over the fp32 row
        hipLaunchKernelGGL(norm_from_partials_kernel, dim3(1), dim3(kRowWG), 0, st, m->fx.part,
                           np_d, m->fx.a, m->fx.b, m->layers[nl - 1].out_scale, H, c.eps, m->xf);
        SGQ_HIP(hipGetLastError());
        return launch_gemv_q6_k(st, m->embd, m->embd_stride, m->xf, logits, c.vocab, (uint32_t)H,
                                c.final_softcap);
    }
    GemvTargets head{};
    head.w[0] = m->embd, head.y[0] = logits, head.end[0] = (int)c.vocab, head.count = 1;
    head.softcap = c.final_softcap;
    GemvFuse ph{};
    ph.eps = c.eps;
    ph.part = m->fx.part, ph.np = np_d;
    ph.A = m->fx.a, ph.B = m->fx.b;
    ph.scale = m->layers[nl - 1].out_scale;
    return launch_gemv_fused(st, head, nullptr, (uint32_t)H, kProNorm, kEpiRows, ph);
}

}  // namespace

extern "C" {

void sgq_model_default_config(sgq_model_config *c) {
    std::memset(c, 0, sizeof *c);
    c->n_layers = 62;
    c->hidden = 5376;
    c->ffn = 21504;
    c->n_q_heads = 32;
    c->n_kv_heads = 16;
    c->head_dim = 128;
    c->vocab = 262144;
    c->sliding_window = 1024;
    c->global_every = 6;
    c->max_ctx = 16384;
    c->rope_theta_sliding = 10000.f;
    c->rope_theta_global = 1000000.f;
    c->global_rope_frac = 0.25f;
    c->eps = 1e-6f;
    c->attn_scale = 1.0f;
    c->final_softcap = 30.f;
    c->weight_sigma = 0.02f;
    c->seed = 0x5EED;
    c->global_k_eq_v = 1;
    c->prefill_chunk = 4096;
}

int sgq_model_create(sgq_ctx *ctx, const sgq_model_config *cfg, sgq_model **out) {
    if (!ctx || !cfg || !out) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    const sgq_model_config &c = *cfg;
    // per-kind geometry: sliding (head_dim, n_kv_heads) and global
    const uint32_t hd_s = c.head_dim, hd_g = c.head_dim_global ? c.head_dim_global : c.head_dim;
    const uint32_t kv_s = c.n_kv_heads, kv_g = c.n_kv_heads_global ? c.n_kv_heads_global : c.n_kv_heads;
    const bool generic = hd_s != kHeadDim || hd_g != kHeadDim || kv_g != kv_s || c.embed_q6k;
    auto ok_hd = [](uint32_t hd) { return hd == 128 || hd == 256 || hd == 512; };
    auto ok_qpk = [&](uint32_t kv) {
        if (kv == 0 || c.n_q_heads % kv) return false;
        const uint32_t r = c.n_q_heads / kv;
        return generic ? (r == 1 || r == 2 || r == 4 || r == 8) : r <= 2;
    };
    SGQ_CHECK(ok_hd(hd_s) && ok_hd(hd_g), "model: head_dim %u / %u (128, 256 or 512)", hd_s, hd_g);
    SGQ_CHECK(ok_qpk(kv_s) && ok_qpk(kv_g),
              "model: %u q heads over %u / %u kv heads (1 or 2 per kv head at the benchmark "
              "geometry, 1/2/4/8 otherwise)", c.n_q_heads, kv_s, kv_g);
    SGQ_CHECK(c.hidden % 256 == 0 && c.ffn % 256 == 0 && (c.n_q_heads * hd_s) % 256 == 0 &&
                  (c.n_q_heads * hd_g) % 256 == 0,
              "model: hidden, ffn and both layer kinds' q_dim must be multiples of 256");
    SGQ_CHECK(c.reserved == 0, "model: the reserved config field must be 0");
    SGQ_CHECK(c.hidden <= 16384, "model: hidden above 16384 (row kernels)");
    SGQ_CHECK(c.ffn <= 65536 && c.n_q_heads * std::max(hd_s, hd_g) <= 65536,
              "model: GEMV K above 65536");
    SGQ_CHECK(!c.embed_q6k || c.hidden <= 6144, "model: Q6_K head needs hidden <= 6144");
    SGQ_CHECK(c.n_layers >= 1 && c.vocab >= 1 && c.max_ctx >= 1 && c.sliding_window >= 1,
              "model: empty dimension");
    SGQ_CHECK(c.global_every >= 1, "model: global_every must be >= 1");
    SGQ_CHECK(c.global_rope_frac >= 0.f && c.global_rope_frac <= 1.f, "model: global_rope_frac");
    SGQ_CHECK(c.prefill_chunk >= 1 && c.prefill_chunk <= 65536, "model: prefill_chunk %u",
              c.prefill_chunk);
    if (int rc0 = gemv_prepare()) return rc0;
    if (int rc0 = attn_prepare()) return rc0;
    (void)device_info();
    auto *m = new sgq_model;
    m->ctx = ctx;
    m->cfg = c;
    m->generic = generic;
    m->mode = generic ? 2 : 0;
    const size_t H = c.hidden, F = c.ffn;
    const size_t QD_max = c.n_q_heads * std::max(hd_s, hd_g),
                 KD_max = std::max<size_t>((size_t)kv_s * hd_s, (size_t)kv_g * hd_g);
    int rc = SGQ_OK;
    auto fail_out = [&](int r) {
        sgq_model_destroy(m);
        return r;
    };
    uint64_t s = c.seed;
    if (c.embed_q6k) {
        m->embd_stride = ((H / 256) * 210 + 15) / 16 * 16;
        if ((rc = alloc(m, c.vocab * m->embd_stride, &m->embd)) ||
            (rc = launch_fill_q6k(ctx_stream(ctx), m->embd, c.vocab, (uint32_t)H, m->embd_stride,
                                  mix(s, 1))))
            return fail_out(rc);
    } else {
        m->embd_stride = (H / 32) * 18;
        if ((rc = q4_tensor(m, c.vocab, H, mix(s, 1), &m->embd))) return fail_out(rc);
    }
    if ((rc = f32_tensor(m, H, mix(s, 2), 1.0f, 0.1f, &m->out_norm))) return fail_out(rc);
    m->layers.resize(c.n_layers);
    for (uint32_t li = 0; li < c.n_layers; li++) {
        LayerW &L = m->layers[li];
        const uint64_t ls = mix(s, 1000 + li);
        L.global = (li % c.global_every) == c.global_every - 1;
        L.hd = L.global ? hd_g : hd_s;
        L.n_kv = L.global ? kv_g : kv_s;
        const size_t QD = c.n_q_heads * L.hd, KD = (size_t)L.n_kv * L.hd;
        if ((rc = q4_tensor(m, QD, H, mix(ls, 1), &L.wq)) || (rc = q4_tensor(m, KD, H, mix(ls, 2), &L.wk)) ||
            (!(L.global && c.global_k_eq_v) && (rc = q4_tensor(m, KD, H, mix(ls, 3), &L.wv))) ||
            (rc = q4_tensor(m, H, QD, mix(ls, 4), &L.wo)) ||
            (rc = q4_tensor(m, F, H, mix(ls, 5), &L.wg)) || (rc = q4_tensor(m, F, H, mix(ls, 6), &L.wu)) ||
            (rc = q4_tensor(m, H, F, mix(ls, 7), &L.wd)) ||
            (rc = f32_tensor(m, H, mix(ls, 8), 1.f, 0.1f, &L.attn_norm)) ||
            (rc = f32_tensor(m, L.hd, mix(ls, 9), 1.f, 0.1f, &L.q_norm)) ||
            (rc = f32_tensor(m, L.hd, mix(ls, 10), 1.f, 0.1f, &L.k_norm)) ||
            (rc = f32_tensor(m, H, mix(ls, 11), 1.f, 0.1f, &L.post_attn_norm)) ||
            (rc = f32_tensor(m, H, mix(ls, 12), 1.f, 0.1f, &L.ffn_norm)) ||
            (rc = f32_tensor(m, H, mix(ls, 13), 1.f, 0.1f, &L.post_ffw_norm)) ||
            (rc = f32_tensor(m, 1, mix(ls, 14), 0.9f, 0.05f, &L.out_scale)))
            return fail_out(rc);
        L.slots = L.global ? c.max_ctx : std::min(c.sliding_window, c.max_ctx);
        const size_t kvn = (size_t)L.slots * KD;
        if ((rc = alloc(m, kvn, reinterpret_cast<void **>(&L.kq))) ||
            (rc = alloc(m, kvn, reinterpret_cast<void **>(&L.vq))) ||
            (rc = alloc(m, kvn / 32 * 2, reinterpret_cast<void **>(&L.ks))) ||
            (rc = alloc(m, kvn / 32 * 2, reinterpret_cast<void **>(&L.vs))))
            return fail_out(rc);
    }
    float **acts[] = {&m->x, &m->q_raw, &m->k_raw, &m->v_raw, &m->q, &m->attn, &m->o, &m->g, &m->u, &m->f};
    const size_t act_n[] = {H, QD_max, KD_max, KD_max, QD_max, QD_max, H, F, F, 4 * H};  // f: up to 4 K-slices
    for (int i = 0; i < 10; i++)
        if ((rc = alloc(m, act_n[i] * 4, reinterpret_cast<void **>(acts[i])))) return fail_out(rc);
    if ((rc = alloc(m, std::max({H, F, QD_max}) / 32 * sizeof(BlockLimbs), &m->xl))) return fail_out(rc);
    {
        float **fb[] = {&m->fx.xb, &m->fx.u, &m->fx.a, &m->fx.b};
        for (float **b : fb)
            if ((rc = alloc(m, H * 4, reinterpret_cast<void **>(b)))) return fail_out(rc);
        if ((rc = alloc(m, kGemvMaxPartials * sizeof(float4), reinterpret_cast<void **>(&m->fx.part))) ||
            (rc = alloc(m, QD_max / 32 * sizeof(BlockLimbs), &m->fx.xl_o)) ||
            (rc = alloc(m, F / 32 * sizeof(BlockLimbs), &m->fx.hl)))
            return fail_out(rc);
    }
    if ((rc = alloc(m, 64, reinterpret_cast<void **>(&m->step)))) return fail_out(rc);
    if ((rc = alloc(m, 2 * kHeadDim * 4, reinterpret_cast<void **>(&m->rope_cs))))
        return fail_out(rc);
    {   // mode 3 buffers
        uint32_t max_splits = 1;
        for (const LayerW &L : m->layers) max_splits = std::max<uint32_t>(max_splits, attn_generic_splits(L.slots));
        if ((rc = alloc(m, (hd_s + hd_g) * 4, reinterpret_cast<void **>(&m->rope_g))) ||
            (rc = alloc(m, KD_max * 4, reinterpret_cast<void **>(&m->kx))) ||
            (rc = alloc(m, KD_max * 4, reinterpret_cast<void **>(&m->vx))) ||
            (rc = alloc(m, (size_t)c.n_q_heads * max_splits * (std::max(hd_s, hd_g) + 2) * 4,
                        reinterpret_cast<void **>(&m->part_g))) ||
            (rc = alloc(m, H * 4, reinterpret_cast<void **>(&m->xf))) ||
            (rc = alloc(m, (size_t)c.vocab * 4, reinterpret_cast<void **>(&m->logits_tmp))))
            return fail_out(rc);
    }
    if (hipStreamSynchronize(ctx_stream(ctx)) != hipSuccess) return fail_out(fail(SGQ_ERR_HIP, "init sync"));
    *out = m;
    return SGQ_OK;
}

int sgq_model_destroy(sgq_model *m) {
    if (!m) return SGQ_OK;
    if (m->graph) sgq_graph_destroy(m->graph);
    (void)hipDeviceSynchronize();
    for (void *p : m->allocs) (void)hipFree(p);
    delete m;
    return SGQ_OK;
}

int sgq_model_reset(sgq_model *m) {
    if (!m) return fail(SGQ_ERR_VALIDATION, "NULL model");
    m->pos = 0;
    return SGQ_OK;
}

uint32_t sgq_model_position(const sgq_model *m) { return m ? m->pos : 0; }

static int write_step(sgq_model *m, uint32_t token) {
    const sgq_model_config &c = m->cfg;
    SGQ_CHECK(token < c.vocab, "model: token %u >= vocab %u", token, c.vocab);
    SGQ_CHECK(m->pos < c.max_ctx, "model: context full (%u)", c.max_ctx);
    const uint32_t kv_sl = std::min(m->pos + 1, std::min(c.sliding_window, c.max_ctx));
    hipLaunchKernelGGL(model_step_kernel, dim3(1), dim3(kHeadDim), 0, ctx_stream(m->ctx), m->step,
                       m->pos, kv_sl, m->pos + 1, m->pos, token, m->rope_cs,
                       c.rope_theta_sliding, c.rope_theta_global,
                       (int)lroundf(c.global_rope_frac * kHeadDim / 2));
    SGQ_HIP(hipGetLastError());
    if (m->mode == 3 || m->generic) {
        const int hd_s = (int)c.head_dim, hd_g = (int)(c.head_dim_global ? c.head_dim_global : c.head_dim);
        hipLaunchKernelGGL(rope_table_generic_kernel, dim3((hd_s / 2 + hd_g / 2 + 255) / 256),
                           dim3(256), 0, ctx_stream(m->ctx), m->step, m->rope_g, hd_s, hd_g,
                           c.rope_theta_sliding, c.rope_theta_global,
                           (int)lroundf(c.global_rope_frac * hd_g / 2));
        SGQ_HIP(hipGetLastError());
    }
    return SGQ_OK;
}

int sgq_model_decode(sgq_model *m, uint32_t token, float *logits) {
    if (!m || !logits) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    int rc = write_step(m, token);
    if (rc) return rc;
    if ((rc = m->mode == 2   ? record_step_fused(m, logits)
               : m->mode == 3 ? record_step_generic(m, logits, true)
                              : record_step(m, logits)))
        return rc;
    m->pos++;
    return SGQ_OK;
}

int sgq_model_decode_graph(sgq_model *m, uint32_t token, float *logits) {
    if (!m || !logits) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    SGQ_CHECK(ctx_stream(m->ctx) != nullptr,
              "model: graph decode needs a non-null stream (sgq_ctx_set_stream)");
    int rc = write_step(m, token);
    if (rc) return rc;
    if (!m->graph || m->graph_logits != logits) {
        if (m->graph) {
            sgq_graph_destroy(m->graph);
            m->graph = nullptr;
        }
        if ((rc = sgq_graph_begin(m->ctx))) return rc;
        rc = m->mode == 2   ? record_step_fused(m, logits)
             : m->mode == 3 ? record_step_generic(m, logits, true)
                            : record_step(m, logits);
        sgq_graph *g = nullptr;
        const int rc2 = sgq_graph_end(m->ctx, &g);
        if (rc) {
            if (g) sgq_graph_destroy(g);
            return rc;
        }
        if (rc2) return rc2;
        m->graph = g;
        m->graph_logits = logits;
    }
    if ((rc = sgq_graph_submit(m->ctx, m->graph))) return rc;
    m->pos++;
    return SGQ_OK;
}

int sgq_model_set_decode_mode(sgq_model *m, int mode) {
    if (!m) return fail(SGQ_ERR_VALIDATION, "NULL model");
    SGQ_CHECK(mode == 0 || mode == 2 || mode == 3,
              "model: decode mode %d (0 kernels, 2 fused, 3 any geometry; 1, a persistent "
              "one-launch step, measured slower and was removed)", mode);
    SGQ_CHECK(!m->generic || mode >= 2,
              "model: this geometry (head_dim %u/%u, Q6_K embedding %u) runs in modes 2 and 3 only",
              m->cfg.head_dim, m->cfg.head_dim_global, m->cfg.embed_q6k);
    if (mode != m->mode && m->graph) {  // a captured step belongs to one mode
        sgq_graph_destroy(m->graph);
        m->graph = nullptr;
    }
    m->mode = mode;
    return SGQ_OK;
}

int sgq_model_decode_mode(const sgq_model *m) { return m ? m->mode : -1; }

int sgq_model_status(sgq_model *m) {
    if (!m) return fail(SGQ_ERR_VALIDATION, "NULL model");
    SGQ_HIP(hipStreamSynchronize(ctx_stream(m->ctx)));
    return SGQ_OK;
}

int sgq_model_fill_cache(sgq_model *m, uint32_t n_tokens, uint64_t seed) {
    if (!m) return fail(SGQ_ERR_VALIDATION, "NULL model");
    const sgq_model_config &c = m->cfg;
    SGQ_CHECK(n_tokens <= c.max_ctx, "model: fill_cache %u > max_ctx %u", n_tokens, c.max_ctx);
    hipStream_t st = ctx_stream(m->ctx);
    size_t most = 0;
    for (const LayerW &L : m->layers)
        most = std::max(most, (size_t)std::min(n_tokens, L.slots) * L.n_kv * L.hd);
    float *tmp = nullptr;
    if (most) SGQ_HIP(hipMalloc(&tmp, most * 4));
    int rc = SGQ_OK;
    for (size_t li = 0; li < m->layers.size() && !rc; li++) {
        const LayerW &L = m->layers[li];
        const size_t KD = (size_t)L.n_kv * L.hd;
        const size_t rows = std::min(n_tokens, L.slots);
        if (!rows) continue;
        for (int kv = 0; kv < 2 && !rc; kv++) {
            rc = launch_fill_normal(st, tmp, rows * KD, mix(seed, li * 2 + kv), 0.f, 1.f);
            if (!rc)
                rc = launch_quant_q8_0(st, tmp, kv ? L.vs : L.ks, kv ? L.vq : L.kq, rows * KD);
        }
    }
    if (tmp) {
        const hipError_t e = hipStreamSynchronize(st);
        (void)hipFree(tmp);
        if (!rc && e != hipSuccess) rc = check_hip(e, "fill_cache sync");
    }
    if (!rc) m->pos = n_tokens;
    return rc;
}

}  // extern "C"

namespace {

// Split-K factor for an MMQ of m×n×k: enough (tile, split) work items to fill
// the chip's workgroup slots, at least 16 blocks of K per split.
uint32_t mmq_split(uint32_t m, uint32_t n, uint32_t k) {
    const uint64_t tiles = (uint64_t)((m + 127) / 128) * ((n + 127) / 128);
    uint32_t split = 1;
    while (split < 8 && tiles * split * 2 <= 1024 && (k / 32) / (split * 2) >= 16) split *= 2;
    return split;
}
constexpr size_t kPfPartialFloats = 1024ull * 128 * 128;  // >= split·m·n for every choice above

int pf_alloc(sgq_model *m) {
    const sgq_model_config &c = m->cfg;
    const size_t C = c.prefill_chunk, H = c.hidden, F = c.ffn;
    size_t QD = 0, KD = 0, HD2 = 0;  // widest layer; both kinds' rope pairs
    for (const LayerW &L : m->layers) {
        QD = std::max<size_t>(QD, (size_t)c.n_q_heads * L.hd);
        KD = std::max<size_t>(KD, (size_t)L.n_kv * L.hd);
    }
    HD2 = c.head_dim + (c.head_dim_global ? c.head_dim_global : c.head_dim);
    auto &p = m->pf;
    void **f32s[] = {(void **)&p.x, (void **)&p.q_raw, (void **)&p.k_raw, (void **)&p.v_raw,
                     (void **)&p.q, (void **)&p.attn, (void **)&p.o, (void **)&p.g,
                     (void **)&p.u, (void **)&p.f, (void **)&p.part, (void **)&p.head_in,
                     (void **)&p.rope};
    const size_t f32n[] = {C * H, C * QD, C * KD, C * KD, C * QD, C * QD, C * H, C * F, C * F,
                           C * H, kPfPartialFloats, H, C * HD2};
    int rc;
    for (int i = 0; i < 13; i++)
        if ((rc = alloc(m, f32n[i] * 4, f32s[i]))) return rc;
    void **q8s[] = {(void **)&p.xq, (void **)&p.aq, (void **)&p.hq, (void **)&p.ckq, (void **)&p.cvq};
    void **scs[] = {(void **)&p.xs, (void **)&p.as, (void **)&p.hs, (void **)&p.cks, (void **)&p.cvs};
    const size_t q8n[] = {C * H, C * QD, C * F, C * KD, C * KD};
    for (int i = 0; i < 5; i++)
        if ((rc = alloc(m, q8n[i], q8s[i])) || (rc = alloc(m, q8n[i] / 32 * 2, scs[i]))) return rc;
    if ((rc = alloc(m, C * 4, (void **)&p.tok))) return rc;
    p.chunk = (uint32_t)C;
    return SGQ_OK;
}

int mmq(sgq_model *m, hipStream_t st, const void *w, const int8_t *xq, const uint16_t *xs,
        float *y, uint32_t M, uint32_t n, uint32_t k) {
    const uint32_t split = mmq_split(M, n, k);
    // split 1: the partials buffer lets the last part-filled round of tiles
    // split over K (at most one round of 128x128 tiles: 2 per CU)
    const bool tail_ok = (uint64_t)M * n <= kPfPartialFloats ||
                         2ull * device_info().cus * 128 * 128 <= kPfPartialFloats;
    return launch_gemm_q4_0_q8(st, w, xq, xs, y, M, n, k, split,
                               split > 1 || tail_ok ? m->pf.part : nullptr);
}

// One chunk of M tokens at positions q0..q0+M-1 (tokens already on the device).
int pf_chunk(sgq_model *m, uint32_t M, uint32_t q0) {
    const sgq_model_config &c = m->cfg;
    hipStream_t st = ctx_stream(m->ctx);
    auto &p = m->pf;
    const uint32_t H = c.hidden, F = c.ffn, nq = c.n_q_heads;
    const int hd_s = (int)c.head_dim, hd_g = (int)(c.head_dim_global ? c.head_dim_global : c.head_dim);
    int rc;
    const int live = (int)lroundf(c.global_rope_frac * hd_g / 2);
    hipLaunchKernelGGL(pf_rope_table_kernel, dim3((M * (hd_s / 2 + hd_g / 2) + 255) / 256),
                       dim3(256), 0, st, p.rope, (int)q0, (int)M, hd_s, hd_g, c.rope_theta_sliding,
                       c.rope_theta_global, live);
    if (c.embed_q6k)
        hipLaunchKernelGGL(pf_embed_q6k_norm_q8_kernel, dim3(M), dim3(kPfWG), 0, st,
                           static_cast<const uint8_t *>(m->embd), m->embd_stride, p.tok, (int)H,
                           sqrtf((float)H), m->layers[0].attn_norm, c.eps, p.x, p.xq, p.xs);
    else
        hipLaunchKernelGGL(pf_embed_norm_q8_kernel, dim3(M), dim3(kPfWG), 0, st,
                           static_cast<const uint8_t *>(m->embd), p.tok, (int)H, sqrtf((float)H),
                           m->layers[0].attn_norm, c.eps, p.x, p.xq, p.xs);
    SGQ_HIP(hipGetLastError());
    for (size_t li = 0; li < m->layers.size(); li++) {
        const LayerW &L = m->layers[li];
        const uint32_t hd = L.hd, nkv = L.n_kv, QD = nq * hd, KD = nkv * hd;
        if ((rc = mmq(m, st, L.wq, p.xq, p.xs, p.q_raw, M, QD, H)) ||
            (rc = mmq(m, st, L.wk, p.xq, p.xs, p.k_raw, M, KD, H)))
            return rc;
        if (L.wv && (rc = mmq(m, st, L.wv, p.xq, p.xs, p.v_raw, M, KD, H))) return rc;
        const float *rope = p.rope + (L.global ? (size_t)M * hd_s : 0);
        const float *v_src = L.wv ? p.v_raw : p.k_raw;
        const long prow = (long)M * (nq + 2 * nkv);  // (token, head row) pairs
#define SGQ_PF_WIDE(HDV)                                                                           \
    hipLaunchKernelGGL(pf_qkv_post_wide_kernel<HDV>,                                             \
                       dim3((unsigned)((prow + 4 * (HDV == 128 ? 2 : 1) - 1) /                     \
                                       (4 * (HDV == 128 ? 2 : 1)))),                              \
                       dim3(256), 0, st, p.q_raw,                                                 \
                       p.k_raw, v_src, L.q_norm, L.k_norm, rope, (int)nq, (int)nkv, (int)M, c.eps, \
                       p.q, p.ckq, p.cks, p.cvq, p.cvs)
        if (hd == 128) SGQ_PF_WIDE(128);
        else if (hd == 256) SGQ_PF_WIDE(256);
        else SGQ_PF_WIDE(512);
#undef SGQ_PF_WIDE
        SGQ_HIP(hipGetLastError());
        const int ring = L.global ? 0 : (int)L.slots;
        const int window = L.global ? 0 : (int)std::min(c.sliding_window, L.slots);
        if ((rc = launch_attn_prefill_q8(st, p.q, L.kq, L.ks, L.vq, L.vs, p.attn, (int)M, (int)q0,
                                         (int)nq, (int)nkv, (int)hd, window,
                                         c.attn_scale, ring, p.ckq, p.cks, p.cvq, p.cvs)))
            return rc;
        {
            const int i0 = ring && (int)M > ring ? (int)M - ring : 0;
            const long threads = (long)(M - i0) * (KD / 16);
            hipLaunchKernelGGL(pf_kv_append_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256),
                               0, st, p.ckq, p.cks, p.cvq, p.cvs, L.kq, L.ks, L.vq, L.vs, (int)M,
                               (int)q0, ring, (int)KD);
            SGQ_HIP(hipGetLastError());
        }
        if ((rc = launch_quant_q8_0(st, p.attn, p.as, p.aq, (uint64_t)M * QD))) return rc;
        if ((rc = mmq(m, st, L.wo, p.aq, p.as, p.o, M, H, QD))) return rc;
        hipLaunchKernelGGL(pf_residual_norm_q8_kernel, dim3(M), dim3(kPfWG), 0, st, p.o,
                           L.post_attn_norm, p.x, (const float *)nullptr, L.ffn_norm, (int)H,
                           c.eps, p.xq, p.xs);
        SGQ_HIP(hipGetLastError());
        if ((rc = mmq(m, st, L.wg, p.xq, p.xs, p.g, M, F, H)) ||
            (rc = mmq(m, st, L.wu, p.xq, p.xs, p.u, M, F, H)))
            return rc;
        const uint64_t n4 = (uint64_t)M * F / 4;
        hipLaunchKernelGGL(pf_geglu_q8_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st,
                           reinterpret_cast<const float4 *>(p.g), reinterpret_cast<const float4 *>(p.u),
                           n4, reinterpret_cast<int *>(p.hq), p.hs);
        SGQ_HIP(hipGetLastError());
        if ((rc = mmq(m, st, L.wd, p.hq, p.hs, p.f, M, H, F))) return rc;
        const float *w_next = li + 1 < m->layers.size() ? m->layers[li + 1].attn_norm : m->out_norm;
        hipLaunchKernelGGL(pf_residual_norm_q8_kernel, dim3(M), dim3(kPfWG), 0, st, p.f,
                           L.post_ffw_norm, p.x, L.out_scale, w_next, (int)H, c.eps, p.xq, p.xs);
        SGQ_HIP(hipGetLastError());
    }
    return SGQ_OK;
}

}  // namespace

extern "C" {

int sgq_model_prefill(sgq_model *m, const uint32_t *tokens, uint32_t n_tokens, float *logits) {
    if (!m || !tokens) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    const sgq_model_config &c = m->cfg;
    SGQ_CHECK(n_tokens >= 1, "model: empty prompt");
    SGQ_CHECK((uint64_t)m->pos + n_tokens <= c.max_ctx, "model: prompt of %u at position %u exceeds max_ctx %u",
              n_tokens, m->pos, c.max_ctx);
    for (uint32_t i = 0; i < n_tokens; i++)
        SGQ_CHECK(tokens[i] < c.vocab, "model: token %u at %u >= vocab %u", tokens[i], i, c.vocab);
    int rc;
    if (!m->pf.chunk && (rc = pf_alloc(m))) return rc;
    hipStream_t st = ctx_stream(m->ctx);
    uint32_t M = 0;
    for (uint32_t c0 = 0; c0 < n_tokens; c0 += M) {
        M = std::min(m->pf.chunk, n_tokens - c0);
        SGQ_HIP(hipMemcpyAsync(m->pf.tok, tokens + c0, (size_t)M * 4, hipMemcpyHostToDevice, st));
        SGQ_HIP(hipStreamSynchronize(st));  // the host array may go away
        if ((rc = pf_chunk(m, M, m->pos))) return rc;
        m->pos += M;
    }
    if (logits) {  // the last token's logits: output norm, limbs, tied head with softcap
        const uint32_t H = c.hidden;
        if ((rc = launch_rmsnorm(st, m->pf.x + (size_t)(M - 1) * H, m->out_norm, m->pf.head_in, 1, H, 0,
                                 c.eps)))
            return rc;
        if (c.embed_q6k)
            return launch_gemv_q6_k(st, m->embd, m->embd_stride, m->pf.head_in, logits, c.vocab, H,
                                    c.final_softcap);
        if ((rc = launch_quant_limbs(st, m->pf.head_in, m->xl, H))) return rc;
        GemvTargets head{};
        head.w[0] = m->embd, head.y[0] = logits, head.end[0] = (int)c.vocab, head.count = 1;
        head.softcap = c.final_softcap;
        if ((rc = launch_gemv_limbs(st, head, m->xl, H))) return rc;
    }
    return SGQ_OK;
}

int sgq_model_load_gguf(sgq_model *m, const sgq_gguf *g) {
    if (!m || !g) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    const sgq_model_config &c = m->cfg;
    const uint64_t H = c.hidden, F = c.ffn;
    // the tensor table of crates/sg-gguf/src/desc.rs:150-193 at this model's
    // geometry: per-kind q/kv dims and norm lengths, attn_v absent on layers
    // that share K=V, token_embd Q4_0 or Q6_K (type 14)
    constexpr uint32_t kQ6K = 14;
    struct Want {
        std::string name;
        const char *model_name;
        int layer;
        uint32_t type;  // 0 F32, 2 Q4_0, 14 Q6_K
        uint64_t d0, d1;
    };
    std::vector<Want> want = {{"token_embd.weight", "token_embd", -1, c.embed_q6k ? kQ6K : 2u, H, c.vocab},
                              {"output_norm.weight", "output_norm", -1, 0, H, 1}};
    for (uint32_t l = 0; l < c.n_layers; l++) {
        const LayerW &L = m->layers[l];
        const uint64_t QD = (uint64_t)c.n_q_heads * L.hd, KD = (uint64_t)L.n_kv * L.hd;
        const std::string b = "blk." + std::to_string(l) + ".";
        want.push_back({b + "attn_q.weight", "attn_q", (int)l, 2, H, QD});
        want.push_back({b + "attn_k.weight", "attn_k", (int)l, 2, H, KD});
        if (L.wv) want.push_back({b + "attn_v.weight", "attn_v", (int)l, 2, H, KD});
        want.push_back({b + "attn_output.weight", "attn_output", (int)l, 2, QD, H});
        want.push_back({b + "attn_q_norm.weight", "attn_q_norm", (int)l, 0, L.hd, 1});
        want.push_back({b + "attn_k_norm.weight", "attn_k_norm", (int)l, 0, L.hd, 1});
        want.push_back({b + "attn_norm.weight", "attn_norm", (int)l, 0, H, 1});
        want.push_back({b + "post_attention_norm.weight", "post_attention_norm", (int)l, 0, H, 1});
        want.push_back({b + "ffn_norm.weight", "ffn_norm", (int)l, 0, H, 1});
        want.push_back({b + "post_ffw_norm.weight", "post_ffw_norm", (int)l, 0, H, 1});
        want.push_back({b + "ffn_gate.weight", "ffn_gate", (int)l, 2, H, F});
        want.push_back({b + "ffn_up.weight", "ffn_up", (int)l, 2, H, F});
        want.push_back({b + "ffn_down.weight", "ffn_down", (int)l, 2, F, H});
        want.push_back({b + "layer_output_scale.weight", "layer_output_scale", (int)l, 0, 1, 1});
    }
    // Check everything before writing anything.
    std::vector<sgq_gguf_tensor> found(want.size());
    for (size_t i = 0; i < want.size(); i++) {
        const Want &w = want[i];
        if (int rc = sgq_gguf_tensor_find(g, w.name.c_str(), &found[i])) return rc;
        const sgq_gguf_tensor &t = found[i];
        const uint64_t t1 = t.n_dims >= 2 ? t.dims[1] : 1;
        if (t.type != w.type || t.dims[0] != w.d0 || t1 != w.d1 || t.n_dims > 2)
            return fail(SGQ_ERR_VALIDATION,
                        "gguf: tensor '%s' is type %u [%llu, %llu]; the model needs type %u [%llu, %llu]",
                        w.name.c_str(), t.type, (unsigned long long)t.dims[0], (unsigned long long)t1,
                        w.type, (unsigned long long)w.d0, (unsigned long long)w.d1);
    }
    sgq_gguf_tensor rf;
    if (sgq_gguf_tensor_find(g, "rope_freqs.weight", &rf) == SGQ_OK) {
        // divisor factors of the global layers' partial rotation (rope.rs:13-16)
        const int half = (int)(c.head_dim_global ? c.head_dim_global : c.head_dim) / 2;
        const int live = (int)lroundf(c.global_rope_frac * half);
        SGQ_CHECK(rf.type == 0 && rf.dims[0] == (uint64_t)half && rf.n_dims == 1,
                  "gguf: rope_freqs.weight must be F32 [%d]", half);
        const float *f = static_cast<const float *>(rf.data);
        for (int i = 0; i < half; i++)
            SGQ_CHECK(i < live ? f[i] == 1.0f : f[i] >= 1e20f,
                      "gguf: rope_freqs.weight[%d] = %g does not match global_rope_frac", i, f[i]);
    }
    hipStream_t st = ctx_stream(m->ctx);
    for (size_t i = 0; i < want.size(); i++) {
        void *dst;
        uint64_t bytes;
        if (int rc = sgq_model_tensor(m, want[i].layer, want[i].model_name, &dst, &bytes)) return rc;
        if (want[i].type == kQ6K) {
            // GGUF rows are k/256·210 bytes; the device rows are padded
            const uint64_t row = (H / 256) * 210;
            SGQ_CHECK(found[i].bytes == row * c.vocab, "gguf: token_embd is %llu bytes, not %llu",
                      (unsigned long long)found[i].bytes, (unsigned long long)(row * c.vocab));
            SGQ_HIP(hipMemsetAsync(dst, 0, bytes, st));
            SGQ_HIP(hipMemcpy2DAsync(dst, m->embd_stride, found[i].data, row, row, c.vocab,
                                     hipMemcpyHostToDevice, st));
            continue;
        }
        SGQ_CHECK(bytes == found[i].bytes, "gguf: tensor '%s' is %llu bytes, the model's %llu",
                  want[i].name.c_str(), (unsigned long long)found[i].bytes, (unsigned long long)bytes);
        SGQ_HIP(hipMemcpyAsync(dst, found[i].data, bytes, hipMemcpyHostToDevice, st));
    }
    SGQ_HIP(hipStreamSynchronize(st));
    return SGQ_OK;
}

int sgq_model_tensor(const sgq_model *m, int layer, const char *name, void **ptr,
                     uint64_t *bytes) {
    if (!m || !name || !ptr || !bytes) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    const sgq_model_config &c = m->cfg;
    const uint32_t hd_max = std::max(c.head_dim, c.head_dim_global);
    const size_t H = c.hidden, F = c.ffn, QD = c.n_q_heads * hd_max;
    size_t KD = 0;
    for (const LayerW &L : m->layers) KD = std::max(KD, (size_t)L.n_kv * L.hd);
    auto q4 = [](size_t r, size_t k) { return (uint64_t)(r * (k / 32) * 18); };
    std::string n(name);
    if (layer < 0) {
        // token_embd: Q4_0 rows, or Q6_K rows padded to embd_stride bytes
        if (n == "token_embd") { *ptr = m->embd; *bytes = (uint64_t)c.vocab * m->embd_stride; return SGQ_OK; }
        if (n == "output_norm") { *ptr = m->out_norm; *bytes = H * 4; return SGQ_OK; }
        if (n == "x") { *ptr = m->x; *bytes = H * 4; return SGQ_OK; }
        // decode-step activations (the last layer's, after a step)
        const struct { const char *n; void *p; uint64_t b; } acts[] = {
            {"q_raw", m->q_raw, QD * 4}, {"k_raw", m->k_raw, KD * 4}, {"v_raw", m->v_raw, KD * 4},
            {"attn_out", m->attn, QD * 4}, {"x_mid", m->fx.xb, H * 4},
            {"resid_u", m->fx.u, H * 4}, {"resid_a", m->fx.a, H * 4}, {"resid_b", m->fx.b, H * 4},
            {"resid_partials", m->fx.part, kGemvMaxPartials * 16},
            {"attn_out_limbs", m->fx.xl_o, QD / 32 * sizeof(BlockLimbs)},
            {"ffn_limbs", m->fx.hl, F / 32 * sizeof(BlockLimbs)},
        };
        for (const auto &e : acts)
            if (n == e.n) {
                *ptr = e.p;
                *bytes = e.b;
                return SGQ_OK;
            }
        if (n == "prefill_x") {  // residual rows of the last prefill chunk
            SGQ_CHECK(m->pf.chunk, "model: no prefill has run (prefill_x)");
            *ptr = m->pf.x;
            *bytes = (size_t)m->pf.chunk * H * 4;
            return SGQ_OK;
        }
        return fail(SGQ_ERR_VALIDATION, "model: no global tensor '%s'", name);
    }
    SGQ_CHECK(layer < (int)m->layers.size(), "model: layer %d out of range", layer);
    const LayerW &L = m->layers[layer];
    struct E { const char *n; void *p; uint64_t b; };
    const size_t hd = L.hd;
    const size_t QDl = c.n_q_heads * hd, KDl = (size_t)L.n_kv * hd;
    const uint64_t kvn = (uint64_t)L.slots * KDl;
    const E table[] = {
        {"attn_q", L.wq, q4(QDl, H)}, {"attn_k", L.wk, q4(KDl, H)}, {"attn_v", L.wv, q4(KDl, H)},
        {"attn_output", L.wo, q4(H, QDl)}, {"ffn_gate", L.wg, q4(F, H)}, {"ffn_up", L.wu, q4(F, H)},
        {"ffn_down", L.wd, q4(H, F)}, {"attn_norm", L.attn_norm, H * 4},
        {"attn_q_norm", L.q_norm, hd * 4}, {"attn_k_norm", L.k_norm, hd * 4},
        {"post_attention_norm", L.post_attn_norm, H * 4}, {"ffn_norm", L.ffn_norm, H * 4},
        {"post_ffw_norm", L.post_ffw_norm, H * 4}, {"layer_output_scale", L.out_scale, 4},
        {"k_quants", L.kq, kvn}, {"v_quants", L.vq, kvn}, {"k_scales", L.ks, kvn / 16},
        {"v_scales", L.vs, kvn / 16},
    };
    for (const E &e : table)
        if (n == e.n && e.p) {
            *ptr = e.p;
            *bytes = e.b;
            return SGQ_OK;
        }
    return fail(SGQ_ERR_VALIDATION, "model: no layer tensor '%s'", name);
}

}  // extern "C"
