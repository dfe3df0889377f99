// Q8_0-KV attention for gfx950: split-K decode.
//
// Semantics: attn_decode_global_q8k / attn_decode_sliding + attn_reduce
// (crates/sg-gpu/shaders/attn_decode_global_q8k.wgsl:41-112,
// attn_reduce.wgsl:24-57): for each query head h (GQA: kv head h/QPK),
// s_t = scale · q_h·k_t over the valid cache slots t < kv_len (physical
// order), softmax, out_h = Σ p_t v_t.  K and V are Q8_0 pages in the
// structure-of-arrays format (int8 quants [slot × n_kv × hd], f16 scales
// [slot × n_kv × hd/32], 32-blocks along head_dim), dequantized on the fly
// as f16(d)·q — the reference keeps V in f16; here both K and V are Q8_0.
//
// Design (HBM-bound: 2·(hd + hd/16) bytes per slot and kv head against
// ~QPK·4·hd flops):
//  * Grid [n_kv, n_splits]: each workgroup streams one kv head's slots of one
//    contiguous chunk, 256 slots at a time: thread i scores slot i for all
//    QPK query heads (K row = 128 B = one cache line; q from LDS,
//    broadcast), the sub-chunk's scores go through an online softmax
//    (m, l, rescaled acc), and PV runs with thread (head, 4-dim word, slot
//    group) so that a wave reads whole V rows.
//  * Each workgroup writes its (acc, m, l) partial; a small merge kernel
//    (one workgroup per kv head) combines them in split order 0..S-1, the
//    fixed order of attn_reduce.wgsl:40-52.  A second launch is cheaper
//    than merging in the same launch: that needs a device-scope release
//    fence per workgroup, which on a multi-XCD part writes back L2.
//    Empty splits carry (m = -3e38, l = 0, acc = 0).
//  * K row, V row and both scale words of a slot are issued together, so a
//    sub-chunk costs one memory round trip; V is staged in LDS for PV.
#include "limbs.h"

namespace sgq {
namespace {

constexpr int kHD = 128;
constexpr int kAWG = 256;
constexpr int kSub = 256;             // slots scored per pass
constexpr float kNegBig = -3.0e38f;

// Dequantized dot of a 128-wide K row (int8 + 4 f16 scales) with q (LDS).
__device__ __forceinline__ float k_row_dot(const int4 (&kr)[8], const float (&ksc)[4],
                                           const float *qs) {
    float s = 0.f;
#pragma unroll
    for (int b = 0; b < 4; b++) {
        float part = 0.f;
#pragma unroll
        for (int c = 0; c < 2; c++) {
            const int4 v = kr[2 * b + c];
            const int w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float4 q4 = *reinterpret_cast<const float4 *>(qs + 32 * b + 16 * c + 4 * e);
                part = __builtin_fmaf(q4.x, (float)(int8_t)(w[e] & 0xff), part);
                part = __builtin_fmaf(q4.y, (float)(int8_t)((w[e] >> 8) & 0xff), part);
                part = __builtin_fmaf(q4.z, (float)(int8_t)((w[e] >> 16) & 0xff), part);
                part = __builtin_fmaf(q4.w, (float)(int8_t)((w[e] >> 24) & 0xff), part);
            }
        }
        s = __builtin_fmaf(ksc[b], part, s);
    }
    return s;
}

template <int QPK>
__global__ __launch_bounds__(kAWG) void attn_decode_q8_kernel(
    const float *__restrict__ q, const int8_t *__restrict__ kq, const uint16_t *__restrict__ ks,
    const int8_t *__restrict__ vq, const uint16_t *__restrict__ vs,
    const uint32_t *__restrict__ step, int step_word, uint32_t kv_len_direct, int n_kv,
    int n_splits, float scale, float *__restrict__ part) {
    constexpr int G = kAWG / (QPK * (kHD / 4));  // slot groups in the PV phase
    static_assert(G >= 1, "QPK too large for one workgroup");
    constexpr int kVRow = kHD / 4 + 4;           // V row in LDS, ints (padded)
    __shared__ __align__(16) float q_s[QPK][kHD];
    __shared__ float s_s[QPK][kSub];             // probabilities of the sub-chunk
    __shared__ float vs_s[kSub][kHD / 32];       // V scales of the sub-chunk
    __shared__ __align__(16) int v_s[kSub][kVRow];  // V quants of the sub-chunk
    __shared__ float red[QPK][kAWG / kWave];
    __shared__ float acc_s[G][QPK][kHD];

    const int kvh = blockIdx.x, split = blockIdx.y, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const uint32_t kv_len = step ? step[step_word] : kv_len_direct;
    const uint32_t chunk = (kv_len + n_splits - 1) / n_splits;
    const uint32_t t_begin = min((uint32_t)split * chunk, kv_len);
    const uint32_t t_end = min(t_begin + chunk, kv_len);

    for (int i = tid; i < QPK * kHD; i += kAWG)
        q_s[i / kHD][i % kHD] = q[(size_t)(kvh * QPK) * kHD + i];

    // PV thread role: head ph, 4-dim word pw, slot group pg
    const int ph = tid / (kHD / 4) % QPK, pw = tid % (kHD / 4), pg = tid / (QPK * kHD / 4);
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    float m_run[QPK], l_run[QPK];
#pragma unroll
    for (int h = 0; h < QPK; h++) {
        m_run[h] = kNegBig;
        l_run[h] = 0.f;
    }

    for (uint32_t base = t_begin; base < t_end; base += kSub) {
        const int n_here = (int)min((uint32_t)kSub, t_end - base);
        const int t = tid;
        // ---- one slot per thread: K row, V row and both scale words issued
        // together (one memory round trip for the whole sub-chunk)
        int4 kr[8], vr[8];
        uint2 kss = {0u, 0u}, vss = {0u, 0u};
        if (t < n_here) {
            const size_t row = (size_t)(base + t) * n_kv + kvh;
            const int4 *kp = reinterpret_cast<const int4 *>(kq + row * kHD);
            const int4 *vp = reinterpret_cast<const int4 *>(vq + row * kHD);
#pragma unroll
            for (int c = 0; c < 8; c++) kr[c] = kp[c];
#pragma unroll
            for (int c = 0; c < 8; c++) vr[c] = vp[c];
            kss = *reinterpret_cast<const uint2 *>(ks + row * (kHD / 32));
            vss = *reinterpret_cast<const uint2 *>(vs + row * (kHD / 32));
        }
        __syncthreads();  // q_s ready; previous sub-chunk's LDS reads done
        float sc[QPK];
        if (t < n_here) {
#pragma unroll
            for (int c = 0; c < 8; c++) *reinterpret_cast<int4 *>(&v_s[t][4 * c]) = vr[c];
            vs_s[t][0] = f16_bits_to_f32(vss.x & 0xffff);
            vs_s[t][1] = f16_bits_to_f32(vss.x >> 16);
            vs_s[t][2] = f16_bits_to_f32(vss.y & 0xffff);
            vs_s[t][3] = f16_bits_to_f32(vss.y >> 16);
            const float ksc[4] = {f16_bits_to_f32(kss.x & 0xffff), f16_bits_to_f32(kss.x >> 16),
                                  f16_bits_to_f32(kss.y & 0xffff), f16_bits_to_f32(kss.y >> 16)};
#pragma unroll
            for (int h = 0; h < QPK; h++) sc[h] = k_row_dot(kr, ksc, q_s[h]) * scale;
        } else {
#pragma unroll
            for (int h = 0; h < QPK; h++) sc[h] = kNegBig;
        }
        // ---- online softmax over this sub-chunk: one max and one sum
        // round per sub-chunk for all heads (fixed-order trees)
        float mx[QPK];
#pragma unroll
        for (int h = 0; h < QPK; h++) {
            float v = sc[h];
            for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
            if (lane == 0) red[h][wave] = v;
        }
        __syncthreads();
#pragma unroll
        for (int h = 0; h < QPK; h++) {
            float r = red[h][0];
            for (int w = 1; w < kAWG / kWave; w++) r = fmaxf(r, red[h][w]);
            mx[h] = r;
        }
        float p[QPK], corr[QPK];
#pragma unroll
        for (int h = 0; h < QPK; h++) {
            const float m_new = fmaxf(m_run[h], mx[h]);
            p[h] = t < n_here ? __expf(sc[h] - m_new) : 0.f;
            s_s[h][t] = p[h];
            corr[h] = __expf(m_run[h] - m_new);
            m_run[h] = m_new;
        }
        __syncthreads();  // red (max) consumed; s_s, v_s, vs_s written
#pragma unroll
        for (int h = 0; h < QPK; h++) {
            float v = p[h];
            for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
            if (lane == 0) red[h][wave] = v;
        }
        const float cph = QPK == 1 ? corr[0] : (ph == 0 ? corr[0] : corr[QPK - 1]);
#pragma unroll
        for (int e = 0; e < 4; e++) acc[e] *= cph;
        // ---- PV from LDS: thread (ph, pw, pg) takes slots pg, pg+G, ...
        for (int i = pg; i < n_here; i += G) {
            const int v4 = v_s[i][pw];
            const float pp = s_s[ph][i] * vs_s[i][pw / 8];
            acc[0] = __builtin_fmaf(pp, (float)(int8_t)(v4 & 0xff), acc[0]);
            acc[1] = __builtin_fmaf(pp, (float)(int8_t)((v4 >> 8) & 0xff), acc[1]);
            acc[2] = __builtin_fmaf(pp, (float)(int8_t)((v4 >> 16) & 0xff), acc[2]);
            acc[3] = __builtin_fmaf(pp, (float)(int8_t)((v4 >> 24) & 0xff), acc[3]);
        }
        __syncthreads();  // red (sum) written
#pragma unroll
        for (int h = 0; h < QPK; h++) {
            float r = red[h][0];
            for (int w = 1; w < kAWG / kWave; w++) r += red[h][w];
            l_run[h] = l_run[h] * corr[h] + r;
        }
    }

    // ---- combine the G slot groups (fixed order) and write the partial
#pragma unroll
    for (int e = 0; e < 4; e++) acc_s[pg][ph][4 * pw + e] = acc[e];
    __syncthreads();
    const int stride = kHD + 2;
    for (int i = tid; i < QPK * kHD; i += kAWG) {
        const int h = i / kHD, d = i % kHD;
        float a = 0.f;
        for (int g = 0; g < G; g++) a += acc_s[g][h][d];
        part[((size_t)(kvh * QPK + h) * n_splits + split) * stride + d] = a;
    }
    if (tid < QPK) {
        const size_t rowp = ((size_t)(kvh * QPK + tid) * n_splits + split) * stride;
        float mv = m_run[0], lv = l_run[0];
#pragma unroll
        for (int h = 1; h < QPK; h++)
            if (tid == h) mv = m_run[h], lv = l_run[h];
        part[rowp + kHD] = mv;
        part[rowp + kHD + 1] = lv;
    }

}

// Merge of the split partials (attn_reduce.wgsl:24-57): for query head h,
// out = Σ_s a_s·e^(m_s−M) / Σ_s l_s·e^(m_s−M), M = max_s m_s, both sums in
// split order 0..S-1.  One workgroup per kv head, thread (h, d); the
// kernel boundary after the split kernel makes the partials visible (no
// device-scope fences or atomics).  Optionally writes the x limbs of the
// output rows for the next GEMV (8 lanes per 32-block).
template <int QPK>
__global__ __launch_bounds__(QPK * kHD) void attn_merge_kernel(const float *__restrict__ part,
                                                               int n_splits,
                                                               float *__restrict__ out,
                                                               BlockLimbs *__restrict__ limbs_out) {
    __shared__ __align__(16) float o_s[QPK * kHD];
    const int kvh = blockIdx.x, tid = threadIdx.x;
    const int h = tid / kHD, d = tid % kHD;
    const int stride = kHD + 2;
    const float *ph_part = part + (size_t)(kvh * QPK + h) * n_splits * stride;
    float M = kNegBig;
    int s0 = 0;
    for (; s0 + 8 <= n_splits; s0 += 8) {
        float mv[8];
#pragma unroll
        for (int u = 0; u < 8; u++) mv[u] = ph_part[(size_t)(s0 + u) * stride + kHD];
#pragma unroll
        for (int u = 0; u < 8; u++) M = fmaxf(M, mv[u]);
    }
    for (; s0 < n_splits; s0++) M = fmaxf(M, ph_part[(size_t)s0 * stride + kHD]);
    float a = 0.f, l = 0.f;
    s0 = 0;
    for (; s0 + 8 <= n_splits; s0 += 8) {
        float mv[8], lv[8], av[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const float *r = ph_part + (size_t)(s0 + u) * stride;
            mv[u] = r[kHD];
            lv[u] = r[kHD + 1];
            av[u] = r[d];
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const float w = __expf(mv[u] - M);
            a = __builtin_fmaf(av[u], w, a);
            l = __builtin_fmaf(lv[u], w, l);
        }
    }
    for (; s0 < n_splits; s0++) {
        const float *r = ph_part + (size_t)s0 * stride;
        const float w = __expf(r[kHD] - M);
        a = __builtin_fmaf(r[d], w, a);
        l = __builtin_fmaf(r[kHD + 1], w, l);
    }
    const float res = a / l;
    out[(size_t)(kvh * QPK + h) * kHD + d] = res;
    if (limbs_out == nullptr) return;
    o_s[tid] = res;
    __syncthreads();
    if (tid < QPK * kHD / 4) {
        const float4 v = *reinterpret_cast<const float4 *>(&o_s[4 * tid]);
        limbs_block8(v, tid & 7, &limbs_out[(kvh * QPK * kHD) / 32 + (tid >> 3)]);
    }
}

}  // namespace

int launch_attn_decode_q8(hipStream_t st, const float *q, const int8_t *kq, const uint16_t *ks,
                          const int8_t *vq, const uint16_t *vs, const uint32_t *step,
                          int step_word, uint32_t kv_len, int n_q, int n_kv, int head_dim,
                          int n_splits, float scale, float *out, void *workspace,
                          size_t workspace_bytes, void *limbs_out) {
    SGQ_CHECK(head_dim == kHD, "attn_decode_q8: head_dim %d unsupported (128)", head_dim);
    SGQ_CHECK(n_kv > 0 && n_q % n_kv == 0, "attn_decode_q8: n_q %% n_kv != 0");
    SGQ_CHECK(n_splits >= 1 && n_splits <= 1024, "attn_decode_q8: n_splits %d out of range", n_splits);
    SGQ_CHECK(step != nullptr || kv_len > 0, "attn_decode_q8: kv_len must be > 0");
    SGQ_CHECK(((uintptr_t)kq & 15) == 0 && ((uintptr_t)vq & 3) == 0 && ((uintptr_t)ks & 7) == 0 &&
                  ((uintptr_t)vs & 7) == 0,
              "attn_decode_q8: misaligned cache");
    SGQ_CHECK(n_kv <= kAttnMaxKv, "attn_decode_q8: n_kv %d > %d", n_kv, kAttnMaxKv);
    const size_t part_bytes = (size_t)n_q * n_splits * (kHD + 2) * 4;
    SGQ_CHECK(kAttnPartOff + part_bytes <= workspace_bytes,
              "attn_decode_q8: workspace too small (%zu < %zu)", workspace_bytes,
              kAttnPartOff + part_bytes);
    float *part = reinterpret_cast<float *>(static_cast<uint8_t *>(workspace) + kAttnPartOff);
    const int qpk = n_q / n_kv;
    dim3 grid(n_kv, n_splits);
#define SGQ_ATTN(Q)                                                                               \
    case Q:                                                                                       \
        hipLaunchKernelGGL(attn_decode_q8_kernel<Q>, grid, dim3(kAWG), 0, st, q, kq, ks, vq, vs,  \
                           step, step_word, kv_len, n_kv, n_splits, scale, part);                 \
        SGQ_HIP(hipGetLastError());                                                               \
        hipLaunchKernelGGL(attn_merge_kernel<Q>, dim3(n_kv), dim3(Q * kHD), 0, st, part,          \
                           n_splits, out, static_cast<BlockLimbs *>(limbs_out));                  \
        break;
    switch (qpk) {
        SGQ_ATTN(1)
        SGQ_ATTN(2)
        default:
            return fail(SGQ_ERR_VALIDATION, "attn_decode_q8: %d q heads per kv head unsupported",
                        qpk);
    }
#undef SGQ_ATTN
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}

}  // namespace sgq
