// Decode attention over the reference's own page formats for the released
// checkpoint's names (crates/sg-gpu/build.rs:255-394), so that its
// record_layer (crates/sg-model/src/graph.rs:572-650) dispatches unchanged:
//   attn_decode_sliding     f16 q, f16 K and V ring pages, head_dim 256,
//                           16 kv heads, 2 query heads per kv head, kv_len
//                           = step[1]   (attn_decode_sliding.wgsl:51-121)
//   attn_decode_global      the same at head_dim 512, 4 kv heads, 8 query
//                           heads per kv head, kv_len = step[2]
//   attn_decode_global_q8k  K from Q8_0 pages (i8 quants, f16 scale per
//                           32 dims), V f16  (attn_decode_global_q8k.wgsl)
//   attn_reduce_d256 / _d512   the split merge, f16 rows out (attn_reduce.wgsl)
//   kv_append_sliding / _global   f16 rows into the ring (slot = (pos + t)
//                           mod 1024) or the linear cache (kv_append.wgsl)
// Semantics: split s of kv head g covers slots [s·c, min(s·c + c, kv_len)),
// c = ceil(kv_len / n_splits), in physical slot order; score = (q·k)·scale;
// the partial (acc, m, l) of query head h at [(h·n_splits + s)·(head_dim +
// 2)] is the unnormalised softmax-weighted V sum, its max and its sum (an
// empty split: acc 0, m -3e38, l 0).  The model driver keeps Q8_0 K and V
// (csrc/attn_generic.hip); these serve callers that hold f16 pages.
//
// Design: one 256-thread workgroup per (kv head, split) walks its chunk in
// tiles of 64 slots: scores with lane = slot and wave = a quarter of the
// dims (q in LDS), the tile's max and exponentials per head (one wave per
// head), then PV with each thread owning head_dim/256 dims of every query
// head, all 64 V values of a tile issued before their FMAs, and the running
// (m, l) rescale applied per tile.
#include "sgq_internal.h"

namespace sgq {
namespace {

constexpr int kPTile = 64;  // slots per tile
constexpr float kPNegBig = -3.0e38f;

__device__ __forceinline__ float h2f(uint16_t b) {
    return (float)__builtin_bit_cast(_Float16, b);
}

template <int HD, int QPK, bool KQ8>
__global__ __launch_bounds__(256) void attn_decode_pages_kernel(
    const uint16_t *__restrict__ q16, const void *__restrict__ kp,
    const uint16_t *__restrict__ k_scales, const uint16_t *__restrict__ v16,
    float *__restrict__ part, const uint32_t *__restrict__ step, int step_word, int n_kv,
    int n_splits, float scale) {
    constexpr int DW = HD / 4;    // score dims per wave
    constexpr int PB = DW / 32;   // 32-dim blocks per wave
    constexpr int ND = HD / 256;  // PV dims per thread
    __shared__ float q_s[QPK][HD];
    __shared__ float sp_s[4][QPK][kPTile];
    __shared__ float p_s[QPK][kPTile];
    __shared__ float m_s[QPK], l_s[QPK], corr_s[QPK];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kvh = blockIdx.x, split = blockIdx.y;
    const uint32_t kv_len = step[step_word];
    const uint32_t chunk = (kv_len + (uint32_t)n_splits - 1) / (uint32_t)n_splits;
    const uint32_t t_begin = min((uint32_t)split * chunk, kv_len);
    const uint32_t t_end = min(t_begin + chunk, kv_len);

    for (int i = tid; i < QPK * HD; i += 256)
        q_s[i / HD][i % HD] = h2f(q16[((size_t)kvh * QPK + i / HD) * HD + i % HD]);
    if (tid < QPK) m_s[tid] = kPNegBig, l_s[tid] = 0.f;
    float acc[QPK][ND];
#pragma unroll
    for (int h = 0; h < QPK; h++)
#pragma unroll
        for (int e = 0; e < ND; e++) acc[h][e] = 0.f;
    __syncthreads();

    for (uint32_t t0 = t_begin; t0 < t_end; t0 += kPTile) {
        const int n = (int)min((uint32_t)kPTile, t_end - t0);
        // ---- scores of the tile's slots (lane = slot), this wave's dims
        float a[QPK];
#pragma unroll
        for (int h = 0; h < QPK; h++) a[h] = 0.f;
        if (lane < n) {
            const size_t row = (size_t)(t0 + lane) * n_kv + kvh;
#pragma unroll
            for (int b = 0; b < PB; b++) {
                const int d0 = wave * DW + 32 * b;
                float kf[32];
                float d = 1.f;
                if (KQ8) {
                    const int8_t *kr = static_cast<const int8_t *>(kp) + row * HD + d0;
                    const int4 w0 = reinterpret_cast<const int4 *>(kr)[0];
                    const int4 w1 = reinterpret_cast<const int4 *>(kr)[1];
                    const int ww[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
                    for (int j = 0; j < 8; j++)
#pragma unroll
                        for (int e = 0; e < 4; e++) kf[4 * j + e] = (float)(int8_t)(ww[j] >> (8 * e));
                    d = h2f(k_scales[row * (HD / 32) + d0 / 32]);
                } else {
                    const uint4 *kr = reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(kp) +
                                                                      row * HD + d0);
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        const uint4 w = kr[c];
                        const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            kf[8 * c + 2 * e] = h2f((uint16_t)(ww[e] & 0xffffu));
                            kf[8 * c + 2 * e + 1] = h2f((uint16_t)(ww[e] >> 16));
                        }
                    }
                }
#pragma unroll
                for (int h = 0; h < QPK; h++) {
                    float dot = 0.f;
#pragma unroll
                    for (int j = 0; j < 32; j++) dot = __builtin_fmaf(q_s[h][d0 + j], kf[j], dot);
                    a[h] = KQ8 ? __builtin_fmaf(d, dot, a[h]) : a[h] + dot;
                }
            }
        }
#pragma unroll
        for (int h = 0; h < QPK; h++) sp_s[wave][h][lane] = a[h];
        __syncthreads();
        // ---- the tile's softmax step per head (wave w: heads w, w + 4)
        for (int h = wave; h < QPK; h += 4) {
            const float s = lane < n ? (((sp_s[0][h][lane] + sp_s[1][h][lane]) + sp_s[2][h][lane]) +
                                        sp_s[3][h][lane]) * scale
                                     : kPNegBig;
            float mt = s;
            for (int o = 32; o > 0; o >>= 1) mt = fmaxf(mt, __shfl_xor(mt, o, kWave));
            const float m_old = m_s[h];
            const float m_new = fmaxf(m_old, mt);
            const float p = lane < n ? expf(s - m_new) : 0.f;
            float ps = p;
            for (int o = 32; o > 0; o >>= 1) ps += __shfl_xor(ps, o, kWave);
            p_s[h][lane] = p;
            if (lane == 0) {
                const float corr = expf(m_old - m_new);  // the first tile: exp(-3e38 - m) = 0
                corr_s[h] = corr;
                l_s[h] = l_s[h] * corr + ps;
                m_s[h] = m_new;
            }
        }
        __syncthreads();
        // ---- PV: this thread's ND dims of every query head
        {
            uint32_t vw[kPTile];
#pragma unroll
            for (int i = 0; i < kPTile; i++) {
                const size_t row = (size_t)(t0 + min(i, n - 1)) * n_kv + kvh;
                const uint16_t *vr = v16 + row * HD + tid * ND;
                vw[i] = ND == 2 ? *reinterpret_cast<const uint32_t *>(vr) : (uint32_t)vr[0];
            }
#pragma unroll
            for (int h = 0; h < QPK; h++) {
                const float c = corr_s[h];
#pragma unroll
                for (int e = 0; e < ND; e++) acc[h][e] *= c;
            }
#pragma unroll
            for (int i = 0; i < kPTile; i++) {
                if (i < n) {  // workgroup-uniform
                    float v[ND];
#pragma unroll
                    for (int e = 0; e < ND; e++) v[e] = h2f((uint16_t)(vw[i] >> (16 * e)));
#pragma unroll
                    for (int h = 0; h < QPK; h++) {
                        const float p = p_s[h][i];
#pragma unroll
                        for (int e = 0; e < ND; e++) acc[h][e] = __builtin_fmaf(p, v[e], acc[h][e]);
                    }
                }
            }
        }
        __syncthreads();  // p_s / sp_s are rewritten by the next tile
    }

    constexpr int stride = HD + 2;
#pragma unroll
    for (int h = 0; h < QPK; h++) {
        float *pr = part + ((size_t)(kvh * QPK + h) * n_splits + split) * stride;
#pragma unroll
        for (int e = 0; e < ND; e++) pr[tid * ND + e] = acc[h][e];
        if (tid == 0) {
            pr[HD] = m_s[h];
            pr[HD + 1] = l_s[h];
        }
    }
}

// The split merge in split order, as attn_reduce.wgsl:33-56 folds it:
// m' = max(m, m_s), acc = acc·e^(m - m') + acc_s·e^(m_s - m'), l likewise;
// out = f16(acc / l).  One 256-thread workgroup per query head.
template <int HD>
__global__ __launch_bounds__(256) void attn_reduce_pages_kernel(const float *__restrict__ part,
                                                                 int n_splits,
                                                                 uint16_t *__restrict__ out) {
    constexpr int ND = HD / 256, stride = HD + 2;
    const int h = blockIdx.x, tid = threadIdx.x;
    float m = kPNegBig, l = 0.f, acc[ND];
#pragma unroll
    for (int e = 0; e < ND; e++) acc[e] = 0.f;
    for (int s = 0; s < n_splits; s++) {
        const float *pr = part + ((size_t)h * n_splits + s) * stride;
        const float ms = pr[HD], ls = pr[HD + 1];
        const float m_new = fmaxf(m, ms);
        const float ca = expf(m - m_new), cb = expf(ms - m_new);
#pragma unroll
        for (int e = 0; e < ND; e++) acc[e] = acc[e] * ca + pr[tid * ND + e] * cb;
        l = l * ca + ls * cb;
        m = m_new;
    }
#pragma unroll
    for (int e = 0; e < ND; e++)
        out[(size_t)h * HD + tid * ND + e] = __builtin_bit_cast(uint16_t, (_Float16)(acc[e] / l));
}

// f16 rows [n_tok × row] to slot step[0] + t (mod ring when ring > 0); eight
// halves per thread.
__global__ __launch_bounds__(256) void kv_append_f16_kernel(const uint4 *__restrict__ src,
                                                            uint4 *__restrict__ dst,
                                                            const uint32_t *__restrict__ step,
                                                            uint64_t n8, uint32_t row8,
                                                            uint32_t ring) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n8) return;
    const uint32_t t = (uint32_t)(i / row8), j = (uint32_t)(i % row8);
    const uint32_t slot = ring ? (step[0] + t) % ring : step[0] + t;
    dst[(size_t)slot * row8 + j] = src[i];
}

}  // namespace

int launch_attn_decode_pages(hipStream_t st, const uint16_t *q, const void *k,
                             const uint16_t *k_scales, const uint16_t *v, float *part,
                             const uint32_t *step, int step_word, int head_dim, int n_q, int n_kv,
                             int n_splits, float scale) {
    SGQ_CHECK(q && k && v && part && step, "attn_decode_pages: NULL operand");
    SGQ_CHECK(n_kv > 0 && n_q % n_kv == 0, "attn_decode_pages: n_q %% n_kv != 0");
    SGQ_CHECK(n_splits >= 1 && n_splits <= 65535, "attn_decode_pages: n_splits %d", n_splits);
    SGQ_CHECK(((uintptr_t)k & 15) == 0 && ((uintptr_t)v & 3) == 0,
              "attn_decode_pages: misaligned pages");
    const int qpk = n_q / n_kv;
    const dim3 grid(n_kv, n_splits);
    if (head_dim == 256 && qpk == 2 && !k_scales)
        hipLaunchKernelGGL((attn_decode_pages_kernel<256, 2, false>), grid, dim3(256), 0, st, q, k,
                           k_scales, v, part, step, step_word, n_kv, n_splits, scale);
    else if (head_dim == 512 && qpk == 8 && !k_scales)
        hipLaunchKernelGGL((attn_decode_pages_kernel<512, 8, false>), grid, dim3(256), 0, st, q, k,
                           k_scales, v, part, step, step_word, n_kv, n_splits, scale);
    else if (head_dim == 512 && qpk == 8 && k_scales)
        hipLaunchKernelGGL((attn_decode_pages_kernel<512, 8, true>), grid, dim3(256), 0, st, q, k,
                           k_scales, v, part, step, step_word, n_kv, n_splits, scale);
    else
        return fail(SGQ_ERR_VALIDATION,
                    "attn_decode_pages: head_dim %d with %d query heads per kv head (%s K) is "
                    "not a built variant", head_dim, qpk, k_scales ? "Q8_0" : "f16");
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}

int launch_attn_reduce_pages(hipStream_t st, const float *part, int n_q, int head_dim,
                             int n_splits, uint16_t *out) {
    SGQ_CHECK(part && out && n_q > 0 && n_splits >= 1, "attn_reduce_pages: bad operands");
    if (head_dim == 256)
        hipLaunchKernelGGL(attn_reduce_pages_kernel<256>, dim3(n_q), dim3(256), 0, st, part,
                           n_splits, out);
    else if (head_dim == 512)
        hipLaunchKernelGGL(attn_reduce_pages_kernel<512>, dim3(n_q), dim3(256), 0, st, part,
                           n_splits, out);
    else
        return fail(SGQ_ERR_VALIDATION, "attn_reduce_pages: head_dim %d (256 / 512)", head_dim);
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}

int launch_kv_append_f16(hipStream_t st, const uint16_t *src, uint16_t *dst,
                         const uint32_t *step, uint32_t n_tok, uint32_t row, uint32_t ring) {
    SGQ_CHECK(src && dst && step, "kv_append_f16: NULL operand");
    SGQ_CHECK(row % 8 == 0 && ((uintptr_t)src & 15) == 0 && ((uintptr_t)dst & 15) == 0,
              "kv_append_f16: rows must be 16-byte aligned multiples of 8 halves");
    const uint64_t n8 = (uint64_t)n_tok * (row / 8);
    if (n8 == 0) return SGQ_OK;
    hipLaunchKernelGGL(kv_append_f16_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, st,
                       reinterpret_cast<const uint4 *>(src), reinterpret_cast<uint4 *>(dst), step,
                       n8, row / 8, ring);
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}

}  // namespace sgq
