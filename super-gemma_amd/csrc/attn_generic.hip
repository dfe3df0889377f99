// Decode attention over a Q8_0 KV cache at any head_dim in {128, 256, 512}
// and 1..8 query heads per kv head: the released checkpoint's geometry
// (sliding layers 16 kv heads of 256, global layers 4 kv heads of 512 under
// 32 query heads; crates/sg-gguf/src/desc.rs:66-93), which the int8-MFMA
// kernel (attn_mfma.h: head_dim 128, <= 2 heads per kv head) does not cover.
//
// Semantics as attn_decode_global_q8k.wgsl:41-112 / attn_reduce.wgsl:24-57:
// s_t = scale·q_h·k_t over a split's slots, softmax per split, partials
// (acc, m, l) per (query head, split), merged over the splits in split order.
// The post-projection before it (q/k norms with weights, the weightless v
// norm, NEOX RoPE, the Q8_0 append; rmsnorm.wgsl:24-61, rope.wgsl:35-52,
// kv_append_global_q8.wgsl:29-60) is one launch of its own.
//
// Three launches per layer:
//  * post-projection: one wave per head row (q heads, then k, then v);
//    lane j holds float4 j (and j + 64 at head_dim 512); the NEOX partner
//    of float4 j is j ± head_dim/8, a lane shuffle or the lane's other
//    float4; q goes out in fp32, k and v as Q8_0 into the cache slot;
//  * attention: workgroup = (kv head, split of 64 slots), 4 waves.  Scores:
//    lane = slot, wave = a quarter of the head's dims (the quarter's K bytes
//    in 16-byte loads, q from LDS as wave-uniform broadcasts), quarters
//    summed in order.  Softmax over the 64 slots per head (one wave per
//    head).  PV: wave = 16 of the split's slots, lane = head_dim/64
//    consecutive dims (a wave reads whole V rows), all 16 V words of a lane
//    issued at once; the waves' sums are added in LDS in wave order;
//    splits past the current kv length exit at once;
//  * merge: workgroup = (query head, 64 dims), splits folded in order up to
//    the current kv length; writes fp32 rows and/or the O projection's x
//    limbs (32-blocks, limbs.h).
#include <algorithm>

#include "limbs.h"
#include "q8.h"

namespace sgq {
namespace {

constexpr int kGSlots = 64;  // slots per split
constexpr float kGNegBig = -3.0e38f;

// (GenericPost is declared in sgq_internal.h)

// One head row in one wave: RMSNorm (weight w, or none), then NEOX RoPE
// with cs when w_rope; lane j holds float4 j (and j + 64 at head_dim 512),
// the partner float4 j ± head_dim/8 a lane shuffle or the lane's other
// float4.  Lanes past the row (head_dim 128: lanes 32..63) hold zeros.
template <int HD>
__device__ __forceinline__ void norm_rope_row(const float *__restrict__ src,
                                              const float *__restrict__ w,
                                              const float2 *__restrict__ cs, float eps,
                                              bool w_rope, int lane,
                                              float4 (&x)[(HD / 4 + 63) / 64]) {
    constexpr int NF = HD / 4;
    constexpr int NV = (NF + 63) / 64;
    float ss = 0.f;
#pragma unroll
    for (int v = 0; v < NV; v++) {
        const int j = lane + 64 * v;
        x[v] = j < NF ? reinterpret_cast<const float4 *>(src)[j] : make_float4(0.f, 0.f, 0.f, 0.f);
        ss += x[v].x * x[v].x + x[v].y * x[v].y + x[v].z * x[v].z + x[v].w * x[v].w;
    }
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, kWave);
    const float inv = 1.0f / sqrtf(ss / (float)HD + eps);
#pragma unroll
    for (int v = 0; v < NV; v++) {
        const int j = lane + 64 * v;
        float4 wt = make_float4(1.f, 1.f, 1.f, 1.f);
        if (w && j < NF) wt = reinterpret_cast<const float4 *>(w)[j];
        x[v] = make_float4(x[v].x * inv * wt.x, x[v].y * inv * wt.y, x[v].z * inv * wt.z,
                           x[v].w * inv * wt.w);
    }
    if (!w_rope) return;
    float4 pr[NV];
    if (NV == 1) {
        const int pj = lane < NF / 2 ? lane + NF / 2 : lane - NF / 2;
        const int src_lane = pj < 64 ? pj : 0;
        pr[0] = make_float4(__shfl(x[0].x, src_lane, kWave), __shfl(x[0].y, src_lane, kWave),
                            __shfl(x[0].z, src_lane, kWave), __shfl(x[0].w, src_lane, kWave));
    } else {
#pragma unroll
        for (int v = 0; v < NV; v++) pr[v] = x[NV - 1 - v];  // NF = 128: j ± 64
    }
#pragma unroll
    for (int v = 0; v < NV; v++) {
        const int j = lane + 64 * v;
        if (j >= NF) continue;
        const bool lo = j < NF / 2;
        const int i0 = (lo ? j : j - NF / 2) * 4;  // pair index of the float4's first dim
        const float sg = lo ? -1.f : 1.f;
        const float2 c0 = cs[i0], c1 = cs[i0 + 1], c2 = cs[i0 + 2], c3 = cs[i0 + 3];
        x[v] = make_float4(x[v].x * c0.x + sg * pr[v].x * c0.y, x[v].y * c1.x + sg * pr[v].y * c1.y,
                           x[v].z * c2.x + sg * pr[v].z * c2.y, x[v].w * c3.x + sg * pr[v].w * c3.y);
    }
}

template <int HD, int QPK>
__global__ __launch_bounds__(256) void attn_generic_kernel(
    // the cache pages are not __restrict__: with post set this kernel writes
    // the new slot's rows and reads them back after a barrier
    const float *__restrict__ q, const int8_t *kq, const uint16_t *ks, const int8_t *vq,
    const uint16_t *vs, const uint32_t *__restrict__ step, int step_word, int n_kv, int n_splits,
    float scale, float *__restrict__ part, GenericPost post) {
    constexpr int NB = HD / 32;   // Q8 blocks per row
    constexpr int DW = HD / 4;    // dims per wave (a quarter of the head)
    constexpr int PB = DW / 32;   // Q8 blocks per quarter
    __shared__ float q_s[QPK][HD];
    __shared__ float sp_s[4][QPK][kGSlots];
    __shared__ float p_s[QPK][kGSlots];
    __shared__ float ml_s[QPK][2];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kvh = blockIdx.x, split = blockIdx.y;
    const uint32_t kv_len = step[step_word];
    const uint32_t t0 = (uint32_t)split * kGSlots;
    if (t0 >= kv_len) return;  // the merge folds only the live splits
    const int n = (int)min((uint32_t)kGSlots, kv_len - t0);

    if (post.q_raw == nullptr) {
        for (int i = tid; i < QPK * HD; i += 256)
            q_s[i / HD][i % HD] = q[((size_t)kvh * QPK + i / HD) * HD + i % HD] * scale;
    } else {
        // the post-projection in every split: this kv head's query heads
        // (norm, RoPE, pre-scaled) into LDS; the split holding the new slot
        // also writes the new K/V rows to the cache (norms, RoPE of k, Q8_0),
        // which its own score and PV loops then read after the barrier
        constexpr int NF = HD / 4, NV = (NF + 63) / 64;
        for (int h = wave; h < QPK; h += 4) {
            float4 x[NV];
            norm_rope_row<HD>(post.q_raw + ((size_t)kvh * QPK + h) * HD, post.q_norm, post.cs,
                              post.eps, true, lane, x);
#pragma unroll
            for (int v = 0; v < NV; v++) {
                const int j = lane + 64 * v;
                if (j < NF)
                    *reinterpret_cast<float4 *>(&q_s[h][4 * j]) =
                        make_float4(x[v].x * scale, x[v].y * scale, x[v].z * scale, x[v].w * scale);
            }
        }
        const uint32_t pos = step[0];
        const uint32_t slot = post.ring ? pos % post.ring : pos;
        if (slot - t0 < (uint32_t)n && wave < 2) {
            float4 x[NV];
            norm_rope_row<HD>((wave == 0 ? post.k_raw : post.v_src) + (size_t)kvh * HD,
                              wave == 0 ? post.k_norm : nullptr, post.cs, post.eps, wave == 0,
                              lane, x);
            const size_t e0 = ((size_t)slot * n_kv + kvh) * HD;  // row start, elements
            uint16_t *sc = wave == 0 ? post.ks_w : post.vs_w;
            int *qt = reinterpret_cast<int *>(wave == 0 ? post.kq_w : post.vq_w);
#pragma unroll
            for (int v = 0; v < NV; v++) {
                const int j = lane + 64 * v;
                if (j < NF) {  // whole 8-lane groups (NF is a multiple of 8)
                    int qv;
                    quant_lane(x[v], j & 7, &sc[(e0 + 4 * j) / 32], &qv);
                    qt[(e0 + 4 * j) / 4] = qv;
                }
            }
        }
    }
    __syncthreads();

    // ---- scores: lane = slot, wave = dims [wave·DW, wave·DW + DW)
    {
        float acc[QPK];
#pragma unroll
        for (int h = 0; h < QPK; h++) acc[h] = 0.f;
        if (lane < n) {
            const size_t row = (size_t)(t0 + lane) * n_kv + kvh;
            const int8_t *kr = kq + row * HD + wave * DW;
            const uint16_t *sr = ks + row * NB + wave * PB;
#pragma unroll
            for (int b = 0; b < PB; b++) {
                const float d = f16_bits_to_f32(sr[b]);
                const int4 w0 = reinterpret_cast<const int4 *>(kr + 32 * b)[0];
                const int4 w1 = reinterpret_cast<const int4 *>(kr + 32 * b)[1];
                const int ww[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
                float kf[32];
#pragma unroll
                for (int j = 0; j < 8; j++)
#pragma unroll
                    for (int e = 0; e < 4; e++) kf[4 * j + e] = (float)(int8_t)(ww[j] >> (8 * e));
#pragma unroll
                for (int h = 0; h < QPK; h++) {
                    const float *qh = &q_s[h][wave * DW + 32 * b];
                    float dot = 0.f;
#pragma unroll
                    for (int j = 0; j < 32; j++) dot = __builtin_fmaf(qh[j], kf[j], dot);
                    acc[h] = __builtin_fmaf(d, dot, acc[h]);
                }
            }
        }
#pragma unroll
        for (int h = 0; h < QPK; h++) sp_s[wave][h][lane] = acc[h];
    }
    __syncthreads();

    // ---- softmax per head over the split: wave w takes heads w, w + 4
    for (int h = wave; h < QPK; h += 4) {
        const float s = lane < n ? ((sp_s[0][h][lane] + sp_s[1][h][lane]) + sp_s[2][h][lane]) +
                                       sp_s[3][h][lane]
                                 : kGNegBig;
        float m = s;
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, kWave));
        const float p = lane < n ? __expf(s - m) : 0.f;
        float l = p;
        for (int o = 32; o > 0; o >>= 1) l += __shfl_xor(l, o, kWave);
        p_s[h][lane] = p;
        if (lane == 0) ml_s[h][0] = m, ml_s[h][1] = l;
    }
    __syncthreads();

    if constexpr (QPK * HD <= 1024) {
        // ---- PV: wave w = slots 16w .. 16w+15, lane = DPL consecutive dims (the
        // whole head across the wave), all 16 V words issued before the FMAs;
        // the four waves' sums then meet in LDS, added in wave order
        constexpr int DPL = HD / 64;  // dims per lane: 2, 4, 8
        float acc[QPK][DPL];
    #pragma unroll
        for (int h = 0; h < QPK; h++)
    #pragma unroll
            for (int e = 0; e < DPL; e++) acc[h][e] = 0.f;
        {
            const int d0 = lane * DPL;
            uint32_t vw[16][(DPL + 3) / 4];
            float vsc[16];
    #pragma unroll
            for (int i = 0; i < 16; i++) {
                const int slot = 16 * wave + i;
                const size_t row = (size_t)(t0 + min(slot, n - 1)) * n_kv + kvh;
                const int8_t *vr = vq + row * HD + d0;
                if (DPL == 2) {
                    vw[i][0] = *reinterpret_cast<const uint16_t *>(vr);
                } else if (DPL == 4) {
                    vw[i][0] = *reinterpret_cast<const uint32_t *>(vr);
                } else {
                    const uint2 t2 = *reinterpret_cast<const uint2 *>(vr);
                    vw[i][0] = t2.x;
                    vw[i][(DPL + 3) / 4 - 1] = t2.y;
                }
                vsc[i] = f16_bits_to_f32(vs[row * NB + d0 / 32]);
            }
    #pragma unroll
            for (int i = 0; i < 16; i++) {
                const int slot = 16 * wave + i;
                if (slot < n) {  // wave-uniform
                    float v[DPL];
    #pragma unroll
                    for (int e = 0; e < DPL; e++)
                        v[e] = vsc[i] * (float)(int8_t)(vw[i][e / 4] >> (8 * (e % 4)));
    #pragma unroll
                    for (int h = 0; h < QPK; h++) {
                        const float p = p_s[h][slot];
    #pragma unroll
                        for (int e = 0; e < DPL; e++) acc[h][e] = __builtin_fmaf(p, v[e], acc[h][e]);
                    }
                }
            }
        }
        __shared__ float red_s[4][QPK][HD];
    #pragma unroll
        for (int h = 0; h < QPK; h++)
    #pragma unroll
            for (int e = 0; e < DPL; e++) red_s[wave][h][lane * DPL + e] = acc[h][e];
        __syncthreads();
        constexpr int stride = HD + 2;
        for (int i = tid; i < QPK * HD; i += 256) {
            const int h = i / HD, d = i % HD;
            const float a = ((red_s[0][h][d] + red_s[1][h][d]) + red_s[2][h][d]) + red_s[3][h][d];
            part[((size_t)(kvh * QPK + h) * n_splits + split) * stride + d] = a;
        }
        if (tid < QPK) {
            float *pr = part + ((size_t)(kvh * QPK + tid) * n_splits + split) * stride;
            pr[HD] = ml_s[tid][0];
            pr[HD + 1] = ml_s[tid][1];
        }
    } else {
        // ---- PV for wide groups (QPK·HD > 1024, where the LDS reduction
        // above costs more than it saves): wave = dims [wave·DW, wave·DW +
        // DW), lane = 2 of them, over all the split's slots
        constexpr int ND = DW / 64;
        const int d0 = wave * DW + lane * ND;
        float acc[QPK][ND];
#pragma unroll
        for (int h = 0; h < QPK; h++)
#pragma unroll
            for (int e = 0; e < ND; e++) acc[h][e] = 0.f;
        // 32 slots' V words and scales are issued before their FMAs (two
        // round trips for a full split instead of one per few slots)
        constexpr int VB = 32;
        for (int i0 = 0; i0 < n; i0 += VB) {
            uint32_t vw[VB];
            float vsc[VB];
#pragma unroll
            for (int u = 0; u < VB; u++) {
                const size_t row = (size_t)(t0 + min(i0 + u, n - 1)) * n_kv + kvh;
                vsc[u] = f16_bits_to_f32(vs[row * NB + d0 / 32]);
                // ND = 2: one 2-byte word; ND = 1 (head_dim 256): one byte
                vw[u] = ND == 2 ? *reinterpret_cast<const uint16_t *>(vq + row * HD + d0)
                                : (uint32_t)(uint8_t)vq[row * HD + d0];
            }
#pragma unroll
            for (int u = 0; u < VB; u++) {
                if (i0 + u < n) {  // wave-uniform
                    const float v[2] = {vsc[u] * (float)(int8_t)(vw[u] & 0xff),
                                        vsc[u] * (float)(int8_t)(vw[u] >> 8)};
#pragma unroll
                    for (int h = 0; h < QPK; h++) {
                        const float p = p_s[h][i0 + u];
#pragma unroll
                        for (int e = 0; e < ND; e++) acc[h][e] = __builtin_fmaf(p, v[e], acc[h][e]);
                    }
                }
            }
        }
        constexpr int stride = HD + 2;
#pragma unroll
        for (int h = 0; h < QPK; h++) {
            float *pr = part + ((size_t)(kvh * QPK + h) * n_splits + split) * stride;
#pragma unroll
            for (int e = 0; e < ND; e++) pr[d0 + e] = acc[h][e];
            if (tid == 0) {
                pr[HD] = ml_s[h][0];
                pr[HD + 1] = ml_s[h][1];
            }
        }
    }
}

// out[h][d] = Σ_s a_s e^(m_s − M) / Σ_s l_s e^(m_s − M) over the live splits;
// fp32 rows to out and/or the x limbs of the row to xl.  Workgroup (h, 64
// dims), wave w folds the w-th quarter of the splits in 16-split batches
// (all loads of a batch issued together, running max rescaled per batch),
// and wave 0 adds the four (M, a, l) in wave order: a fixed order, so the
// result is bit-reproducible.
template <int HD>
__global__ __launch_bounds__(256) void attn_generic_merge_kernel(
    const float *__restrict__ part, const uint32_t *__restrict__ step, int step_word,
    int n_splits, float *__restrict__ out, BlockLimbs *__restrict__ xl) {
    constexpr int stride = HD + 2, B = 16;
    __shared__ float red_s[3][4][64];
    __shared__ __align__(16) float o_s[64];
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int d = blockIdx.y * 64 + lane;
    const uint32_t kv_len = step[step_word];
    const int n_act = min(n_splits, (int)((kv_len + kGSlots - 1) / kGSlots));
    const int per = (n_act + 3) / 4, s0 = wave * per, s1 = min(n_act, s0 + per);
    const float *ph = part + (size_t)h * n_splits * stride;
    float M = kGNegBig, a = 0.f, l = 0.f;
    for (int sb = s0; sb < s1; sb += B) {
        float mv[B], lv[B], av[B];
#pragma unroll
        for (int u = 0; u < B; u++) {
            const bool live = sb + u < s1;
            const float *pr = ph + (size_t)(live ? sb + u : s0) * stride;
            mv[u] = live ? pr[HD] : kGNegBig;
            lv[u] = live ? pr[HD + 1] : 0.f;
            av[u] = live ? pr[d] : 0.f;
        }
        float Mb = M;
#pragma unroll
        for (int u = 0; u < B; u++) Mb = fmaxf(Mb, mv[u]);
        const float r = __expf(M - Mb);
        a *= r;
        l *= r;
#pragma unroll
        for (int u = 0; u < B; u++) {
            const float f = __expf(mv[u] - Mb);
            a = __builtin_fmaf(av[u], f, a);
            l = __builtin_fmaf(lv[u], f, l);
        }
        M = Mb;
    }
    red_s[0][wave][lane] = M;
    red_s[1][wave][lane] = a;
    red_s[2][wave][lane] = l;
    __syncthreads();
    if (wave == 0) {
        float Mt = red_s[0][0][lane];
#pragma unroll
        for (int w = 1; w < 4; w++) Mt = fmaxf(Mt, red_s[0][w][lane]);
        float A = 0.f, Lt = 0.f;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const float f = __expf(red_s[0][w][lane] - Mt);
            A = __builtin_fmaf(red_s[1][w][lane], f, A);
            Lt = __builtin_fmaf(red_s[2][w][lane], f, Lt);
        }
        const float o = Lt > 0.f ? A / Lt : 0.f;
        if (out) out[(size_t)h * HD + d] = o;
        o_s[lane] = o;
    }
    if (!xl) return;
    __syncthreads();
    if (tid < 16) {  // two 32-blocks: 8-lane groups of float4s
        const float4 v = reinterpret_cast<const float4 *>(o_s)[tid];
        limbs_block8(v, tid & 7, xl + ((size_t)h * HD + blockIdx.y * 64) / 32 + (tid >> 3));
    }
}

}  // namespace

int attn_generic_splits(uint32_t slots) {
    return (int)std::max<uint32_t>(1u, (slots + kGSlots - 1) / kGSlots);
}

int launch_attn_decode_generic(hipStream_t st, const float *q, const int8_t *kq,
                               const uint16_t *ks, const int8_t *vq, const uint16_t *vs,
                               const uint32_t *step, int step_word, int n_q, int n_kv,
                               int head_dim, int n_splits, float scale, float *part, float *out,
                               void *xl, const GenericPost *post) {
    SGQ_CHECK((q || post) && kq && ks && vq && vs && step && part && (out || xl),
              "attn_generic: NULL operand");
    GenericPost gp{};
    if (post) {
        gp = *post;
        SGQ_CHECK(gp.q_raw && gp.k_raw && gp.v_src && gp.q_norm && gp.k_norm && gp.cs && gp.kq_w &&
                      gp.ks_w && gp.vq_w && gp.vs_w,
                  "attn_generic: incomplete post-projection operands");
        SGQ_CHECK(((uintptr_t)gp.q_raw & 15) == 0 && ((uintptr_t)gp.k_raw & 15) == 0 &&
                      ((uintptr_t)gp.v_src & 15) == 0 && ((uintptr_t)gp.kq_w & 3) == 0 &&
                      ((uintptr_t)gp.vq_w & 3) == 0,
                  "attn_generic: misaligned post-projection operands");
    }
    SGQ_CHECK(n_kv > 0 && n_q % n_kv == 0, "attn_generic: n_q %% n_kv != 0");
    const int qpk = n_q / n_kv;
    SGQ_CHECK(n_splits >= 1 && n_splits <= 65535, "attn_generic: n_splits %d", n_splits);
    SGQ_CHECK(((uintptr_t)kq & 15) == 0 && ((uintptr_t)vq & 7) == 0,
              "attn_generic: misaligned cache");
    dim3 grid(n_kv, n_splits);
#define SGQ_G(HD, Q)                                                                             \
    hipLaunchKernelGGL((attn_generic_kernel<HD, Q>), grid, dim3(256), 0, st, q, kq, ks, vq, vs,  \
                       step, step_word, n_kv, n_splits, scale, part, gp)
#define SGQ_GQ(HD)                                                      \
    switch (qpk) {                                                      \
        case 1: SGQ_G(HD, 1); break;                                    \
        case 2: SGQ_G(HD, 2); break;                                    \
        case 4: SGQ_G(HD, 4); break;                                    \
        case 8: SGQ_G(HD, 8); break;                                    \
        default: return fail(SGQ_ERR_VALIDATION, "attn_generic: %d q heads per kv head", qpk); \
    }
    switch (head_dim) {
        case 128: SGQ_GQ(128); break;
        case 256: SGQ_GQ(256); break;
        case 512: SGQ_GQ(512); break;
        default: return fail(SGQ_ERR_VALIDATION, "attn_generic: head_dim %d (128/256/512)", head_dim);
    }
#undef SGQ_GQ
#undef SGQ_G
    SGQ_HIP(hipGetLastError());
    BlockLimbs *xt = static_cast<BlockLimbs *>(xl);
    const dim3 mg(n_q, head_dim / 64);
    switch (head_dim) {
        case 128:
            hipLaunchKernelGGL(attn_generic_merge_kernel<128>, mg, dim3(256), 0, st, part, step,
                               step_word, n_splits, out, xt);
            break;
        case 256:
            hipLaunchKernelGGL(attn_generic_merge_kernel<256>, mg, dim3(256), 0, st, part, step,
                               step_word, n_splits, out, xt);
            break;
        default:
            hipLaunchKernelGGL(attn_generic_merge_kernel<512>, mg, dim3(256), 0, st, part, step,
                               step_word, n_splits, out, xt);
    }
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}

}  // namespace sgq
