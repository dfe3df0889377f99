// Shared pieces of the Q8_0-KV split-K decode attention (the MFMA split
// kernel is attn_mfma.h; the launches are in attn.hip).
//
// Semantics: attn_decode_global_q8k / attn_decode_sliding + attn_reduce
// (crates/sg-gpu/shaders/attn_decode_global_q8k.wgsl:41-112,
// attn_reduce.wgsl:24-57): for each query head h (GQA: kv head h/QPK),
// s_t = scale · q_h·k_t over the valid cache slots t < kv_len, softmax,
// out_h = Σ p_t v_t.  Each (kv head, split) work item leaves a partial
// (acc[hd], m, l) per query head (row stride hd + 2; an empty split is
// m = -3e38, l = 0, acc = 0), and the merges here combine a head's splits
// in split order 0..S-1, the fixed order of attn_reduce.wgsl:40-52:
//  * attn_merge: one kv head's QPK query heads by the first QPK·128
//    threads of a workgroup, 16 splits per load batch with a running max;
//  * attn_merge_head: one query head by a workgroup of 4 or 16 waves, the
//    loads spread over the splits (lanes over splits for (m, l), waves over
//    shares of the splits for acc).
// Both can also write the O projection's x limbs (limbs.h) instead of, or
// besides, the fp32 rows.  Also here: the inputs of the fused q/k/v
// post-projection (AttnPost) and agent-scope load/store helpers for
// partials exchanged between workgroups of one launch.
#pragma once
#include "limbs.h"

namespace sgq {
namespace {

constexpr int kHD = 128;
constexpr float kNegBig = -3.0e38f;

// Native 4 × i32 vector: HIP's int4 is a struct, and copying one into LDS
// becomes a memcpy out of a stack array (scratch) instead of registers.
typedef int i32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void st_agent(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}


// Inputs of the fused post-projection (attn_decode_q8_kernel<*, true>).
struct AttnPost {
    const float *q_raw, *k_raw, *v_src;  // projections of this token
    const float *wq, *wk;                // q_norm / k_norm weights [head_dim]
    const float *rope_cs;                // (cos, sin) × head_dim/2 for this position
    float eps;
    int ring;                            // slots of a ring cache, 0 = linear
    int8_t *kq_w, *vq_w;                 // the cache pages, written by split 0
    uint16_t *ks_w, *vs_w;
};

// Merge of kv head `kvh`'s partials by the workgroup's first QPK·kHD
// threads (thread (h, d)); all threads must call (one barrier when limbs
// are written).  `out` and `limbs_out` may each be null; AGENT selects
// agent-scope loads of the partials (written by other workgroups of the
// same launch) and agent-scope stores for the limbs (read by other
// workgroups of the same launch).
template <int QPK, bool AGENT>
__device__ __forceinline__ void attn_merge(const float *__restrict__ part, int n_splits, int kvh,
                                           float *__restrict__ out,
                                           BlockLimbs *__restrict__ limbs_out, float *o_s) {
    const int tid = threadIdx.x;
    const bool active = tid < QPK * kHD;
    const int h = active ? tid / kHD : 0, d = tid % kHD;
    const int stride = kHD + 2;
    const float *ph_part = part + (size_t)(kvh * QPK + h) * n_splits * stride;
    // one pass: (m, l, a) of up to 16 splits loaded together, then combined
    // in split order; more splits go through the same loop in batches with
    // a running max (rescaling the partial sums when it grows)
    float M = kNegBig, a = 0.f, l = 0.f;
    if (active) {
        for (int s0 = 0; s0 < n_splits; s0 += 16) {
            float mv[16], lv[16], av[16];
            const int nb = min(16, n_splits - s0);
#pragma unroll
            for (int u = 0; u < 16; u++) {
                const float *r = ph_part + (size_t)(s0 + min(u, nb - 1)) * stride;
                const float m_ = AGENT ? ld_agent(r + kHD) : r[kHD];
                const float l_ = AGENT ? ld_agent(r + kHD + 1) : r[kHD + 1];
                const float a_ = AGENT ? ld_agent(r + d) : r[d];
                mv[u] = u < nb ? m_ : kNegBig;
                lv[u] = u < nb ? l_ : 0.f;
                av[u] = u < nb ? a_ : 0.f;
            }
            float Mn = M;
#pragma unroll
            for (int u = 0; u < 16; u++) Mn = fmaxf(Mn, mv[u]);
            const float corr = __expf(M - Mn);
            a *= corr;
            l *= corr;
#pragma unroll
            for (int u = 0; u < 16; u++) {
                const float w = __expf(mv[u] - Mn);
                a = __builtin_fmaf(av[u], w, a);
                l = __builtin_fmaf(lv[u], w, l);
            }
            M = Mn;
        }
    }
    const float res = l > 0.f ? a / l : 0.f;  // all splits empty: 0
    if (active && out) out[(size_t)(kvh * QPK + h) * kHD + d] = res;
    if (limbs_out == nullptr) return;
    if (active) o_s[tid] = res;
    __syncthreads();
    if (tid < QPK * kHD / 4) {
        const float4 v = *reinterpret_cast<const float4 *>(&o_s[4 * tid]);
        limbs_block8<AGENT>(v, tid & 7, &limbs_out[(kvh * QPK * kHD) / 32 + (tid >> 3)]);
    }
}

// Merge of query head hq's n_splits partials (row stride kHD + 2: acc, m, l)
// by a workgroup of NW waves, spreading the loads over the splits instead of
// folding them one after another:
//   1. lanes over splits load (m_s, l_s) into LDS; M = max_s m_s;
//   2. w_s = e^(m_s − M) in LDS, L = Σ_s w_s·l_s;
//   3. wave w sums w_s·acc_s over the w-th NW-th of the splits, lane
//      (dims 2·lane, 2·lane + 1) by 16-split batches of row loads (the
//      first batch is loaded together with (m, l): up to 16·NW splits take
//      one round trip);
//   4. the NW wave sums are added in wave order; out = sum / L.
// Every reduction has a fixed order, so results are bit-reproducible for a
// given NW.  `sm` holds merge_smem(NW) floats.  `out` and `limbs_out` may
// each be null.  All NW·64 threads call.
constexpr int kMergeMaxSplits = 1024;
constexpr int merge_smem(int nw) { return 2 * kMergeMaxSplits + nw * kHD + 2 * nw; }
template <int NW>
__device__ __forceinline__ void attn_merge_head(const float *__restrict__ part, int n_splits,
                                                int hq, float *__restrict__ out,
                                                BlockLimbs *__restrict__ limbs_out, float *sm) {
    constexpr int stride = kHD + 2, NT = NW * 64;
    float *w_s = sm, *l_s = sm + kMergeMaxSplits, *acc_s = sm + 2 * kMergeMaxSplits;
    float *red = acc_s + NW * kHD;  // [0, NW): wave maxima, [NW, 2NW): wave sums of w·l
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float *ph = part + (size_t)hq * n_splits * stride;
    const int per = (n_splits + NW - 1) / NW;
    const int s_lo = min(wave * per, n_splits), s_hi = min(s_lo + per, n_splits);
    float2 av[16];
    auto load_rows = [&](int s0, int nb) {
#pragma unroll
        for (int u = 0; u < 16; u++) {
            const float *r = ph + (size_t)(s0 + min(u, max(nb - 1, 0))) * stride + 2 * lane;
            av[u] = *reinterpret_cast<const float2 *>(r);
        }
    };
    load_rows(min(s_lo, n_splits - 1), min(16, s_hi - s_lo));
    float mx = kNegBig;
    for (int s = tid; s < n_splits; s += NT) {
        const float m_ = ph[(size_t)s * stride + kHD];
        const float l_ = ph[(size_t)s * stride + kHD + 1];
        w_s[s] = m_;
        l_s[s] = l_;
        mx = fmaxf(mx, m_);
    }
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    float M = red[0];
#pragma unroll
    for (int w = 1; w < NW; w++) M = fmaxf(M, red[w]);
    float lsum = 0.f;
    for (int s = tid; s < n_splits; s += NT) {
        const float w = __expf(w_s[s] - M);
        w_s[s] = w;
        lsum = __builtin_fmaf(w, l_s[s], lsum);
    }
    for (int o = 32; o > 0; o >>= 1) lsum += __shfl_xor(lsum, o, kWave);
    __syncthreads();  // w_s complete; red[0, NW) read
    if (lane == 0) red[NW + wave] = lsum;
    // 3. this wave's share of the splits
    float2 acc = make_float2(0.f, 0.f);
    for (int s0 = s_lo; s0 < s_hi; s0 += 16) {
        const int nb = min(16, s_hi - s0);
        if (s0 != s_lo) load_rows(s0, nb);
#pragma unroll
        for (int u = 0; u < 16; u++) {
            const float w = u < nb ? w_s[s0 + u] : 0.f;
            acc.x = __builtin_fmaf(w, av[u].x, acc.x);
            acc.y = __builtin_fmaf(w, av[u].y, acc.y);
        }
    }
    *reinterpret_cast<float2 *>(&acc_s[wave * kHD + 2 * lane]) = acc;
    __syncthreads();
    float res = 0.f;
    if (tid < kHD) {
        float L = red[NW], a = acc_s[tid];
#pragma unroll
        for (int w = 1; w < NW; w++) {
            L += red[NW + w];
            a += acc_s[w * kHD + tid];
        }
        res = L > 0.f ? a / L : 0.f;  // all splits empty: 0
        if (out) out[(size_t)hq * kHD + tid] = res;
    }
    if (limbs_out == nullptr) return;
    __syncthreads();  // acc_s reads done
    if (tid < kHD) acc_s[tid] = res;
    __syncthreads();
    if (tid < kHD / 4) {
        const float4 v = *reinterpret_cast<const float4 *>(&acc_s[4 * tid]);
        limbs_block8<false>(v, tid & 7, &limbs_out[(hq * kHD) / 32 + (tid >> 3)]);
    }
}

}  // namespace
}  // namespace sgq
