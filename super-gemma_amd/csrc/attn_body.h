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
#pragma once
#include "limbs.h"

namespace sgq {
namespace {

constexpr int kHD = 128;
constexpr int kAWG = 256;             // split kernel workgroup (= slots per pass)
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

constexpr size_t attn_lds_bytes(int qpk, int wg) {
    return (size_t)wg * kHD + (size_t)qpk * wg * 4 + (size_t)wg * 8;
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

// Dequantized dots of a 128-wide K row (int8 + 4 f16 scales) with the QPK
// query heads of a kv head (LDS): one pass over the row, every converted
// K word used for all heads at once (the converted floats die at once).
template <int QPK>
__device__ __forceinline__ void k_row_dots(const i32x4 (&kr)[8], uint2 kss, const float *q0,
                                           float scale, float (&sc)[QPK]) {
    const float ksc[4] = {f16_bits_to_f32(kss.x & 0xffff), f16_bits_to_f32(kss.x >> 16),
                          f16_bits_to_f32(kss.y & 0xffff), f16_bits_to_f32(kss.y >> 16)};
    float s[QPK];
#pragma unroll
    for (int h = 0; h < QPK; h++) s[h] = 0.f;
#pragma unroll
    for (int b = 0; b < 4; b++) {
        float part[QPK];
#pragma unroll
        for (int h = 0; h < QPK; h++) part[h] = 0.f;
#pragma unroll
        for (int c = 0; c < 2; c++) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int w = kr[2 * b + c][e];
                const float k0 = (float)(int8_t)(w & 0xff), k1 = (float)(int8_t)((w >> 8) & 0xff);
                const float k2 = (float)(int8_t)((w >> 16) & 0xff), k3 = (float)(int8_t)(w >> 24);
#pragma unroll
                for (int h = 0; h < QPK; h++) {
                    const float4 q4 =
                        *reinterpret_cast<const float4 *>(q0 + h * kHD + 32 * b + 16 * c + 4 * e);
                    part[h] = __builtin_fmaf(q4.x, k0, part[h]);
                    part[h] = __builtin_fmaf(q4.y, k1, part[h]);
                    part[h] = __builtin_fmaf(q4.z, k2, part[h]);
                    part[h] = __builtin_fmaf(q4.w, k3, part[h]);
                }
            }
        }
#pragma unroll
        for (int h = 0; h < QPK; h++) s[h] = __builtin_fmaf(ksc[b], part[h], s[h]);
    }
#pragma unroll
    for (int h = 0; h < QPK; h++) sc[h] = s[h] * scale;
}

// One (kv head, split) work item: the split's partial (acc, m, l) for the
// QPK query heads of kv head `kvh`, written with agent-scope stores so that
// a merge in the same launch can read them after an atomic handoff.
// The dynamic LDS area of attn_lds_bytes(QPK, WG) bytes starts `smem_off`
// bytes into the kernel's dynamic LDS (an offset, not a pointer, so that
// every access stays an LDS access); `pos` is the current position (FUSED
// only).  Called by all WG threads.
template <int QPK, bool FUSED, int WG>
__device__ __forceinline__ void attn_split(
    const float *__restrict__ q, const int8_t *__restrict__ kq, const uint16_t *__restrict__ ks,
    const int8_t *__restrict__ vq, const uint16_t *__restrict__ vs, uint32_t kv_len, int n_kv,
    int n_splits, float scale, float *__restrict__ part, const AttnPost &post, int kvh, int split,
    uint32_t smem_off, uint32_t pos) {
    constexpr int G = WG / (QPK * (kHD / 4));  // slot groups in the PV phase
    static_assert(G >= 1, "QPK too large for one workgroup");
    // Dynamic LDS (attn_lds_bytes): V quants of the sub-chunk, one 128-B row
    // per slot with its eight 16-B chunks XOR-swizzled by slot (conflict-
    // free row writes and PV reads); probabilities; V scales (f16 × 4).
    // After the last PV the V area holds the per-group accumulators.
    extern __shared__ __align__(16) uint8_t attn_dyn_smem[];
    uint8_t *smem = attn_dyn_smem + smem_off;
    int *v_s = reinterpret_cast<int *>(smem);
    float *s_s = reinterpret_cast<float *>(smem + WG * kHD);
    uint2 *vsc_s = reinterpret_cast<uint2 *>(smem + WG * kHD + QPK * WG * 4);
    float *acc_s = reinterpret_cast<float *>(smem);  // [G][QPK][kHD]
    __shared__ __align__(16) float q_s[QPK][kHD];
    __shared__ float red[QPK][WG / kWave];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const uint32_t chunk = (kv_len + n_splits - 1) / n_splits;
    const uint32_t t_begin = min((uint32_t)split * chunk, kv_len);
    const uint32_t t_end = min(t_begin + chunk, kv_len);

    // ---- one slot per thread: K row, V row and both scale words issued
    // together (one memory round trip per sub-chunk); the first sub-chunk is
    // issued before the post-projection, later ones while PV runs.
    i32x4 kr[8], vr[8];
    uint2 kss = {0u, 0u}, vss = {0u, 0u};
#define SGQ_LOAD_SUB(BASE)                                                          \
    if ((uint32_t)tid < min((uint32_t)WG, t_end - (BASE))) {                        \
        const size_t row = (size_t)((BASE) + tid) * n_kv + kvh;                     \
        const i32x4 *kp = reinterpret_cast<const i32x4 *>(kq + row * kHD);          \
        const i32x4 *vp = reinterpret_cast<const i32x4 *>(vq + row * kHD);          \
        _Pragma("unroll") for (int c = 0; c < 8; c++) kr[c] = kp[c];                \
        _Pragma("unroll") for (int c = 0; c < 8; c++) vr[c] = vp[c];                \
        kss = *reinterpret_cast<const uint2 *>(ks + row * (kHD / 32));              \
        vss = *reinterpret_cast<const uint2 *>(vs + row * (kHD / 32));              \
    }
    if (t_begin < t_end) {
        SGQ_LOAD_SUB(t_begin)
    }
    uint32_t fresh_slot = 0xffffffffu;
    __shared__ __align__(16) int fk_s[kHD / 4], fv_s[kHD / 4];  // new K/V row quants
    __shared__ __align__(8) uint16_t fks_s[kHD / 32], fvs_s[kHD / 32];
    if (FUSED) {
        static_assert(2 * kHD <= WG && QPK * kHD <= 2 * kHD, "post layout");
        __shared__ float pq_s[QPK * kHD], pkv_s[2 * kHD], pred[2][2 * kHD / kWave];
        fresh_slot = post.ring ? pos % (uint32_t)post.ring : pos;
        // threads 0..255: q head g / k (g = 0) or v (g = 1) element d
        const bool pt = tid < 2 * kHD;
        const int g = pt ? tid / kHD : 0, d = tid % kHD;
        float qv = tid < QPK * kHD ? post.q_raw[(size_t)kvh * QPK * kHD + tid] : 0.f;
        float kvv = !pt ? 0.f
                  : g == 0 ? post.k_raw[(size_t)kvh * kHD + d] : post.v_src[(size_t)kvh * kHD + d];
        float a = qv * qv, b = kvv * kvv;
        for (int o = 32; o > 0; o >>= 1) {
            a += __shfl_xor(a, o, kWave);
            b += __shfl_xor(b, o, kWave);
        }
        if (lane == 0 && pt) pred[0][wave] = a, pred[1][wave] = b;
        __syncthreads();
        const float sq = pred[0][2 * g] + pred[0][2 * g + 1];
        const float skv = pred[1][2 * g] + pred[1][2 * g + 1];
        qv = qv * (1.0f / sqrtf(sq / (float)kHD + post.eps)) * post.wq[d];
        kvv = kvv * (1.0f / sqrtf(skv / (float)kHD + post.eps)) * (g == 0 ? post.wk[d] : 1.f);
        if (tid < QPK * kHD) pq_s[tid] = qv;
        if (pt) pkv_s[tid] = kvv;
        __syncthreads();
        {  // NEOX RoPE: pair i couples dims (i, i + 64)
            const int i = d % (kHD / 2), hb = tid - d;  // head base
            const float c = post.rope_cs[2 * i], sn = post.rope_cs[2 * i + 1];
            if (tid < QPK * kHD) {
                const float x0 = pq_s[hb + i], x1 = pq_s[hb + i + kHD / 2];
                q_s[g][d] = d < kHD / 2 ? x0 * c - x1 * sn : x1 * c + x0 * sn;
            }
            if (pt && g == 0) {
                const float x0 = pkv_s[i], x1 = pkv_s[i + kHD / 2];
                kvv = d < kHD / 2 ? x0 * c - x1 * sn : x1 * c + x0 * sn;
            }
        }
        // Q8_0 of the new row (kv_quant_q8.wgsl:41-56): 32-lane groups
        float amax = fabsf(kvv);
        for (int o = 16; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, kWave));
        const float dq = amax * (1.0f / 127.0f);
        const float id = dq > 0.f ? 1.0f / dq : 0.f;
        const int8_t qi = (int8_t)(int)__builtin_rintf(kvv * id);
        const uint16_t sc = f32_to_f16_bits(dq);
        if (pt) {
            reinterpret_cast<int8_t *>(g == 0 ? fk_s : fv_s)[d] = qi;
            if ((d & 31) == 0) (g == 0 ? fks_s : fvs_s)[d / 32] = sc;
        }
        if (pt && split == 0) {
            const size_t e = ((size_t)fresh_slot * n_kv + kvh) * kHD + d;
            (g == 0 ? post.kq_w : post.vq_w)[e] = qi;
            if ((d & 31) == 0) (g == 0 ? post.ks_w : post.vs_w)[e / 32] = sc;
        }
    } else {
        for (int i = tid; i < QPK * kHD; i += WG)
            q_s[i / kHD][i % kHD] = q[(size_t)(kvh * QPK) * kHD + i];
    }

    // PV thread role: head ph, 4-dim word pw, slot group pg
    const int ph = tid / (kHD / 4) % QPK, pw = tid % (kHD / 4), pg = tid / (QPK * kHD / 4);
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    float m_run[QPK], l_run[QPK];
#pragma unroll
    for (int h = 0; h < QPK; h++) {
        m_run[h] = kNegBig;
        l_run[h] = 0.f;
    }

    for (uint32_t base = t_begin; base < t_end; base += WG) {
        const int n_here = (int)min((uint32_t)WG, t_end - base);
        const int t = tid;
        __syncthreads();  // q_s (and the new row) ready; previous sub-chunk's LDS reads done
        float sc[QPK];
        // q is re-read from LDS for every pass (an opaque zero offset keeps
        // the compiler from hoisting 32·QPK float4 out of the loop into
        // registers, which a 1024-thread workgroup cannot afford)
        int zoff;
        asm volatile("s_mov_b32 %0, 0" : "=s"(zoff));
        if (FUSED) {  // the new row replaces what the cache load returned for it
            const bool fresh = t < n_here && base + t == fresh_slot;
#pragma unroll
            for (int c = 0; c < 8; c++) {
                const i32x4 fk = reinterpret_cast<const i32x4 *>(fk_s + zoff)[c];
                const i32x4 fv = reinterpret_cast<const i32x4 *>(fv_s + zoff)[c];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    kr[c][e] = fresh ? fk[e] : kr[c][e];
                    vr[c][e] = fresh ? fv[e] : vr[c][e];
                }
            }
            const uint2 fks = *reinterpret_cast<const uint2 *>(fks_s + zoff);
            const uint2 fvs = *reinterpret_cast<const uint2 *>(fvs_s + zoff);
            kss.x = fresh ? fks.x : kss.x;
            kss.y = fresh ? fks.y : kss.y;
            vss.x = fresh ? fvs.x : vss.x;
            vss.y = fresh ? fvs.y : vss.y;
        }
        if (t < n_here) {
#pragma unroll
            for (int c = 0; c < 8; c++)
                *reinterpret_cast<i32x4 *>(&v_s[t * 32 + 4 * (c ^ (t & 7))]) = vr[c];
            vsc_s[t] = vss;
            k_row_dots<QPK>(kr, kss, &q_s[0][0] + zoff, scale, sc);
        } else {
#pragma unroll
            for (int h = 0; h < QPK; h++) sc[h] = kNegBig;
        }
        if (base + WG < t_end) {  // lands while this one finishes
            SGQ_LOAD_SUB(base + WG)
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
            for (int w = 1; w < WG / kWave; w++) r = fmaxf(r, red[h][w]);
            mx[h] = r;
        }
        float p[QPK], corr[QPK];
#pragma unroll
        for (int h = 0; h < QPK; h++) {
            const float m_new = fmaxf(m_run[h], mx[h]);
            p[h] = t < n_here ? __expf(sc[h] - m_new) : 0.f;
            s_s[h * WG + t] = p[h];
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
        const int pb = pw / 8;  // this thread's 32-block of head_dim
        for (int i = pg; i < n_here; i += G) {
            const int v4 = v_s[i * 32 + 4 * ((pw >> 2) ^ (i & 7)) + (pw & 3)];
            const uint2 sv = vsc_s[i];
            const uint32_t sw = pb < 2 ? sv.x : sv.y;
            const float pp = s_s[ph * WG + i] * f16_bits_to_f32((sw >> ((pb & 1) * 16)) & 0xffffu);
            acc[0] = __builtin_fmaf(pp, (float)(int8_t)(v4 & 0xff), acc[0]);
            acc[1] = __builtin_fmaf(pp, (float)(int8_t)((v4 >> 8) & 0xff), acc[1]);
            acc[2] = __builtin_fmaf(pp, (float)(int8_t)((v4 >> 16) & 0xff), acc[2]);
            acc[3] = __builtin_fmaf(pp, (float)(int8_t)((v4 >> 24) & 0xff), acc[3]);
        }
        __syncthreads();  // red (sum) written
#pragma unroll
        for (int h = 0; h < QPK; h++) {
            float r = red[h][0];
            for (int w = 1; w < WG / kWave; w++) r += red[h][w];
            l_run[h] = l_run[h] * corr[h] + r;
        }
    }

    // ---- combine the G slot groups (fixed order) and write the partial
    __syncthreads();  // v_s (now acc_s) free
#pragma unroll
    for (int e = 0; e < 4; e++) acc_s[(pg * QPK + ph) * kHD + 4 * pw + e] = acc[e];
    __syncthreads();
    const int stride = kHD + 2;
    if (tid < QPK * kHD) {
        const int h = tid / kHD, d = tid % kHD;
        float a = 0.f;
        for (int g = 0; g < G; g++) a += acc_s[(g * QPK + h) * kHD + d];
        st_agent(&part[((size_t)(kvh * QPK + h) * n_splits + split) * stride + d], a);
    }
    if (tid < QPK) {
        const size_t rowp = ((size_t)(kvh * QPK + tid) * n_splits + split) * stride;
        float mv = m_run[0], lv = l_run[0];
#pragma unroll
        for (int h = 1; h < QPK; h++)
            if (tid == h) mv = m_run[h], lv = l_run[h];
        st_agent(&part[rowp + kHD], mv);
        st_agent(&part[rowp + kHD + 1], lv);
    }
}

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
    const float res = a / l;
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
// by a 256-thread workgroup, spreading the loads over the splits instead of
// folding them one after another:
//   1. lanes over splits load (m_s, l_s) into LDS; M = max_s m_s;
//   2. w_s = e^(m_s − M) in LDS, L = Σ_s w_s·l_s;
//   3. wave w sums w_s·acc_s over the w-th quarter of the splits, lane
//      (dims 2·lane, 2·lane + 1) by 16-split batches of row loads;
//   4. the four wave sums are added in wave order; out = sum / L.
// Every reduction has a fixed order, so results are bit-reproducible.
// `sm` holds kMergeSmem floats.  `out` and `limbs_out` may each be null;
// AGENT selects agent-scope loads of the partials and stores of the limbs
// (written / read by other workgroups of the same launch).  All 256 threads
// call; the caller separates two calls with a barrier.
constexpr int kMergeMaxSplits = 1024;
constexpr int kMergeSmem = 2 * kMergeMaxSplits + 4 * kHD + 8;
template <bool AGENT>
__device__ __forceinline__ void attn_merge_head(const float *__restrict__ part, int n_splits,
                                                int hq, float *__restrict__ out,
                                                BlockLimbs *__restrict__ limbs_out, float *sm) {
    constexpr int stride = kHD + 2, NT = 256;
    float *w_s = sm, *l_s = sm + kMergeMaxSplits, *acc_s = sm + 2 * kMergeMaxSplits;
    float *red = acc_s + 4 * kHD;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float *ph = part + (size_t)hq * n_splits * stride;
    // this wave's quarter of the splits; its first 16 rows are loaded now,
    // alongside (m, l), so that up to 64 splits take one round trip
    const int per = (n_splits + 3) / 4;
    const int s_lo = min(wave * per, n_splits), s_hi = min(s_lo + per, n_splits);
    float2 av[16];
    auto load_rows = [&](int s0, int nb) {
#pragma unroll
        for (int u = 0; u < 16; u++) {
            const float *r = ph + (size_t)(s0 + min(u, max(nb - 1, 0))) * stride + 2 * lane;
            av[u] = AGENT ? make_float2(ld_agent(r), ld_agent(r + 1))
                          : *reinterpret_cast<const float2 *>(r);
        }
    };
    load_rows(min(s_lo, n_splits - 1), min(16, s_hi - s_lo));
    float mx = kNegBig;
    for (int s = tid; s < n_splits; s += NT) {
        const float m_ = AGENT ? ld_agent(ph + (size_t)s * stride + kHD) : ph[(size_t)s * stride + kHD];
        const float l_ = AGENT ? ld_agent(ph + (size_t)s * stride + kHD + 1)
                               : ph[(size_t)s * stride + kHD + 1];
        w_s[s] = m_;
        l_s[s] = l_;
        mx = fmaxf(mx, m_);
    }
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float lsum = 0.f;
    for (int s = tid; s < n_splits; s += NT) {
        const float w = __expf(w_s[s] - M);
        w_s[s] = w;
        lsum = __builtin_fmaf(w, l_s[s], lsum);
    }
    for (int o = 32; o > 0; o >>= 1) lsum += __shfl_xor(lsum, o, kWave);
    __syncthreads();  // w_s complete; red[0..3] read
    if (lane == 0) red[4 + wave] = lsum;
    // 3. this wave's quarter of the splits
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
        const float L = ((red[4] + red[5]) + red[6]) + red[7];
        const float a = ((acc_s[tid] + acc_s[kHD + tid]) + acc_s[2 * kHD + tid]) + acc_s[3 * kHD + tid];
        res = a / L;
        if (out) out[(size_t)hq * kHD + tid] = res;
    }
    if (limbs_out == nullptr) return;
    __syncthreads();  // acc_s reads done
    if (tid < kHD) acc_s[tid] = res;
    __syncthreads();
    if (tid < kHD / 4) {
        const float4 v = *reinterpret_cast<const float4 *>(&acc_s[4 * tid]);
        limbs_block8<AGENT>(v, tid & 7, &limbs_out[(hq * kHD) / 32 + (tid >> 3)]);
    }
}

}  // namespace
}  // namespace sgq
