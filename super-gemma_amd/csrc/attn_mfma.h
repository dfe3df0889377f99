// Q8_0-KV split-K decode attention for gfx950, QK on the int8 matrix cores.
//
// Semantics as attn_split (attn_body.h; attn_decode_global_q8k.wgsl:41-112):
// s_t = scale · q_h·k_t over the valid slots t of the split's chunk, online
// softmax, partial (acc, m, l) per (query head, split) merged later in
// split order (attn_reduce.wgsl:40-52).  K and V are Q8_0 pages (int8
// quants [slot × n_kv × 128], f16 scales [slot × n_kv × 4]).
//
// Design (one wave = 32 slots at a time, no workgroup barrier in the loop):
//  * q in int8 limbs.  Each query head h is written as
//    q ≈ d_h·(l0 + l1/254 + l2/254²), d_h = ‖q_h‖₂/127 ≥ max|q_h|/127,
//    |l_i| ≤ 127 (representation error ≤ 6.1e-8·‖q_h‖, below fp32
//    rounding of the dot; the 2-norm is a bound that RoPE preserves, so it
//    comes from the norm's own reduction).  One v_mfma_i32_32x32x32_i8 per 32-dim block b then gives, for
//    32 slots at once, the exact integer dots of the block's K quants with
//    every limb of both heads: A row r = 8b' + 4h + limb holds the limb of
//    q_h on block b' (zero elsewhere, so the four block MFMAs accumulate
//    into one tile without mixing blocks), B column t is slot t's K row.
//    Lane (t, h) = (lane%32, lane/32) ends up with the 12 integer dots of
//    its slot and head, and the score is
//    s = scale·d_h·Σ_b ks[t,b]·(C0 + C1/254 + C2/254²).
//    The K quants go from HBM straight into the MFMA operand registers.
//  * Online softmax per wave and head (two 32-lane halves), the running
//    sum kept per lane and reduced once at the end.
//  * PV on the VALU: lane (c, parity) = (lane%32, lane/32) owns dims
//    4c..4c+3 of both heads for the slots of its parity; p·vs[t, c/8] for
//    both heads comes from a per-wave LDS strip (written by the QK lanes,
//    8 distinct addresses per read, so broadcast), the V word from a
//    dword load issued with the K rows (each load covers two whole rows).
//  * The waves of a workgroup take the chunk's 32-slot groups round robin
//    and prefetch their next group while computing the current one; their
//    states are combined in LDS in wave order at the end.  A workgroup that
//    owns the whole cache of its kv head (one split) writes the output
//    rows and the x limbs of the next GEMV itself.
//  * The projections of the current token (FUSED) are loaded before the
//    first K/V group: vector loads complete in issue order, so the
//    post-projection would otherwise wait for the whole group.
#pragma once
#include "attn_body.h"

namespace sgq {
namespace {

typedef int v4i_a __attribute__((ext_vector_type(4)));
typedef int v16i_a __attribute__((ext_vector_type(16)));

constexpr int kAttnWaves = 4;  // waves per workgroup

template <int CTRL>
__device__ __forceinline__ float dpp_max(float v) {
    const int t = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false);
    return fmaxf(v, __builtin_bit_cast(float, t));
}
// Max over each 16-lane row, in every lane of the row.
__device__ __forceinline__ float row_max_dpp(float v) {
    v = dpp_max<0xB1>(v);   // quad_perm [1,0,3,2]
    v = dpp_max<0x4E>(v);   // quad_perm [2,3,0,1]
    v = dpp_max<0x141>(v);  // row_half_mirror
    return dpp_max<0x140>(v);  // row_mirror
}
__device__ __forceinline__ float readlane_f(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
constexpr float kLimbBase = 254.f;

// One wave's loads for a 32-slot group: lane (t, kh) takes bytes
// [32b + 16kh, +16) of slot t's K row for every block b, and the V word
// 4c..4c+3 of slots 2i + parity.
struct AttnGroup {
    v4i_a k[4];
    uint2 ks, vs;
    int v[16];
};

__device__ __forceinline__ void attn_group_load(AttnGroup &g, const int8_t *__restrict__ kq,
                                                const uint16_t *__restrict__ ks,
                                                const int8_t *__restrict__ vq,
                                                const uint16_t *__restrict__ vs, uint32_t tb,
                                                uint32_t t_end, int n_kv, int kvh, int lane) {
    // slots past t_end read the last valid row (their scores are masked and
    // their probabilities are zero), so the loads need no branches
    const uint32_t last = t_end - 1;
    const int kh = lane >> 5, c = lane & 31;
    const size_t row = (size_t)min(tb + (uint32_t)c, last) * n_kv + kvh;
    const v4i_a *kp = reinterpret_cast<const v4i_a *>(kq + row * kHD + 16 * kh);
#pragma unroll
    for (int b = 0; b < 4; b++) g.k[b] = kp[2 * b];
    g.ks = *reinterpret_cast<const uint2 *>(ks + row * (kHD / 32));
    g.vs = *reinterpret_cast<const uint2 *>(vs + row * (kHD / 32));
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const size_t rv = (size_t)min(tb + 2 * i + kh, last) * n_kv + kvh;
        g.v[i] = *reinterpret_cast<const int *>(vq + rv * kHD + 4 * c);
    }
}

// One 32-slot group of one wave (slots tb .. tb+31, valid below t_end):
// QK on the int8 matrix cores against the q limbs in qa (this lane feeds
// block myb), scores scaled by dh, online softmax per head (the running
// max m_run and this lane's sum l_lane), p·vs into the wave's LDS strip
// pw, and PV on the VALU into acc (dims 4c..4c+3 of both heads, slots of
// this lane's parity).
template <int QPK>
__device__ __forceinline__ void attn_group_compute(const AttnGroup &g, uint32_t tb,
                                                   uint32_t t_end, int lane, v4i_a qa, int myb,
                                                   float dh, float (&m_run)[2], float &l_lane,
                                                   float (&acc)[2][4], float *pw) {
    const int hq = lane >> 5, c = lane & 31, par = lane >> 5;
    // ---- QK: four block MFMAs into one tile
    v16i_a dacc = {};
#pragma unroll
    for (int b = 0; b < 4; b++) {
        const v4i_a a = myb == b ? qa : v4i_a{0, 0, 0, 0};
        dacc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, g.k[b], dacc, 0, 0, 0);
    }
    float s = 0.f;
    {
        const float ksf[4] = {f16_bits_to_f32(g.ks.x & 0xffff), f16_bits_to_f32(g.ks.x >> 16),
                              f16_bits_to_f32(g.ks.y & 0xffff), f16_bits_to_f32(g.ks.y >> 16)};
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const float blk = (float)dacc[4 * b] +
                              (float)dacc[4 * b + 1] * (1.0f / kLimbBase) +
                              (float)dacc[4 * b + 2] * (1.0f / (kLimbBase * kLimbBase));
            s = __builtin_fmaf(ksf[b], blk, s);
        }
    }
    const bool valid = tb + (uint32_t)c < t_end && hq < QPK;
    s = valid ? s * dh : kNegBig;
    // ---- online softmax per head (32-lane halves)
    // max over each 16-lane row on the VALU (DPP), then over the two
    // rows of each head from lanes 0/16 and 32/48
    const float mx = row_max_dpp(s);
    const float M0 = fmaxf(readlane_f(mx, 0), readlane_f(mx, 16));
    const float M1 = fmaxf(readlane_f(mx, 32), readlane_f(mx, 48));
    const float mn0 = fmaxf(m_run[0], M0), mn1 = fmaxf(m_run[1], M1);
    const float corr0 = __expf(m_run[0] - mn0), corr1 = __expf(m_run[1] - mn1);
    m_run[0] = mn0;
    m_run[1] = mn1;
    const float p = valid ? __expf(s - (hq ? mn1 : mn0)) : 0.f;
    l_lane = __builtin_fmaf(l_lane, hq ? corr1 : corr0, p);
    // p·vs[t, b] for the PV lanes: strip [t][b][h]
    {
        const float vsf[4] = {f16_bits_to_f32(g.vs.x & 0xffff), f16_bits_to_f32(g.vs.x >> 16),
                              f16_bits_to_f32(g.vs.y & 0xffff), f16_bits_to_f32(g.vs.y >> 16)};
#pragma unroll
        // (select, not multiply: a masked slot's scale may be any bits)
        for (int b = 0; b < 4; b++) pw[(c * 4 + b) * 2 + hq] = valid ? p * vsf[b] : 0.f;
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int e = 0; e < 4; e++) {
        acc[0][e] *= corr0;
        acc[1][e] *= corr1;
    }
    // ---- PV: dims 4c..4c+3, slots 2i + par
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const float2 pp =
            *reinterpret_cast<const float2 *>(&pw[((2 * i + par) * 4 + (c >> 3)) * 2]);
        const int w = g.v[i];
        const float v0 = (float)(int8_t)(w & 0xff), v1 = (float)(int8_t)((w >> 8) & 0xff);
        const float v2 = (float)(int8_t)((w >> 16) & 0xff), v3 = (float)(int8_t)(w >> 24);
        acc[0][0] = __builtin_fmaf(pp.x, v0, acc[0][0]);
        acc[0][1] = __builtin_fmaf(pp.x, v1, acc[0][1]);
        acc[0][2] = __builtin_fmaf(pp.x, v2, acc[0][2]);
        acc[0][3] = __builtin_fmaf(pp.x, v3, acc[0][3]);
        if (QPK == 2) {
            acc[1][0] = __builtin_fmaf(pp.y, v0, acc[1][0]);
            acc[1][1] = __builtin_fmaf(pp.y, v1, acc[1][1]);
            acc[1][2] = __builtin_fmaf(pp.y, v2, acc[1][2]);
            acc[1][3] = __builtin_fmaf(pp.y, v3, acc[1][3]);
        }
    }
    __builtin_amdgcn_wave_barrier();
}

// The split work item of kv head kvh over the split's slots.  With
// n_splits > 1, or with neither out nor limbs_out given, it writes the
// partial (acc, m, l) of its QPK query heads to part (agent-scope stores, so
// a merge in the same launch may read them after an atomic handoff);
// otherwise (one split) it writes the normalised rows to out and/or their x
// limbs to limbs_out.  q is read
// from global memory unless FUSED, in which case the post-projection of
// AttnPost runs first (and split 0 appends the new K/V row).  All W·64
// threads call.
template <int QPK, bool FUSED, int W>
__device__ __forceinline__ void attn_chunk(const float *__restrict__ q,
                                           const int8_t *__restrict__ kq,
                                           const uint16_t *__restrict__ ks,
                                           const int8_t *__restrict__ vq,
                                           const uint16_t *__restrict__ vs, uint32_t kv_len,
                                           int n_kv, int n_splits, float scale,
                                           float *__restrict__ part, float *__restrict__ out,
                                           BlockLimbs *__restrict__ limbs_out,
                                           const AttnPost &post, int kvh, int split,
                                           uint32_t pos) {
    static_assert(QPK == 1 || QPK == 2, "1 or 2 query heads per kv head");
    static_assert(W == 4, "the post-projection maps 256 threads");
    // q limbs [head][limb][dim] (limb 3 = zero row)
    __shared__ __align__(16) int8_t ql_s[2][4][kHD];
    __shared__ float amax_s[2];  // ‖q_h‖, the limb scale bound
    __shared__ __align__(16) int fk_s[kHD / 4], fv_s[kHD / 4];
    __shared__ __align__(8) uint16_t fks_s[kHD / 32], fvs_s[kHD / 32];
    __shared__ __align__(16) float pw_s[W][32 * 4 * 2];     // per wave: [t][b][h]
    __shared__ __align__(16) float wacc_s[W][QPK][kHD];
    __shared__ float wml_s[W][2][2];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // chunk of 32-slot groups: groups never straddle a split boundary
    const uint32_t per = (kv_len + n_splits - 1) / n_splits;
    const uint32_t chunk = (per + 31) & ~31u;
    const uint32_t t_begin = min((uint32_t)split * chunk, kv_len);
    const uint32_t t_end = min(t_begin + chunk, kv_len);
    const uint32_t n_groups = (t_end - t_begin + 31) / 32;

    // ---- this token's projections, all loaded up front.  Threads 0..255:
    // head (or k|v) h = tid/128; within it wave half w2 and lane l take
    // dim d = i + 64·(l/32), i = 32·w2 + l%32, so the NEOX RoPE partner
    // (dim i ↔ i + 64) is lane l^32 of the same wave, and each 32-lane half
    // holds one 32-dim block.
    const bool pt = tid < 2 * kHD;
    const int h = (tid >> 7) & 1, i_r = 32 * ((tid >> 6) & 1) + (lane & 31);
    const int d = i_r + 64 * (lane >> 5);
    float qv = 0.f, kvv = 0.f, wqd = 0.f, wkd = 0.f, cs_c = 1.f, cs_s = 0.f;
    if (pt && h < QPK) qv = FUSED ? post.q_raw[(size_t)kvh * QPK * kHD + h * kHD + d]
                                  : q[(size_t)kvh * QPK * kHD + h * kHD + d];
    if (FUSED && pt) {
        kvv = h == 0 ? post.k_raw[(size_t)kvh * kHD + d] : post.v_src[(size_t)kvh * kHD + d];
        wqd = post.wq[d];
        wkd = h == 0 ? post.wk[d] : 1.f;
        cs_c = post.rope_cs[2 * i_r];
        cs_s = post.rope_cs[2 * i_r + 1];
    }

    AttnGroup ga, gb;
    if ((uint32_t)wave < n_groups)
        attn_group_load(ga, kq, ks, vq, vs, t_begin + 32 * wave, t_end, n_kv, kvh, lane);

    // per-head sums: Σq², Σk² | Σv², Σ(q·w_q)²  (two waves per head)
    __shared__ float pred[3][4];
    {
        float a = qv * qv, b = kvv * kvv, e = qv * wqd * qv * wqd;
        for (int o = 32; o > 0; o >>= 1) {
            a += __shfl_xor(a, o, kWave);
            if (FUSED) {
                b += __shfl_xor(b, o, kWave);
                e += __shfl_xor(e, o, kWave);
            }
        }
        if (lane == 0 && pt) pred[0][wave] = a, pred[1][wave] = b, pred[2][wave] = e;
    }
    __syncthreads();
    uint32_t fresh_slot = 0xffffffffu;
    float qnorm;  // ‖q_h‖ after norm and RoPE (RoPE keeps it)
    if (FUSED) {
        fresh_slot = post.ring ? pos % (uint32_t)post.ring : pos;
        const float sq = pred[0][2 * h] + pred[0][2 * h + 1];
        const float skv = pred[1][2 * h] + pred[1][2 * h + 1];
        const float sqw = pred[2][2 * h] + pred[2][2 * h + 1];
        const float rq = 1.0f / sqrtf(sq / (float)kHD + post.eps);
        qv = qv * rq * wqd;
        qnorm = sqrtf(sqw) * rq;
        kvv = kvv * (1.0f / sqrtf(skv / (float)kHD + post.eps)) * wkd;
        // NEOX RoPE with the partner lane
        const float qp = __shfl_xor(qv, 32, kWave), kp = __shfl_xor(kvv, 32, kWave);
        const bool lo = lane < 32;
        qv = lo ? qv * cs_c - qp * cs_s : qv * cs_c + qp * cs_s;
        if (h == 0) kvv = lo ? kvv * cs_c - kp * cs_s : kvv * cs_c + kp * cs_s;
        // Q8_0 of the new row (kv_quant_q8.wgsl:41-56): 32-lane groups
        float amax = fabsf(kvv);
        for (int o = 16; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, kWave));
        const float dq = amax * (1.0f / 127.0f);
        const float id = dq > 0.f ? 1.0f / dq : 0.f;
        const int8_t qi = (int8_t)(int)__builtin_rintf(kvv * id);
        const uint16_t sc = f32_to_f16_bits(dq);
        if (pt) {
            reinterpret_cast<int8_t *>(h == 0 ? fk_s : fv_s)[d] = qi;
            if ((d & 31) == 0) (h == 0 ? fks_s : fvs_s)[d / 32] = sc;
            if (split == 0) {
                const size_t e = ((size_t)fresh_slot * n_kv + kvh) * kHD + d;
                (h == 0 ? post.kq_w : post.vq_w)[e] = qi;
                if ((d & 31) == 0) (h == 0 ? post.ks_w : post.vs_w)[e / 32] = sc;
            }
        }
    } else {
        qnorm = sqrtf(pred[0][2 * h] + pred[0][2 * h + 1]);
    }
    // ---- q limbs against the bound ‖q_h‖ ≥ max|q_h|: l0, l1, l2
    if (pt) {
        const float y = qnorm > 0.f ? qv * (127.0f / qnorm) : 0.f;
        const float l0 = __builtin_rintf(y);
        const float r1 = (y - l0) * kLimbBase;
        const float l1 = __builtin_rintf(r1);
        const float l2 = __builtin_rintf((r1 - l1) * kLimbBase);
        ql_s[h][0][d] = (int8_t)(int)l0;
        ql_s[h][1][d] = (int8_t)(int)l1;
        ql_s[h][2][d] = (int8_t)(int)l2;
        ql_s[h][3][d] = 0;
        if (d == 0) amax_s[h] = qnorm;
    }
    __syncthreads();
    // A operand: lane (r, kh), r = 8b + 4h + limb: 16 limb bytes of
    // q_h[32b + 16kh ..] (heads >= QPK hold zeros)
    const int myb = (lane & 31) >> 3;  // the block whose MFMA this lane's A feeds
    const v4i_a qa = *reinterpret_cast<const v4i_a *>(
        &ql_s[(lane >> 2) & 1][lane & 3][32 * myb + 16 * (lane >> 5)]);
    // score factor of lane (t, h): scale·d_h
    const int hq = lane >> 5;
    const float dh = amax_s[hq] * (1.0f / 127.0f) * scale;

    float m_run[2] = {kNegBig, kNegBig};
    float l_lane = 0.f;
    float acc[2][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    float *pw = pw_s[wave];
    const int c = lane & 31, par = lane >> 5;

    const uint32_t n_mine = (uint32_t)wave < n_groups ? (n_groups - 1 - wave) / W + 1 : 0;
    // group j of this wave in g, group j+1 loading into gn (loop unrolled by
    // two so that the two buffers keep fixed registers)
    auto step = [&](uint32_t j, AttnGroup &g, AttnGroup &gn) {
        const uint32_t tb = t_begin + 32 * (wave + W * j);
        if (j + 1 < n_mine)
            attn_group_load(gn, kq, ks, vq, vs, tb + 32 * W, t_end, n_kv, kvh, lane);
        if (FUSED && fresh_slot - tb < 32u) {  // the new row replaces the cache's
            if (tb + (uint32_t)c == fresh_slot) {
#pragma unroll
                for (int b = 0; b < 4; b++)
                    g.k[b] = *reinterpret_cast<const v4i_a *>(&fk_s[8 * b + 4 * par]);
                g.ks = *reinterpret_cast<const uint2 *>(fks_s);
                g.vs = *reinterpret_cast<const uint2 *>(fvs_s);
            }
#pragma unroll
            for (int i = 0; i < 16; i++)
                if (tb + 2 * i + par == fresh_slot) g.v[i] = fv_s[c];
        }
        attn_group_compute<QPK>(g, tb, t_end, lane, qa, myb, dh, m_run, l_lane, acc, pw);
    };
    for (uint32_t j = 0; j < n_mine; j += 2) {
        step(j, ga, gb);
        if (j + 1 < n_mine) step(j + 1, gb, ga);
    }

    // ---- wave state: sum of p per head, both slot parities of acc
    for (int o = 16; o > 0; o >>= 1) l_lane += __shfl_xor(l_lane, o, kWave);
#pragma unroll
    for (int hh = 0; hh < QPK; hh++)
#pragma unroll
        for (int e = 0; e < 4; e++) acc[hh][e] += __shfl_xor(acc[hh][e], 32, kWave);
    if (lane < 32) {
#pragma unroll
        for (int hh = 0; hh < QPK; hh++)
            *reinterpret_cast<float4 *>(&wacc_s[wave][hh][4 * c]) =
                make_float4(acc[hh][0], acc[hh][1], acc[hh][2], acc[hh][3]);
    }
    if (lane == 0 || lane == 32) {
        wml_s[wave][hq][0] = m_run[hq];
        wml_s[wave][hq][1] = l_lane;
    }
    __syncthreads();
    // ---- combine the waves in wave order
    const int stride = kHD + 2;
    float a = 0.f, l = 0.f, M = kNegBig;
    const bool ot = tid < QPK * kHD;
    const int oh = ot ? tid / kHD : 0;
    if (ot) {
#pragma unroll
        for (int w = 0; w < W; w++) M = fmaxf(M, wml_s[w][oh][0]);
#pragma unroll
        for (int w = 0; w < W; w++) {
            const float f = __expf(wml_s[w][oh][0] - M);
            a = __builtin_fmaf(wacc_s[w][oh][d], f, a);
            l = __builtin_fmaf(wml_s[w][oh][1], f, l);
        }
    }
    if (n_splits > 1 || (out == nullptr && limbs_out == nullptr)) {
        if (ot) {
            const size_t rowp = ((size_t)(kvh * QPK + oh) * n_splits + split) * stride;
            st_agent(&part[rowp + d], a);
            if (d == 0) {
                st_agent(&part[rowp + kHD], M);
                st_agent(&part[rowp + kHD + 1], l);
            }
        }
        return;
    }
    // one split: the rows themselves (and the next GEMV's limbs)
    const float res = a / l;
    if (ot && out) out[(size_t)(kvh * QPK + oh) * kHD + d] = res;
    if (limbs_out == nullptr) return;
    __syncthreads();  // wacc_s reads done
    float *o_s = &wacc_s[0][0][0];
    if (ot) o_s[oh * kHD + d] = res;  // thread tid holds dim d of head oh (not dim tid)
    __syncthreads();
    if (tid < QPK * kHD / 4) {
        const float4 v = *reinterpret_cast<const float4 *>(&o_s[4 * tid]);
        limbs_block8<false>(v, tid & 7, &limbs_out[(kvh * QPK * kHD) / 32 + (tid >> 3)]);
    }
}

// The same split work item with one wave per kv head: wave w of the
// workgroup takes kv head kvh0 + w over all the split's 32-slot groups (two
// in flight), so the four waves of a workgroup read the four heads' 128-byte
// rows of the same slots (512 contiguous bytes of each slot's K and V row)
// and share each slot's f16 scale line (one 128-byte line holds all heads'
// scales of a slot) in the CU's caches.  The wave writes its QPK partials
// (acc, m, l) itself; no cross-wave combine.  q from global memory (fp32,
// [n_q × 128]); QPK·128 values per wave, four per lane.
template <int QPK>
__device__ __forceinline__ void attn_split_per_wave(
    const float *__restrict__ q, const int8_t *__restrict__ kq, const uint16_t *__restrict__ ks,
    const int8_t *__restrict__ vq, const uint16_t *__restrict__ vs, uint32_t kv_len, int n_kv,
    int n_splits, float scale, float *__restrict__ part, int kvh, int split,
    int8_t (&ql)[2][4][kHD], float (&qn)[2], float *pw) {
    static_assert(QPK == 1 || QPK == 2, "1 or 2 query heads per kv head");
    const int lane = threadIdx.x & (kWave - 1);
    const uint32_t per = (kv_len + n_splits - 1) / n_splits;
    const uint32_t chunk = (per + 31) & ~31u;
    const uint32_t t_begin = min((uint32_t)split * chunk, kv_len);
    const uint32_t t_end = min(t_begin + chunk, kv_len);
    const uint32_t n_groups = (t_end - t_begin + 31) / 32;

    // the first group's loads go out before the q limbs are formed
    AttnGroup ga, gb;
    if (n_groups > 0) attn_group_load(ga, kq, ks, vq, vs, t_begin, t_end, n_kv, kvh, lane);

    // q limbs against ‖q_h‖: lane (h, i) = (lane/32, lane%32) holds dims
    // 4i..4i+3 of head h (heads >= QPK are zero)
    {
        const int h = lane >> 5, d0 = 4 * (lane & 31);
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (h < QPK) v = *reinterpret_cast<const float4 *>(q + (size_t)(kvh * QPK + h) * kHD + d0);
        float ss = v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        for (int o = 16; o > 0; o >>= 1) ss += __shfl_xor(ss, o, kWave);
        const float qnorm = sqrtf(ss);
        const float f[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float y = qnorm > 0.f ? f[e] * (127.0f / qnorm) : 0.f;
            const float l0 = __builtin_rintf(y);
            const float r1 = (y - l0) * kLimbBase;
            const float l1 = __builtin_rintf(r1);
            const float l2 = __builtin_rintf((r1 - l1) * kLimbBase);
            ql[h][0][d0 + e] = (int8_t)(int)l0;
            ql[h][1][d0 + e] = (int8_t)(int)l1;
            ql[h][2][d0 + e] = (int8_t)(int)l2;
            ql[h][3][d0 + e] = 0;
        }
        if ((lane & 31) == 0) qn[h] = qnorm;
    }
    __builtin_amdgcn_wave_barrier();  // (LDS operations of one wave complete in order)
    const int myb = (lane & 31) >> 3;
    const v4i_a qa = *reinterpret_cast<const v4i_a *>(
        &ql[(lane >> 2) & 1][lane & 3][32 * myb + 16 * (lane >> 5)]);
    const int hq = lane >> 5;
    const float dh = qn[hq] * (1.0f / 127.0f) * scale;

    float m_run[2] = {kNegBig, kNegBig};
    float l_lane = 0.f;
    float acc[2][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    for (uint32_t j = 0; j < n_groups; j += 2) {
        const uint32_t tb = t_begin + 32 * j;
        if (j + 1 < n_groups) attn_group_load(gb, kq, ks, vq, vs, tb + 32, t_end, n_kv, kvh, lane);
        attn_group_compute<QPK>(ga, tb, t_end, lane, qa, myb, dh, m_run, l_lane, acc, pw);
        if (j + 1 >= n_groups) break;
        if (j + 2 < n_groups) attn_group_load(ga, kq, ks, vq, vs, tb + 64, t_end, n_kv, kvh, lane);
        attn_group_compute<QPK>(gb, tb + 32, t_end, lane, qa, myb, dh, m_run, l_lane, acc, pw);
    }
    // the wave's partials: sum of p per head, both slot parities of acc
    for (int o = 16; o > 0; o >>= 1) l_lane += __shfl_xor(l_lane, o, kWave);
#pragma unroll
    for (int hh = 0; hh < QPK; hh++)
#pragma unroll
        for (int e = 0; e < 4; e++) acc[hh][e] += __shfl_xor(acc[hh][e], 32, kWave);
    constexpr int stride = kHD + 2;
    const int c = lane & 31;
    if (lane < 32) {
#pragma unroll
        for (int hh = 0; hh < QPK; hh++) {
            float *pr = part + ((size_t)(kvh * QPK + hh) * n_splits + split) * stride;
            *reinterpret_cast<float2 *>(pr + 4 * c) = make_float2(acc[hh][0], acc[hh][1]);
            *reinterpret_cast<float2 *>(pr + 4 * c + 2) = make_float2(acc[hh][2], acc[hh][3]);
        }
    }
    if ((lane & 31) == 0 && hq < QPK) {
        float *pr = part + ((size_t)(kvh * QPK + hq) * n_splits + split) * stride;
        pr[kHD] = m_run[hq];
        pr[kHD + 1] = l_lane;
    }
}

}  // namespace
}  // namespace sgq
