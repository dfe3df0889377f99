// x limbs for the Q4_0 GEMV: each 32-block of an fp32 vector is split into
// kLimbs signed 4-bit limbs, x ≈ (amax/7)·(l1 + l2/14 + l3/14² + l4/14³),
// l ∈ [-7, 7] (|error| ≤ amax/7/14³/2 = amax·2.6e-5, below the 2^-12
// relative rounding of an f16 activation), packed eight to a 32-bit word in
// the nibble order of a Q4_0 qs word so that v_dot8_i32_i4 can take the
// weights' nibbles as they are.  Shared by the GEMV and by the kernels
// that produce its input (norms, GeGLU, attention output), which write the
// limb table (BlockLimbs per block) directly.
#pragma once
#include "sgq_internal.h"

namespace sgq {

constexpr int kLimbs = 4;
constexpr float kLimbScale = 1.0f / 2744.0f;  // 14^-3

template <int NBL>
struct XLimbs {
    int q[NBL][kLimbs][4];  // i4 × 8 per word, in the nibble order of a qs word
    float d[NBL];           // (amax/7) / 14^3: scale of the Horner-combined sum
};

// Per-block x limbs as stored in the table the streamed GEMV reads (80 B).
struct BlockLimbs {
    int q[kLimbs][4];
    float d;
    int pad[3];
};

static_assert(sizeof(BlockLimbs) == SGQ_X_LIMBS_BYTES_PER_BLOCK, "limb table layout (sgq.h)");

template <int NBL>
__device__ __forceinline__ void quantize_values(const float (&v)[32], XLimbs<NBL> &L, int i) {
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(v[j]));
    const float d = amax * (1.0f / 7.0f);
    const float id = d > 0.f ? 1.0f / d : 0.f;
    L.d[i] = d * kLimbScale;
    uint32_t word[kLimbs][4] = {};
#pragma unroll
    for (int j = 0; j < 32; j++) {
        float r = v[j] * id;
        const int w = (j & 15) >> 2;
        const int shift = 4 * (2 * (j & 3) + (j >> 4));
#pragma unroll
        for (int l = 0; l < kLimbs; l++) {
            const float c = __builtin_rintf(r);
            r = (r - c) * 14.f;
            word[l][w] |= ((uint32_t)(int)c & 0xFu) << shift;
        }
    }
#pragma unroll
    for (int l = 0; l < kLimbs; l++)
#pragma unroll
        for (int w = 0; w < 4; w++) L.q[i][l][w] = (int)word[l][w];
}

template <int NBL>
__device__ __forceinline__ void quantize_block(const float *__restrict__ xb, XLimbs<NBL> &L,
                                               int i) {
    float v[32];
    const float4 *x4 = reinterpret_cast<const float4 *>(xb);
#pragma unroll
    for (int j = 0; j < 8; j++) {
        float4 t = x4[j];
        v[4 * j] = t.x;
        v[4 * j + 1] = t.y;
        v[4 * j + 2] = t.z;
        v[4 * j + 3] = t.w;
    }
    quantize_values(v, L, i);
}

__device__ __forceinline__ void quantize_to_table(const float *__restrict__ xb, BlockLimbs &t) {
    XLimbs<1> L;
    quantize_block(xb, L, 0);
#pragma unroll
    for (int l = 0; l < kLimbs; l++)
#pragma unroll
        for (int w = 0; w < 4; w++) t.q[l][w] = L.q[0][l][w];
    t.d = L.d[0];
    t.pad[0] = t.pad[1] = t.pad[2] = 0;
}

// Block of 32 values already in registers -> table entry.
__device__ __forceinline__ void limbs_from_values(const float (&v)[32], BlockLimbs &t) {
    XLimbs<1> L;
    quantize_values(v, L, 0);
#pragma unroll
    for (int l = 0; l < kLimbs; l++)
#pragma unroll
        for (int w = 0; w < 4; w++) t.q[l][w] = L.q[0][l][w];
    t.d = L.d[0];
    t.pad[0] = t.pad[1] = t.pad[2] = 0;
}

// The same table entry computed by 8 consecutive lanes: lane group g = lane&7
// holds values 4g..4g+3 of the block (a float4).  amax by xor-shuffles; each
// lane packs its 4 values into the nibbles they occupy in word (g & 3) of
// every limb, lanes g and g^4 OR their halves, lanes g < 4 store word g and
// lane 0 the scale.  Bit-identical to quantize_values (same amax, d, 1/d and
// rint sequence per value).  All 8 lanes of a group must be active.  AGENT:
// agent-scope stores, for a table read by other workgroups of one launch.
// The limb words of an 8-lane group's block: lane g gets word (g & 3) of
// every limb (valid in lanes g < 4) and the block scale.
__device__ __forceinline__ float limbs_words8(const float4 v, int g, uint32_t (&word)[kLimbs]) {
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 4, 64));
    const float d = amax * (1.0f / 7.0f);
    const float id = d > 0.f ? 1.0f / d : 0.f;
    const float vals[4] = {v.x, v.y, v.z, v.w};
    const int hi = g >> 2;  // values 16..31 sit in the high nibble of each byte
#pragma unroll
    for (int l = 0; l < kLimbs; l++) word[l] = 0u;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        float r = vals[e] * id;
        const int shift = 4 * (2 * e + hi);
#pragma unroll
        for (int l = 0; l < kLimbs; l++) {
            const float c = __builtin_rintf(r);
            r = (r - c) * 14.f;
            word[l] |= ((uint32_t)(int)c & 0xFu) << shift;
        }
    }
#pragma unroll
    for (int l = 0; l < kLimbs; l++) word[l] |= (uint32_t)__shfl_xor((int)word[l], 4, 64);
    return d * kLimbScale;
}

// The same table entry computed by 8 consecutive lanes: lane group g = lane&7
// holds values 4g..4g+3 of the block (a float4).  amax by xor-shuffles; each
// lane packs its 4 values into the nibbles they occupy in word (g & 3) of
// every limb, lanes g and g^4 OR their halves, lanes g < 4 store word g and
// lane 0 the scale.  Bit-identical to quantize_values (same amax, d, 1/d and
// rint sequence per value).  All 8 lanes of a group must be active.  AGENT:
// agent-scope stores, for a table read by other workgroups of one launch.
template <bool AGENT = false>
__device__ __forceinline__ void limbs_block8(const float4 v, int g, BlockLimbs *__restrict__ dst) {
    uint32_t word[kLimbs];
    const float d = limbs_words8(v, g, word);
    if (g < 4) {
        if (AGENT) {
#pragma unroll
            for (int l = 0; l < kLimbs; l++)
                __hip_atomic_store(&dst->q[l][g], (int)word[l], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            if (g == 0)
                __hip_atomic_store(&dst->d, d, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
#pragma unroll
            for (int l = 0; l < kLimbs; l++) dst->q[l][g] = (int)word[l];
            if (g == 0) {
                dst->d = d;
                dst->pad[0] = dst->pad[1] = dst->pad[2] = 0;
            }
        }
    }
}

}  // namespace sgq
