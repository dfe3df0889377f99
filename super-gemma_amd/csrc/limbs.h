// x limbs for the Q4_0 GEMV: each value of a 32-block of an fp32 vector is
// rounded to an integer v = rint(x·(7/amax)·4096), |v| <= 28672, and v is
// written as four signed base-16 digits, v = 16³·l1 + 16²·l2 + 16·l3 + l4,
// l ∈ [-8, 7]: with u = v + 0x8888 every nibble of u is a digit plus 8, so
// the digits are the nibbles of u ^ 0x8888 read as signed 4-bit numbers.
// x ≈ d·v with d = (amax/7)/4096 (|error| ≤ amax/57344 = amax·1.7e-5, below
// the 2^-12 relative rounding of an f16 activation).  The limbs are packed
// eight to a 32-bit word in the nibble order of a Q4_0 qs word so that
// v_dot8_i32_i4 can take the weights' nibbles as they are.  Shared by the
// GEMV and by the kernels that produce its input (norms, GeGLU, attention
// output), which write the limb table (BlockLimbs per block) directly.
#pragma once
#include "sgq_internal.h"

namespace sgq {

constexpr int kLimbs = 4;
constexpr float kLimbScale = 1.0f / 4096.0f;  // 16^-3
constexpr int kLimbBias = 0x8888;              // Σ 8·16^k, k < 4

template <int NBL>
struct XLimbs {
    int q[NBL][kLimbs][4];  // i4 × 8 per word, in the nibble order of a qs word
    float d[NBL];           // (amax/7) / 16^3: scale of the Horner-combined sum
};

// Per-block x limbs as stored in the table the streamed GEMV reads (80 B).
struct BlockLimbs {
    int q[kLimbs][4];
    float d;
    int pad[3];
};

static_assert(sizeof(BlockLimbs) == SGQ_X_LIMBS_BYTES_PER_BLOCK, "limb table layout (sgq.h)");

// The biased value u = v + 0x8888 of x·(7/amax)·4096 (id = 4096/d with the
// hardware reciprocal: its < 1 ulp error moves x·id by < 0.01, and the
// table's scale is d itself, so it only shifts which way a value rounds):
// one FMA, rint, convert (the bias is added before rounding; |v| <= 28672
// keeps u in [6280, 63624], where a float still resolves 2^-8).  Nibble k
// of u is digit k plus 8; XOR with 8 turns it into the signed 4-bit digit.
__device__ __forceinline__ uint32_t limb_biased(float x, float id) {
    return (uint32_t)(int)__builtin_rintf(__builtin_fmaf(x, id, (float)kLimbBias));
}

template <int NBL>
__device__ __forceinline__ void quantize_values(const float (&v)[32], XLimbs<NBL> &L, int i) {
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(v[j]));
    const float d = amax * (1.0f / 7.0f);
    const float id = d > 0.f ? 4096.0f * __builtin_amdgcn_rcpf(d) : 0.f;
    L.d[i] = d * kLimbScale;
    uint32_t word[kLimbs][4] = {};
#pragma unroll
    for (int j = 0; j < 32; j++) {
        const uint32_t u = limb_biased(v[j], id) ^ (uint32_t)kLimbBias;
        const int w = (j & 15) >> 2;
        const int shift = 4 * (2 * (j & 3) + (j >> 4));
#pragma unroll
        for (int l = 0; l < kLimbs; l++)
            word[l][w] |= ((u >> (4 * (kLimbs - 1 - l))) & 0xFu) << shift;
    }
#pragma unroll
    for (int l = 0; l < kLimbs; l++)
#pragma unroll
        for (int w = 0; w < 4; w++) L.q[i][l][w] = (int)word[l][w];
}

template <int NBL, typename T>
__device__ __forceinline__ void quantize_block(const T *__restrict__ xb, XLimbs<NBL> &L, int i) {
    float v[32];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        float4 t = act_ld4(xb, j);
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

// DPP lane moves inside 8-lane groups (no LDS traffic): quad_perm swaps
// for xor 1 and 2, row_half_mirror (lane i <- 7-i) to meet the other quad,
// row_ror:12 (lane i <- i+4 within a 16-lane row) to fetch lane g+4's word.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_mov(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}
__device__ __forceinline__ float max8(float a) {
    a = fmaxf(a, __builtin_bit_cast(float, dpp_mov<0xB1>(__builtin_bit_cast(uint32_t, a))));
    a = fmaxf(a, __builtin_bit_cast(float, dpp_mov<0x4E>(__builtin_bit_cast(uint32_t, a))));
    return fmaxf(a, __builtin_bit_cast(float, dpp_mov<0x141>(__builtin_bit_cast(uint32_t, a))));
}

// The limb words of an 8-lane group's block, where lane g = lane & 7 holds
// values 4g..4g+3 (a float4): amax over the group; each lane's four biased
// values (16 nibbles) are transposed with two byte permutes so that limb l
// of value e lands in byte e of word l (low nibble for g < 4, high nibble
// for g >= 4), and lanes g < 4 OR in the other half from lane g+4.  Valid
// in lanes g < 4; returns the block scale.  Bit-identical to
// quantize_values (same amax, d, scale, FMA and rint per value).  All 8
// lanes of a group must be active.
__device__ __forceinline__ float limbs_words8(const float4 v, int g, uint32_t (&word)[kLimbs]) {
    const float amax = max8(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    const float d = amax * (1.0f / 7.0f);
    const float id = d > 0.f ? 4096.0f * __builtin_amdgcn_rcpf(d) : 0.f;
    const uint32_t u01 = limb_biased(v.x, id) | (limb_biased(v.y, id) << 16);
    const uint32_t u23 = limb_biased(v.z, id) | (limb_biased(v.w, id) << 16);
    // byte e of hi/lo = digits (3, 2) / (1, 0) of value e, high nibble first
    const uint32_t hi = __builtin_amdgcn_perm(u23, u01, 0x07050301u);
    const uint32_t lo = __builtin_amdgcn_perm(u23, u01, 0x06040200u);
    const uint32_t sh = (uint32_t)(g >> 2) * 4u;  // values 16..31: high nibbles
    const uint32_t m = 0x0F0F0F0Fu, flip = 0x08080808u;
    word[0] = (((hi >> 4) & m) ^ flip) << sh;
    word[1] = ((hi & m) ^ flip) << sh;
    word[2] = (((lo >> 4) & m) ^ flip) << sh;
    word[3] = ((lo & m) ^ flip) << sh;
#pragma unroll
    for (int l = 0; l < kLimbs; l++) word[l] |= dpp_mov<0x12C>(word[l]);  // row_ror:12
    return d * kLimbScale;
}

// The table entry of an 8-lane group's block (limbs_words8): lanes g < 4
// store word g of every limb, lane 0 the scale.  AGENT: agent-scope
// stores, for a table read by other workgroups of one launch.
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
