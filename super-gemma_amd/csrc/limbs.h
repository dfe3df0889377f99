// x limbs for the Q4_0 GEMV: each 32-block of an fp32 vector is split into
// kLimbs signed 4-bit limbs, x ≈ (amax/7)·(l1 + l2/14 + l3/14² + l4/14³ +
// l5/14⁴), l ∈ [-7, 7] (|error| ≤ amax·1.9e-6), packed eight to a 32-bit
// word in the nibble order of a Q4_0 qs word so that v_dot8_i32_i4 can take
// the weights' nibbles as they are.  Shared by the GEMV and by the kernels
// that produce its input (norms, GeGLU, attention output), which write the
// limb table (BlockLimbs per block) directly.
#pragma once
#include "sgq_internal.h"

namespace sgq {

constexpr int kLimbs = 5;

template <int NBL>
struct XLimbs {
    int q[NBL][kLimbs][4];  // i4 × 8 per word, in the nibble order of a qs word
    float d[NBL];           // (amax/7) / 14^4: scale of the Horner-combined sum
};

// Per-block x limbs as stored in the table the streamed GEMV reads (96 B).
struct BlockLimbs {
    int q[kLimbs][4];
    float d;
    int pad[3];
};

template <int NBL>
__device__ __forceinline__ void quantize_values(const float (&v)[32], XLimbs<NBL> &L, int i) {
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(v[j]));
    const float d = amax * (1.0f / 7.0f);
    const float id = d > 0.f ? 1.0f / d : 0.f;
    L.d[i] = d * (1.0f / 38416.0f);  // 14^4
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

}  // namespace sgq
