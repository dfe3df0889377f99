// Q8_0 quantization of a 32-block held by 8 consecutive lanes (one float4
// each), kv_quant_q8 semantics (crates/sg-gpu/shaders/kv_quant_q8.wgsl:41-56):
// amax in f32, d = amax * (1/127), id = d > 0 ? 1/d : 0 from the unrounded d
// (IEEE division), scale = f16(d) RTNE, q = round_ties_even(x * id).  Shared
// by the quant kernel and the producers that emit Q8_0 directly.
#pragma once
#include "sgq_internal.h"

namespace sgq {

__device__ __forceinline__ int pack_q(float a, float b, float c, float d, float id) {
    int qa = (int)__builtin_rintf(a * id);
    int qb = (int)__builtin_rintf(b * id);
    int qc = (int)__builtin_rintf(c * id);
    int qd = (int)__builtin_rintf(d * id);
    return (qa & 0xff) | ((qb & 0xff) << 8) | ((qc & 0xff) << 16) | ((qd & 0xff) << 24);
}

// Quantize the float4 this lane holds; lanes 8g..8g+7 form block g.
__device__ __forceinline__ void quant_lane(float4 v, int sub, uint16_t *scale_out,
                                           int *quant_out) {
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 4, 64));
    const float d = amax * (1.0f / 127.0f);
    const float id = d > 0.f ? 1.0f / d : 0.f;
    *quant_out = pack_q(v.x, v.y, v.z, v.w, id);
    if (sub == 0) *scale_out = f32_to_f16_bits(d);
}


}  // namespace sgq
