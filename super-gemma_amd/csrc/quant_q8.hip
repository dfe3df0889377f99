// Q8_0 quantization / dequantization / KV append for gfx950.
//
// Semantics: kv_quant_q8 (crates/sg-gpu/shaders/kv_quant_q8.wgsl:30-57) and
// kv_append_global_q8 (kv_append_global_q8.wgsl:29-60): per 32-element
// block, amax in f32, d = amax * (1/127) (a multiply, so the f16 scale is
// bit-exact), id = d > 0 ? 1/d : 0 from the unrounded d, scale = f16(d)
// round-to-nearest-even, q = round_ties_even(x * id) as int8.  Unlike the
// reference GPU (a 2.5-ulp reciprocal), 1/d here is the IEEE-correct
// division hipcc emits by default, so the quants match the CPU oracle
// bit for bit as well, not just within ±1.
//
// Layout: structure of arrays (the reference's page format): scales f16
// [n/32], quants int8 [n] (4 per 32-bit word, element order).
//
// HBM-bound streaming op.  Eight lanes share a block, each holding one
// float4: a wave reads 1 KB contiguous per load and writes 256 B of quants
// per store (one dword per lane); amax is a 3-step butterfly inside each
// 8-lane group.
#include "q8.h"

namespace sgq {
namespace {

constexpr int kQWG = 256;
typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned u2 __attribute__((ext_vector_type(2)));

// Elements 4i..4i+3 of a streamed source (read once: nontemporal).
__device__ __forceinline__ float4 ld4_stream(const float *x, uint64_t i) {
    const f4 t = __builtin_nontemporal_load(reinterpret_cast<const f4 *>(x) + i);
    return make_float4(t.x, t.y, t.z, t.w);
}
__device__ __forceinline__ float4 ld4_stream(const uint16_t *x, uint64_t i) {
    const u2 t = __builtin_nontemporal_load(reinterpret_cast<const u2 *>(x) + i);
    return make_float4(f16_bits_to_f32(t.x & 0xffffu), f16_bits_to_f32(t.x >> 16),
                       f16_bits_to_f32(t.y & 0xffffu), f16_bits_to_f32(t.y >> 16));
}

template <typename T>
__global__ __launch_bounds__(kQWG) void quant_q8_0_kernel(const T *__restrict__ x,
                                                          uint16_t *__restrict__ scales,
                                                          int *__restrict__ quants,
                                                          uint64_t n4) {
    for (uint64_t i = (uint64_t)blockIdx.x * kQWG + threadIdx.x; i < n4;
         i += (uint64_t)gridDim.x * kQWG) {
        float4 v = ld4_stream(x, i);
        int q;
        quant_lane(v, (int)(i & 7), &scales[i >> 3], &q);
        quants[i] = q;
    }
}

template <typename T>
__global__ __launch_bounds__(kQWG) void dequant_q8_0_kernel(const uint16_t *__restrict__ scales,
                                                            const int *__restrict__ quants,
                                                            T *__restrict__ out, uint64_t n4) {
    for (uint64_t i = (uint64_t)blockIdx.x * kQWG + threadIdx.x; i < n4;
         i += (uint64_t)gridDim.x * kQWG) {
        const float d = f16_bits_to_f32(scales[i >> 3]);
        const int q = quants[i];
        float4 v;
        v.x = d * (float)(int8_t)(q & 0xff);
        v.y = d * (float)(int8_t)((q >> 8) & 0xff);
        v.z = d * (float)(int8_t)((q >> 16) & 0xff);
        v.w = d * (float)(int8_t)((q >> 24) & 0xff);
        act_st(out, 4 * i, v.x);
        act_st(out, 4 * i + 1, v.y);
        act_st(out, 4 * i + 2, v.z);
        act_st(out, 4 * i + 3, v.w);
    }
}

// kv_append_*_q8: token t of `src` ([n_tokens × row_len], f16 or fp32) is
// quantized into slot (step[0] + t), or (step[0] + t) % ring when ring > 0.
template <typename T>
__global__ __launch_bounds__(kQWG) void kv_append_q8_kernel(const T *__restrict__ src,
                                                            uint16_t *__restrict__ scales,
                                                            int *__restrict__ quants,
                                                            const uint32_t *__restrict__ step,
                                                            uint64_t n4, uint32_t row4,
                                                            uint32_t ring) {
    const uint32_t pos = step[0];
    for (uint64_t i = (uint64_t)blockIdx.x * kQWG + threadIdx.x; i < n4;
         i += (uint64_t)gridDim.x * kQWG) {
        const uint64_t t = i / row4;
        const uint64_t c = i - t * row4;
        uint64_t slot = pos + t;
        if (ring) slot %= ring;
        const uint64_t o = slot * row4 + c;
        float4 v = act_ld4(src, i);
        int q;
        quant_lane(v, (int)(i & 7), &scales[o >> 3], &q);
        quants[o] = q;
    }
}

// Key-blocked V append (kv_append_global_v_q8.wgsl:32-75): thread (key
// block tb, column c) quantizes column c over the block's live rows with the
// kv_quant_q8 rule and writes scale (pos/32 + tb, c) and the block's quants
// at rows pos + t.  Neighbouring threads take neighbouring columns, so every
// load and store is coalesced across the wave.
template <typename T>
__global__ __launch_bounds__(kQWG) void kv_append_v_q8_kernel(const T *__restrict__ src,
                                                              uint16_t *__restrict__ scales,
                                                              int8_t *__restrict__ quants,
                                                              const uint32_t *__restrict__ step,
                                                              uint32_t pos_direct,
                                                              uint32_t n_tok, uint32_t row) {
    const uint32_t pos = step ? step[0] : pos_direct;
    const uint64_t n_items = (uint64_t)((n_tok + 31) / 32) * row;
    for (uint64_t i = (uint64_t)blockIdx.x * kQWG + threadIdx.x; i < n_items;
         i += (uint64_t)gridDim.x * kQWG) {
        const uint32_t tb = (uint32_t)(i / row), c = (uint32_t)(i % row);
        const uint32_t k0 = 32 * tb, k1 = min(k0 + 32u, n_tok);
        float amax = 0.f;
        for (uint32_t t = k0; t < k1; t++) amax = fmaxf(amax, fabsf(act_ld(src, (size_t)t * row + c)));
        const float d = amax * (1.0f / 127.0f);
        const float id = d > 0.f ? 1.0f / d : 0.f;
        scales[(size_t)(pos / 32 + tb) * row + c] = f32_to_f16_bits(d);
        for (uint32_t t = k0; t < k1; t++)
            quants[(size_t)(pos + t) * row + c] =
                (int8_t)(int)__builtin_rintf(act_ld(src, (size_t)t * row + c) * id);
    }
}

int grid_for(uint64_t n4) {
    uint64_t g = (n4 + kQWG - 1) / kQWG;
    const uint64_t cap = (uint64_t)device_info().cus * 8;
    return (int)(g < cap ? (g ? g : 1) : cap);
}

}  // namespace

namespace {
template <typename T>
int quant_t(hipStream_t st, const T *x, uint16_t *scales, int8_t *quants, uint64_t n) {
    SGQ_CHECK(n % 32 == 0, "quant_q8_0: n=%llu must be a multiple of 32", (unsigned long long)n);
    SGQ_CHECK(((uintptr_t)x & (4 * sizeof(T) - 1)) == 0 && ((uintptr_t)quants & 3) == 0 &&
                  ((uintptr_t)scales & 1) == 0,
              "quant_q8_0: misaligned buffers");
    if (n == 0) return SGQ_OK;
    const uint64_t n4 = n / 4;
    hipLaunchKernelGGL(quant_q8_0_kernel<T>, dim3(grid_for(n4)), dim3(kQWG), 0, st, x, scales,
                       reinterpret_cast<int *>(quants), n4);
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}

template <typename T>
int dequant_t(hipStream_t st, const uint16_t *scales, const int8_t *quants, T *out, uint64_t n) {
    SGQ_CHECK(n % 32 == 0, "dequant_q8_0: n must be a multiple of 32");
    SGQ_CHECK(((uintptr_t)out & (sizeof(T) - 1)) == 0 && ((uintptr_t)quants & 3) == 0,
              "dequant_q8_0: misaligned buffers");
    if (n == 0) return SGQ_OK;
    const uint64_t n4 = n / 4;
    hipLaunchKernelGGL(dequant_q8_0_kernel<T>, dim3(grid_for(n4)), dim3(kQWG), 0, st, scales,
                       reinterpret_cast<const int *>(quants), out, n4);
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}

template <typename T>
int append_t(hipStream_t st, const T *src, uint16_t *scales, int8_t *quants, const uint32_t *step,
             uint32_t n_tokens, uint32_t row_len, uint32_t ring) {
    SGQ_CHECK(row_len % 32 == 0 && row_len > 0, "kv_append_q8: row_len must be a multiple of 32");
    SGQ_CHECK(((uintptr_t)src & (4 * sizeof(T) - 1)) == 0 && ((uintptr_t)quants & 3) == 0,
              "kv_append_q8: misaligned buffers");
    if (n_tokens == 0) return SGQ_OK;
    const uint64_t n4 = (uint64_t)n_tokens * row_len / 4;
    hipLaunchKernelGGL(kv_append_q8_kernel<T>, dim3(grid_for(n4)), dim3(kQWG), 0, st, src, scales,
                       reinterpret_cast<int *>(quants), step, n4, row_len / 4, ring);
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}

template <typename T>
int append_v_t(hipStream_t st, const T *src, uint16_t *scales, int8_t *quants, const uint32_t *step,
               uint32_t pos, uint32_t n_tokens, uint32_t row_len) {
    SGQ_CHECK(row_len > 0, "kv_append_v_q8: empty row");
    SGQ_CHECK(step != nullptr || pos % 32 == 0,
              "kv_append_v_q8: pos %u must be a multiple of 32 (32-key blocks)", pos);
    if (n_tokens == 0) return SGQ_OK;
    const uint64_t items = (uint64_t)((n_tokens + 31) / 32) * row_len;
    hipLaunchKernelGGL(kv_append_v_q8_kernel<T>, dim3(grid_for(items)), dim3(kQWG), 0, st, src,
                       scales, quants, step, pos, n_tokens, row_len);
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}
}  // namespace

int launch_quant_q8_0(hipStream_t st, const float *x, uint16_t *scales, int8_t *quants,
                      uint64_t n) {
    return quant_t(st, x, scales, quants, n);
}
int launch_quant_q8_0(hipStream_t st, const uint16_t *x, uint16_t *scales, int8_t *quants,
                      uint64_t n) {
    return quant_t(st, x, scales, quants, n);
}
int launch_dequant_q8_0(hipStream_t st, const uint16_t *scales, const int8_t *quants, float *out,
                        uint64_t n) {
    return dequant_t(st, scales, quants, out, n);
}
int launch_dequant_q8_0(hipStream_t st, const uint16_t *scales, const int8_t *quants,
                        uint16_t *out, uint64_t n) {
    return dequant_t(st, scales, quants, out, n);
}
int launch_kv_append_q8(hipStream_t st, const float *src, uint16_t *scales, int8_t *quants,
                        const uint32_t *step, uint32_t n_tokens, uint32_t row_len, uint32_t ring) {
    return append_t(st, src, scales, quants, step, n_tokens, row_len, ring);
}
int launch_kv_append_q8(hipStream_t st, const uint16_t *src, uint16_t *scales, int8_t *quants,
                        const uint32_t *step, uint32_t n_tokens, uint32_t row_len, uint32_t ring) {
    return append_t(st, src, scales, quants, step, n_tokens, row_len, ring);
}
int launch_kv_append_v_q8(hipStream_t st, const float *src, uint16_t *scales, int8_t *quants,
                          const uint32_t *step, uint32_t pos, uint32_t n_tokens, uint32_t row_len) {
    return append_v_t(st, src, scales, quants, step, pos, n_tokens, row_len);
}
int launch_kv_append_v_q8(hipStream_t st, const uint16_t *src, uint16_t *scales, int8_t *quants,
                          const uint32_t *step, uint32_t pos, uint32_t n_tokens, uint32_t row_len) {
    return append_v_t(st, src, scales, quants, step, pos, n_tokens, row_len);
}

}  // namespace sgq
