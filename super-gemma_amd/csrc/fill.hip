// Synthetic inputs generated on the device (benches and tests; not part of
// the hot path).  Counter-based: element i's value depends only on
// (seed, i), so any sub-range can be regenerated and the output does not
// depend on the launch geometry.
//
//  * Q4_0 weights: d = f16(|N(0, sigma)|), 16 uniform nibble bytes — the
//    weight distribution of the benchmark configurations.
//  * fp32 N(mean, sigma) activations.
// Normals come from Box–Muller on two 24-bit uniforms drawn from splitmix64.
#include "sgq_internal.h"

namespace sgq {
namespace {

__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ float normal_from(uint64_t h) {
    // u1 in (0, 1], u2 in [0, 1)
    const float u1 = ((float)((h >> 40) & 0xFFFFFF) + 1.0f) * (1.0f / 16777216.0f);
    const float u2 = (float)((h >> 8) & 0xFFFFFF) * (1.0f / 16777216.0f);
    return sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2);
}

__global__ void fill_q4_0_kernel(uint8_t *__restrict__ w, uint64_t n_blocks, uint64_t seed,
                                 float sigma) {
    for (uint64_t b = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; b < n_blocks;
         b += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t h0 = splitmix64(seed ^ (b * 3 + 0) * 0xD1B54A32D192ED03ull);
        const uint64_t h1 = splitmix64(seed ^ (b * 3 + 1) * 0xD1B54A32D192ED03ull);
        const uint64_t h2 = splitmix64(seed ^ (b * 3 + 2) * 0xD1B54A32D192ED03ull);
        const uint16_t d = f32_to_f16_bits(fabsf(normal_from(h0)) * sigma);
        uint8_t *blk = w + b * 18;
        // 2-byte aligned block: write as 9 halfwords.
        uint16_t *h = reinterpret_cast<uint16_t *>(blk);
        h[0] = d;
#pragma unroll
        for (int j = 0; j < 4; j++) h[1 + j] = (uint16_t)(h1 >> (16 * j));
#pragma unroll
        for (int j = 0; j < 4; j++) h[5 + j] = (uint16_t)(h2 >> (16 * j));
    }
}

__global__ void fill_normal_kernel(float *__restrict__ x, uint64_t n, uint64_t seed, float mean,
                                   float sigma) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t h = splitmix64(seed ^ (i * 0x9E6C63D0676A9A99ull));
        x[i] = mean + sigma * normal_from(h);
    }
}

// Q6_K rows at a byte stride (q6_k.rs:25-62 block layout: ql[128], qh[64],
// int8 sub-scales[16], f16 d; parity_logits.rs:31-51's distribution: random
// quant bytes, sub-scales in [-8, 7], d = f16(N(0,1)·1e-3)); row padding
// zeroed.  Thread per (row, block).
__global__ void fill_q6k_kernel(uint8_t *__restrict__ w, uint64_t n_rows, int nb,
                                uint64_t row_stride, uint64_t seed) {
    const uint64_t n_items = n_rows * (uint64_t)nb;
    for (uint64_t it = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; it < n_items;
         it += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t r = it / nb;
        const int b = (int)(it % nb);
        uint8_t *blk = w + r * row_stride + (uint64_t)b * 210;
        for (int j = 0; j < 208; j += 8) {
            const uint64_t h = splitmix64(seed ^ ((it * 27 + j / 8) * 0xD1B54A32D192ED03ull));
            for (int e = 0; e < 8 && j + e < 208; e++) {
                const uint8_t byte = (uint8_t)(h >> (8 * e));
                blk[j + e] = j + e >= 192 ? (uint8_t)(int8_t)((int)(byte & 15) - 8) : byte;
            }
        }
        const uint16_t d = f32_to_f16_bits(
            normal_from(splitmix64(seed ^ ((it * 27 + 26) * 0xD1B54A32D192ED03ull))) * 1e-3f);
        blk[208] = (uint8_t)(d & 0xff);
        blk[209] = (uint8_t)(d >> 8);
        if (b == nb - 1)
            for (uint64_t p = (uint64_t)nb * 210; p < row_stride; p++) w[r * row_stride + p] = 0;
    }
}

int fill_grid(uint64_t n) {
    uint64_t g = (n + 255) / 256;
    const uint64_t cap = (uint64_t)device_info().cus * 16;
    return (int)(g < cap ? (g ? g : 1) : cap);
}

}  // namespace

int launch_fill_q4_0(hipStream_t st, void *w, uint64_t n_blocks, uint64_t seed, float sigma) {
    SGQ_CHECK(((uintptr_t)w & 1) == 0, "fill_q4_0: weights must be 2-byte aligned");
    if (n_blocks == 0) return SGQ_OK;
    hipLaunchKernelGGL(fill_q4_0_kernel, dim3(fill_grid(n_blocks)), dim3(256), 0, st,
                       static_cast<uint8_t *>(w), n_blocks, seed, sigma);
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}

int launch_fill_normal(hipStream_t st, float *x, uint64_t n, uint64_t seed, float mean,
                       float sigma) {
    if (n == 0) return SGQ_OK;
    hipLaunchKernelGGL(fill_normal_kernel, dim3(fill_grid(n)), dim3(256), 0, st, x, n, seed, mean,
                       sigma);
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}

int launch_fill_q6k(hipStream_t st, void *w, uint64_t n_rows, uint32_t k, uint64_t row_stride,
                    uint64_t seed) {
    SGQ_CHECK(k % 256 == 0 && row_stride >= (uint64_t)(k / 256) * 210,
              "fill_q6k: k %u, row stride %llu", k, (unsigned long long)row_stride);
    const uint64_t items = n_rows * (k / 256);
    if (items == 0) return SGQ_OK;
    hipLaunchKernelGGL(fill_q6k_kernel, dim3(fill_grid(items)), dim3(256), 0, st,
                       static_cast<uint8_t *>(w), n_rows, (int)(k / 256), row_stride, seed);
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}

}  // namespace sgq
