// Standalone row / elementwise operators of the forward graph, as the
// reference dispatches them (its variants rmsnorm_*, rope_*, geglu,
// add_scaled).  Each is built for f16 activations (the reference's storage:
// read f16, compute in f32 as the shaders do, round the result to f16) and
// for fp32 activations (the model driver's type).  The decode driver fuses
// these into its row kernels instead; these serve the dispatch surface and
// the prefill driver (many rows per launch, latency-bound, one pass over HBM).
#include "sgq_internal.h"

namespace sgq {
namespace {

constexpr int kNormWG = 256;

__device__ __forceinline__ float gelu_tanh_f(float x) {
    const float k = 0.7978845608028654f;  // (2/pi)^0.5
    return 0.5f * x * (1.f + tanhf(k * (x + 0.044715f * x * x * x)));
}

// rmsnorm.wgsl:24-61: one workgroup per row, y = x·rsqrt(mean(x²)+eps)·w
// (or ·(1+w)); fixed-order reduction (deterministic).
template <typename T>
__global__ __launch_bounds__(kNormWG) void rmsnorm_rows_kernel(const T *__restrict__ x,
                                                               const float *__restrict__ w,
                                                               T *__restrict__ y, int row_len,
                                                               int plus_one, float eps) {
    __shared__ float red[kNormWG / kWave];
    const T *xr = x + (size_t)blockIdx.x * row_len;
    T *yr = y + (size_t)blockIdx.x * row_len;
    const int t = threadIdx.x;
    float ss = 0.f;
    for (int i = t; i < row_len; i += kNormWG) {
        const float v = act_ld(xr, i);
        ss += v * v;
    }
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, kWave);
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int i = 0; i < kNormWG / kWave; i++) tot += red[i];
    const float inv = 1.0f / sqrtf(tot / (float)row_len + eps);
    for (int i = t; i < row_len; i += kNormWG) {
        const float wt = w ? (plus_one ? 1.f + w[i] : w[i]) : 1.f;
        act_st(yr, i, act_ld(xr, i) * inv * wt);
    }
}

// rope.wgsl:35-52: NEOX pairing over the whole head (pair i couples dims
// i and i + head_dim/2); only the first rot_dims/2 pairs rotate; table
// cos_sin[token × rot_dims/2] of (cos, sin); rows [token × n_heads × head_dim].
template <typename T>
__global__ __launch_bounds__(256) void rope_kernel(T *__restrict__ xs, const float2 *__restrict__ cs,
                                                   int head_dim, int half_rot, int n_heads,
                                                   uint64_t pairs) {
    const uint64_t g = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (g >= pairs) return;
    const uint64_t row = g / half_rot;
    const int pair = (int)(g % half_rot);
    const uint64_t token = row / n_heads;
    const float2 c = cs[token * half_rot + pair];
    T *base = xs + row * head_dim;
    const float a = act_ld(base, pair), b = act_ld(base, pair + head_dim / 2);
    act_st(base, pair, a * c.x - b * c.y);
    act_st(base, pair + head_dim / 2, b * c.x + a * c.y);
}

// geglu.wgsl:14-24
template <typename T>
__global__ __launch_bounds__(256) void geglu_kernel(const T *__restrict__ g, const T *__restrict__ u,
                                                    T *__restrict__ y, uint64_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) act_st(y, i, gelu_tanh_f(act_ld(g, i)) * act_ld(u, i));
}

// add_scaled.wgsl:21-27
template <typename T>
__global__ __launch_bounds__(256) void add_scaled_kernel(const T *__restrict__ a,
                                                         const T *__restrict__ b,
                                                         T *__restrict__ y, uint64_t n, float s) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) act_st(y, i, (act_ld(a, i) + act_ld(b, i)) * s);
}

uint32_t blocks_for(uint64_t n) { return (uint32_t)((n + 255) / 256); }

template <typename T>
int rmsnorm_t(hipStream_t st, const T *x, const float *w, T *y, uint32_t rows, uint32_t row_len,
              int plus_one, float eps) {
    SGQ_CHECK(rows > 0 && rows < (1u << 31) && row_len > 0, "rmsnorm: %u rows of %u", rows, row_len);
    hipLaunchKernelGGL(rmsnorm_rows_kernel<T>, dim3(rows), dim3(kNormWG), 0, st, x, w, y,
                       (int)row_len, plus_one, eps);
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}

template <typename T>
int rope_t(hipStream_t st, T *xs, const float *cos_sin, uint64_t rows, uint32_t head_dim,
           uint32_t rot_dims, uint32_t n_heads) {
    SGQ_CHECK(head_dim > 0 && head_dim % 2 == 0 && rot_dims % 2 == 0 && rot_dims <= head_dim &&
                  rot_dims > 0 && n_heads > 0,
              "rope: head_dim %u, rot_dims %u, n_heads %u", head_dim, rot_dims, n_heads);
    const uint64_t pairs = rows * (rot_dims / 2);
    if (!pairs) return SGQ_OK;
    SGQ_CHECK(pairs / 256 < (1u << 31), "rope: too many rows");
    hipLaunchKernelGGL(rope_kernel<T>, dim3(blocks_for(pairs)), dim3(256), 0, st, xs,
                       reinterpret_cast<const float2 *>(cos_sin), (int)head_dim,
                       (int)(rot_dims / 2), (int)n_heads, pairs);
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}

template <typename T>
int geglu_t(hipStream_t st, const T *g, const T *u, T *y, uint64_t n) {
    if (!n) return SGQ_OK;
    SGQ_CHECK(n / 256 < (1u << 31), "geglu: n too large");
    hipLaunchKernelGGL(geglu_kernel<T>, dim3(blocks_for(n)), dim3(256), 0, st, g, u, y, n);
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}

template <typename T>
int add_scaled_t(hipStream_t st, const T *a, const T *b, T *y, uint64_t n, float s) {
    if (!n) return SGQ_OK;
    SGQ_CHECK(n / 256 < (1u << 31), "add_scaled: n too large");
    hipLaunchKernelGGL(add_scaled_kernel<T>, dim3(blocks_for(n)), dim3(256), 0, st, a, b, y, n, s);
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}

}  // namespace

int launch_rmsnorm(hipStream_t st, const float *x, const float *w, float *y, uint32_t rows,
                   uint32_t row_len, int plus_one, float eps) {
    return rmsnorm_t(st, x, w, y, rows, row_len, plus_one, eps);
}
int launch_rmsnorm(hipStream_t st, const uint16_t *x, const float *w, uint16_t *y, uint32_t rows,
                   uint32_t row_len, int plus_one, float eps) {
    return rmsnorm_t(st, x, w, y, rows, row_len, plus_one, eps);
}
int launch_rope(hipStream_t st, float *xs, const float *cos_sin, uint64_t rows, uint32_t head_dim,
                uint32_t rot_dims, uint32_t n_heads) {
    return rope_t(st, xs, cos_sin, rows, head_dim, rot_dims, n_heads);
}
int launch_rope(hipStream_t st, uint16_t *xs, const float *cos_sin, uint64_t rows,
                uint32_t head_dim, uint32_t rot_dims, uint32_t n_heads) {
    return rope_t(st, xs, cos_sin, rows, head_dim, rot_dims, n_heads);
}
int launch_geglu(hipStream_t st, const float *g, const float *u, float *y, uint64_t n) {
    return geglu_t(st, g, u, y, n);
}
int launch_geglu(hipStream_t st, const uint16_t *g, const uint16_t *u, uint16_t *y, uint64_t n) {
    return geglu_t(st, g, u, y, n);
}
int launch_add_scaled(hipStream_t st, const float *a, const float *b, float *y, uint64_t n,
                      float s) {
    return add_scaled_t(st, a, b, y, n, s);
}
int launch_add_scaled(hipStream_t st, const uint16_t *a, const uint16_t *b, uint16_t *y,
                      uint64_t n, float s) {
    return add_scaled_t(st, a, b, y, n, s);
}

}  // namespace sgq
