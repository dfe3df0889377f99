// Measurement probes for the roofline denominators (bench.py only; not part
// of the compute path).  Built into libsgq_probe.so.
//
//  * sgqp_mfma: int8 matrix-core throughput with no memory traffic.
//      mode 0  v_mfma_i32_32x32x32_i8 only, four independent accumulator
//              chains per wave (the dense int8 peak the hardware delivers);
//      mode 1  per int8 MFMA (fresh accumulator, as an exact per-32-block
//              MMQ issues it) also 16 v_cvt_f32_i32 + 16 FMA of its result
//              into fp32 accumulators: the ceiling of any kernel that
//              rescales every block's exact i32 dot on the VALU;
//      mode 2  mode 1 plus the v_mfma_f32_32x32x8_f16 that forms the
//              block's d_a x d_w scale outer product (the MMQ's structure);
//      mode 3  the block dot on the f16 matrix cores (exact), the scale
//              MFMA and one FMA per output element, software-pipelined.
//    Ops counted: 2*32*32*32 per int8 MFMA.
//  * sgqp_hbm_read: a streaming read of a large buffer (64 KB chunks per
//    workgroup, 16-byte nontemporal loads), summed so that nothing is
//    elided: the achievable HBM read rate next to the 8 TB/s vendor figure.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// mode 3: the block dot on the f16 matrix cores (int8 and q-8 values are
// exact f16 integers, a 32-term dot is exact in the f32 accumulator: two
// v_mfma_f32_32x32x16_f16 per block), the scale MFMA, and one FMA per output
// element; the MFMAs of block b+1 are issued before block b's FMAs.
__global__ __launch_bounds__(256) void mfma_f16dot_probe_kernel(int iters, int *__restrict__ out) {
    const int t = threadIdx.x;
    const h8 a0 = __builtin_bit_cast(h8, v4i{0x3c003c00 + t, 0x40004000, 0x3c00bc00, t});
    const h8 a1 = __builtin_bit_cast(h8, v4i{0x3c00 + t, 0x4000, 0xbc00, t * 3});
    const h8 sa = __builtin_bit_cast(h8, v4i{0x3c00 + (t & 7), 0, 0, 0});
    const h8 sb = __builtin_bit_cast(h8, v4i{0x3800 + (t & 3), 0, 0, 0});
    const f32x16 fzero = {};
    f32x16 acc0 = {}, acc1 = {};
    f32x16 d0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, a1, fzero, 0, 0, 0);
    d0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, a0, d0, 0, 0, 0);
    f32x16 s0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(sa, sb, fzero, 0, 0, 0);
    for (int i = 0; i < iters; i++) {
        f32x16 d1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, a0, fzero, 0, 0, 0);
        d1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, a1, d1, 0, 0, 0);
        const f32x16 s1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(sb, sa, fzero, 0, 0, 0);
#pragma unroll
        for (int q = 0; q < 16; q++) acc0[q] = __builtin_fmaf(d0[q], s0[q], acc0[q]);
        d0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, a1, fzero, 0, 0, 0);
        d0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, a0, d0, 0, 0, 0);
        s0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(sa, sb, fzero, 0, 0, 0);
#pragma unroll
        for (int q = 0; q < 16; q++) acc1[q] = __builtin_fmaf(d1[q], s1[q], acc1[q]);
    }
    float s = 0.f;
#pragma unroll
    for (int q = 0; q < 16; q++) s += acc0[q] + acc1[q];
    out[blockIdx.x * blockDim.x + t] = __float_as_int(s);
}

template <int MODE>
__global__ __launch_bounds__(256) void mfma_probe_kernel(int iters, int *__restrict__ out) {
    const int t = threadIdx.x;
    const v4i a = {t, t * 3 + 1, t ^ 0x5a5a, 7};
    const v4i b = {t * 5, 11, t + 2, t ^ 0x3c3c};
    if (MODE == 0) {
        v16i c0 = {}, c1 = {}, c2 = {}, c3 = {};
        for (int i = 0; i < iters; i++) {
            c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(b, a, c1, 0, 0, 0);
            c2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, a, c2, 0, 0, 0);
            c3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(b, b, c3, 0, 0, 0);
        }
        int s = 0;
#pragma unroll
        for (int q = 0; q < 16; q++) s += c0[q] ^ c1[q] ^ c2[q] ^ c3[q];
        out[blockIdx.x * blockDim.x + t] = s;
    } else {
        const v16i zero = {};
        const f32x16 fzero = {};
        const h4 sa = __builtin_bit_cast(h4, v2i{0x3c00 + (t & 7), 0});
        const h4 sb = __builtin_bit_cast(h4, v2i{0x3800 + (t & 3), 0});
        f32x16 acc0 = {}, acc1 = {};
        f32x16 sc0, sc1;
#pragma unroll
        for (int q = 0; q < 16; q++) {
            sc0[q] = 1.0f / (q + 1);
            sc1[q] = 0.5f / (q + 2);
        }
        for (int i = 0; i < iters; i++) {
            // two block tiles per iteration: each MFMA's result is rescaled
            // while the other one runs, as in the MMQ's software pipeline
            const v16i d0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, zero, 0, 0, 0);
            if (MODE == 2) sc0 = __builtin_amdgcn_mfma_f32_32x32x8f16(sa, sb, fzero, 0, 0, 0);
            const v16i d1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(b, a, zero, 0, 0, 0);
            if (MODE == 2) sc1 = __builtin_amdgcn_mfma_f32_32x32x8f16(sb, sa, fzero, 0, 0, 0);
#pragma unroll
            for (int q = 0; q < 16; q++) acc0[q] = __builtin_fmaf((float)d0[q], sc0[q], acc0[q]);
#pragma unroll
            for (int q = 0; q < 16; q++) acc1[q] = __builtin_fmaf((float)d1[q], sc1[q], acc1[q]);
        }
        float s = 0.f;
#pragma unroll
        for (int q = 0; q < 16; q++) s += acc0[q] + acc1[q];
        out[blockIdx.x * blockDim.x + t] = __float_as_int(s);
    }
}

// Each workgroup streams contiguous 64 KB chunks (grid-stride over chunks)
// with 16-byte nontemporal loads, four in flight per thread: of the
// patterns swept on the box (grid-stride, 16/64/256 KB chunks, LDS DMA
// rings, with and without the nt bit, 512..4096 workgroups) the fastest,
// 7.1 TB/s at 1024 workgroups against 5.4-6.4 without nt.
__global__ __launch_bounds__(256) void hbm_read_kernel(const float4 *__restrict__ p, uint64_t n4,
                                                       float *__restrict__ out) {
    constexpr uint64_t kChunk4 = 65536 / 16;
    typedef float f4v __attribute__((ext_vector_type(4)));
    const f4v *pv = reinterpret_cast<const f4v *>(p);
    f4v s = {0.f, 0.f, 0.f, 0.f};
    const uint64_t nch = n4 / kChunk4;
    for (uint64_t c = blockIdx.x; c < nch; c += gridDim.x) {
        const f4v *q = pv + c * kChunk4;
        for (uint64_t i = threadIdx.x; i < kChunk4; i += 4 * 256) {
            const f4v a = __builtin_nontemporal_load(q + i), b = __builtin_nontemporal_load(q + i + 256),
                      c2 = __builtin_nontemporal_load(q + i + 512),
                      d = __builtin_nontemporal_load(q + i + 768);
            s += (a + b) + (c2 + d);
        }
    }
    for (uint64_t i = nch * kChunk4 + (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n4;
         i += (uint64_t)gridDim.x * 256)
        s += pv[i];
    out[blockIdx.x * blockDim.x + threadIdx.x] = s.x + s.y + s.z + s.w;
}

}  // namespace

extern "C" {

// blocks x 256 threads; out: blocks*256 ints.  Returns a hipError_t value.
int sgqp_mfma(void *stream, int mode, int blocks, int iters, int *out) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (blocks <= 0 || iters <= 0 || !out) return (int)hipErrorInvalidValue;
    if (mode == 0)
        hipLaunchKernelGGL(mfma_probe_kernel<0>, dim3(blocks), dim3(256), 0, st, iters, out);
    else if (mode == 1)
        hipLaunchKernelGGL(mfma_probe_kernel<1>, dim3(blocks), dim3(256), 0, st, iters, out);
    else if (mode == 2)
        hipLaunchKernelGGL(mfma_probe_kernel<2>, dim3(blocks), dim3(256), 0, st, iters, out);
    else if (mode == 3)
        hipLaunchKernelGGL(mfma_f16dot_probe_kernel, dim3(blocks), dim3(256), 0, st, iters, out);
    else
        return (int)hipErrorInvalidValue;
    return (int)hipGetLastError();
}

// Int8 MFMAs one launch of sgqp_mfma issues (for the ops count).
long long sgqp_mfma_count(int mode, int blocks, int iters) {
    const long long waves = (long long)blocks * 4;
    return waves * iters * (mode == 0 ? 4 : 2);  // mode 3: 2 blocks of 32x32x32 per iteration
}

// Reads `bytes` (a multiple of 16, 16-byte aligned) from `buf`; out:
// blocks*256 floats.
int sgqp_hbm_read(void *stream, const void *buf, uint64_t bytes, int blocks, float *out) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (!buf || !out || blocks <= 0 || (bytes & 15) || ((uintptr_t)buf & 15))
        return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(hbm_read_kernel, dim3(blocks), dim3(256), 0, st,
                       static_cast<const float4 *>(buf), bytes / 16, out);
    return (int)hipGetLastError();
}

}  // extern "C"
