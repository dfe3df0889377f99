// Q6_K LM-head GEMV with fused logit softcap for gfx950:
//     y[n] = softcap·tanh((E[n×k]·x[k]) / softcap)      (softcap <= 0: the dot)
// Semantics of gemv_q6_k_logits (crates/sg-gpu/shaders/gemv_q6_k_logits.wgsl:
// 41-104): E is the tied Q6_K token-embedding matrix, rows of k/256 GGUF
// super-blocks (210 B: ql[128] low nibbles, qh[64] 2-bit highs, int8
// scales[16], f16 d; q6_k.rs:41-62) at a padded byte stride; x is f16
// (here: fp32 in, rounded to f16 once per workgroup, as the reference
// feeds f16 activations); per row an f32 dot, then the softcap.
//
// Design (HBM-bound: 4416 B per row at k = 5376, 1.16 GB for the 262144-row
// vocabulary):
//  * One wave per two rows at a time.  Rows are staged through registers
//    into the wave's two LDS slots (16-byte chunks, coalesced); the wave's
//    next two rows are in flight while two are computed.
//  * Lane task (super-block sb, half h, lane-half j) covers 64 weights: the
//    four 16-weight sub-blocks g = 0..3 that share ql bytes
//    [64h + 16j, +16) / [64h + 32 + 16j, +16) and qh bytes [32h + 16j, +16).
//    Four weights at a time: their 6-bit quants q (nibble | 2 bits << 4)
//    are one dword of bytes; a byte permute against 0x64 makes the f16
//    pairs 1024 + q, and a packed f16 add of -1056 gives q - 32 exactly.
//    v_dot2_f32_f16 takes them against the f16 x pairs into an f32
//    sub-block sum, scaled by d·scale[sub-block] (exact: f16 × int8).
//  * Lane sums are reduced over the wave in a fixed DPP order, so results
//    are bit-reproducible.
#include "ring.h"

namespace sgq {
namespace {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));

constexpr int kQ6WG = 256;               // 4 waves
constexpr int kQ6Waves = kQ6WG / kWave;
constexpr int kQ6BlockBytes = 210;
constexpr int kQ6MaxBlocks = 24;         // k <= 6144: at most 2 tasks per lane
constexpr int kQ6Chunks = 5;             // 16-byte chunks per lane and row (<= 5120 B)

__device__ __forceinline__ uint32_t lds_u32(const uint8_t *p) {
    return *reinterpret_cast<const uint32_t *>(p);
}

// 16 bytes starting at byte offset `off` (even) of an LDS row, as 4 words.
__device__ __forceinline__ void lds_16(const uint8_t *row, int off, uint32_t (&w)[4]) {
    const int mis = off & 3;
    const uint8_t *a = row + (off - mis);
    uint32_t r[5];
#pragma unroll
    for (int i = 0; i < 5; i++) r[i] = lds_u32(a + 4 * i);
#pragma unroll
    for (int i = 0; i < 4; i++) w[i] = __builtin_amdgcn_alignbyte(r[i + 1], r[i], mis);
}

// Sum over a task's four sub-blocks (64 weights); xr: f16 x of the task,
// 16 halves per sub-block g at xr + 32g·2 bytes.
__device__ __forceinline__ float q6_task(const uint8_t *row, const _Float16 *xh, int sb, int h,
                                         int j) {
    const int base = sb * kQ6BlockBytes;
    uint32_t ql0[4], ql1[4], qh[4];
    lds_16(row, base + 64 * h + 16 * j, ql0);
    lds_16(row, base + 64 * h + 32 + 16 * j, ql1);
    lds_16(row, base + 128 + 32 * h + 16 * j, qh);
    // scales 8h + j + 2g (g = 0..3): bytes j, j+2, j+4, j+6 of the 8 at 192 + 8h
    uint32_t sw[2];
    {
        const int off = base + 192 + 8 * h, mis = off & 3;
        const uint8_t *a = row + (off - mis);
        const uint32_t r0 = lds_u32(a), r1 = lds_u32(a + 4), r2 = lds_u32(a + 8);
        sw[0] = __builtin_amdgcn_alignbyte(r1, r0, mis);
        sw[1] = __builtin_amdgcn_alignbyte(r2, r1, mis);
    }
    const int doff = base + 208;
    const uint32_t dw = lds_u32(row + (doff & ~3));
    const float d = f16_bits_to_f32((doff & 2) ? dw >> 16 : dw & 0xffffu);
    const h2_t bias = {(_Float16)-1056.0f, (_Float16)-1056.0f};
    const _Float16 *xt = xh + sb * 256 + 128 * h + 16 * j;
    float acc = 0.f;
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const int sbyte = j + 2 * g;
        const float sc = (float)(int8_t)((sw[sbyte >> 2] >> (8 * (sbyte & 3))) & 0xffu);
        const uint32_t *ql = (g & 1) ? ql1 : ql0;
        const i32x4_t x0 = *reinterpret_cast<const i32x4_t *>(xt + 32 * g);      // halves 0..7
        const i32x4_t x1 = *reinterpret_cast<const i32x4_t *>(xt + 32 * g + 8);  // halves 8..15
        float sub = 0.f;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const uint32_t lo = (g >= 2 ? ql[w] >> 4 : ql[w]) & 0x0F0F0F0Fu;
            const uint32_t q4 = lo | (((qh[w] >> (2 * g)) & 0x03030303u) << 4);
            const h2_t p0 = __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(0x64646464u, q4, 0x04010400u)) + bias;
            const h2_t p1 = __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(0x64646464u, q4, 0x04030402u)) + bias;
            const int xa = w < 2 ? x0[2 * w] : x1[2 * (w - 2)];
            const int xb = w < 2 ? x0[2 * w + 1] : x1[2 * (w - 2) + 1];
            sub = __builtin_amdgcn_fdot2(p0, __builtin_bit_cast(h2_t, xa), sub, false);
            sub = __builtin_amdgcn_fdot2(p1, __builtin_bit_cast(h2_t, xb), sub, false);
        }
        acc = __builtin_fmaf(d * sc, sub, acc);
    }
    return acc;
}

__device__ __forceinline__ _Float16 to_half(float v) { return (_Float16)v; }
__device__ __forceinline__ _Float16 to_half(uint16_t bits) {
    return __builtin_bit_cast(_Float16, bits);
}

template <typename TX>
__global__ __launch_bounds__(kQ6WG) void gemv_q6_k_kernel(const uint8_t *__restrict__ W,
                                                          uint32_t stride,
                                                          const TX *__restrict__ x,
                                                          float *__restrict__ y, int n, int k,
                                                          float softcap) {
    extern __shared__ __align__(16) uint8_t q6_smem[];
    _Float16 *xh = reinterpret_cast<_Float16 *>(q6_smem);  // k halves
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    // two row slots per wave, each padded by 16 B: the scale reads of a
    // row's last block may run 2 B past it
    uint8_t *row0 = q6_smem + ((k * 2 + 15) & ~15) + wave * 2 * (stride + 16);
    uint8_t *row1 = row0 + (stride + 16);
    const int nb = k / 256, ntask = 4 * nb, nchunks = (int)(stride / 16);
    const int G = gridDim.x * kQ6Waves;
    int r = blockIdx.x * kQ6Waves + wave;

    // a wave computes rows r and r + G together (2·4·nb tasks over its 64
    // lanes: 168 at k = 5376, so lanes stay busy where one row's 84 tasks
    // would leave 44 of them idle in the second round), while the next two
    // pairs of rows are in flight: register sets (pa, pb) and (pc, pd) take
    // turns, each refilled two iterations ahead as soon as it is in LDS
    i32x4_t pa[kQ6Chunks], pb[kQ6Chunks], pc[kQ6Chunks], pd[kQ6Chunks];
    auto load = [&](i32x4_t (&pre)[kQ6Chunks], int rr) {
        if (rr >= n) return;
        const i32x4_t *src = reinterpret_cast<const i32x4_t *>(W + (size_t)rr * stride);
#pragma unroll
        for (int c = 0; c < kQ6Chunks; c++) {
            const int idx = lane + kWave * c;
            if (idx < nchunks) pre[c] = __builtin_nontemporal_load(src + idx);
        }
    };
    auto put = [&](const i32x4_t (&pre)[kQ6Chunks], uint8_t *row) {
#pragma unroll
        for (int c = 0; c < kQ6Chunks; c++) {
            const int idx = lane + kWave * c;
            if (idx < nchunks) *reinterpret_cast<i32x4_t *>(row + 16 * idx) = pre[c];
        }
    };
    // rows rr and rr + G from (A, B); A and B then load rows rr + 4G, rr + 5G
    auto step = [&](i32x4_t (&A)[kQ6Chunks], i32x4_t (&B)[kQ6Chunks], int rr)
        __attribute__((always_inline)) {
        const int r1 = rr + G;
        const bool has1 = r1 < n;
        put(A, row0);
        if (has1) put(B, row1);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        load(A, rr + 4 * G);  // land while the next pairs compute
        load(B, r1 + 4 * G);
        float acc0 = 0.f, acc1 = 0.f;
        const int nt = has1 ? 2 * ntask : ntask;
        for (int t = lane; t < nt; t += kWave) {
            const bool second = t >= ntask;
            const int u = second ? t - ntask : t;
            const float v = q6_task(second ? row1 : row0, xh, u >> 2, (u >> 1) & 1, u & 1);
            if (second) acc1 += v;
            else acc0 += v;
        }
        acc0 = wave_sum_dpp(acc0);
        acc1 = wave_sum_dpp(acc1);
        if (lane == 0) {
            y[rr] = softcap > 0.f ? softcap * tanhf(acc0 / softcap) : acc0;
            if (has1) y[r1] = softcap > 0.f ? softcap * tanhf(acc1 / softcap) : acc1;
        }
        __builtin_amdgcn_wave_barrier();  // these rows' LDS reads before the next rows' stores
    };
    load(pa, r);
    load(pb, r + G);
    load(pc, r + 2 * G);
    load(pd, r + 3 * G);
    for (int i = threadIdx.x; i < k; i += kQ6WG) xh[i] = to_half(x[i]);
    __syncthreads();

    for (; r < n; r += 4 * G) {
        step(pa, pb, r);
        if (r + 2 * G >= n) break;
        step(pc, pd, r + 2 * G);
    }
}

}  // namespace

namespace {
template <typename TX>
int gemv_q6_k_t(hipStream_t st, const void *w, size_t row_stride, const TX *x, float *y,
                uint32_t n, uint32_t k, float softcap) {
    SGQ_CHECK(k > 0 && k % 256 == 0 && k / 256 <= (uint32_t)kQ6MaxBlocks,
              "gemv_q6_k: k=%u must be a multiple of 256, at most %d", k, 256 * kQ6MaxBlocks);
    SGQ_CHECK(row_stride % 16 == 0 && row_stride >= (size_t)(k / 256) * kQ6BlockBytes &&
                  row_stride <= (size_t)kQ6Chunks * kWave * 16,
              "gemv_q6_k: row stride %zu must be a multiple of 16 holding k/256 blocks",
              row_stride);
    SGQ_CHECK(((uintptr_t)w & 15) == 0, "gemv_q6_k: weights must be 16-byte aligned");
    SGQ_CHECK(n > 0, "gemv_q6_k: empty");
    const size_t lds = ((size_t)k * 2 + 15) / 16 * 16 + (size_t)kQ6Waves * 2 * (row_stride + 16);
    const int rows_per_wg = 2 * kQ6Waves;
    // three workgroups (12 waves) per CU: the per-row work is a chain of LDS
    // reads and dependent VALU, so more waves hide more of it
    int grid = device_info().cus * 3;
    const int max_grid = (int)((n + rows_per_wg - 1) / rows_per_wg);
    if (grid > max_grid) grid = max_grid;
    hipLaunchKernelGGL(gemv_q6_k_kernel<TX>, dim3(grid), dim3(kQ6WG), lds, st,
                       static_cast<const uint8_t *>(w), (uint32_t)row_stride, x, y, (int)n,
                       (int)k, softcap);
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}
}  // namespace

int launch_gemv_q6_k(hipStream_t st, const void *w, size_t row_stride, const float *x, float *y,
                     uint32_t n, uint32_t k, float softcap) {
    return gemv_q6_k_t(st, w, row_stride, x, y, n, k, softcap);
}
int launch_gemv_q6_k(hipStream_t st, const void *w, size_t row_stride, const uint16_t *x,
                     float *y, uint32_t n, uint32_t k, float softcap) {
    return gemv_q6_k_t(st, w, row_stride, x, y, n, k, softcap);
}

}  // namespace sgq
