// Decode Q4_0 GEMV for gfx950: y[n] = W[n×k] · x[k], W in GGUF Q4_0 blocks
// (f16 d + 16 nibble bytes, 18 B), x and y fp32.
//
// Replaces gemv_q4_0 (crates/sg-gpu/shaders/gemv_q4_0.wgsl:52-112), whose
// semantics are y[n] = sum_b d_b * sum_j (q_j - 8) * x_j in f32.
//
// Design (HBM-bound, ~1.8 flop/B):
//  * The fp32 FMA form costs ~2.4 VALU ops per weight (nibble split, int→f32
//    convert, FMA); on 256 CUs at 64 lanes/clk that is as long as streaming
//    the weights at 8 TB/s.  So each wave first splits its slice of x into
//    three int8 limbs per 32-block, x ≈ d_x·(x1 + x2/128 + x3/128²) with
//    d_x = amax/127 kept in f32 (residual ≤ amax·2^-22, i.e. fp32-grade),
//    and the inner loop is v_dot4_i32_i8 on the raw nibbles: ~1.1 op/weight.
//    The −8 offset folds into the accumulator seed: −8·Σ x_limb per block.
//  * x limbs live in registers for the whole kernel: lane l of a wave always
//    owns blocks l, l+64, l+128 of its K-slice, so the persistent waves walk
//    rows with no LDS traffic for x at all.  K > 6144 is cut into 2 or 4
//    slices handled by the waves of one workgroup, merged through LDS in
//    fixed order.
//  * Each lane reads its block as 20 bytes from a 4-byte-aligned address
//    (even blocks start 4-aligned, odd blocks 2 bytes past); v_perm_b32
//    realigns the 16 nibble bytes with a per-lane selector.  A wave's loads
//    cover 1152 contiguous bytes per row: fully used cache lines.
//  * Row sums: butterfly over the wave (fixed order: deterministic).
#include "sgq_internal.h"

namespace sgq {
namespace {

constexpr int kWG = 256;  // 4 waves
constexpr float kInv128 = 1.0f / 128.0f;

template <int NBL>
struct XLimbs {
    int q[NBL][3][8];   // int8x4 words: limb, word (weights 4w..4w+3)
    int seed[NBL][3];   // -8 * sum(limb) over the block
    float d[NBL];       // d_x (f32, unrounded)
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

__device__ __forceinline__ int pack4(int a, int b, int c, int d) {
    return (a & 0xff) | ((b & 0xff) << 8) | ((c & 0xff) << 16) | ((d & 0xff) << 24);
}

// Split one 32-block of x into three int8 limbs (see file header).
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
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(v[j]));
    float d = amax * (1.0f / 127.0f);
    float id = d > 0.f ? 1.0f / d : 0.f;
    L.d[i] = d;
    int s0 = 0, s1 = 0, s2 = 0;
    int l0[32], l1[32], l2[32];
#pragma unroll
    for (int j = 0; j < 32; j++) {
        float t = v[j] * id;
        float a = __builtin_rintf(t);
        float r = (t - a) * 128.f;
        float b = __builtin_rintf(r);
        float c = __builtin_rintf((r - b) * 128.f);
        l0[j] = (int)a;
        l1[j] = (int)b;
        l2[j] = (int)c;
        s0 += l0[j];
        s1 += l1[j];
        s2 += l2[j];
    }
#pragma unroll
    for (int w = 0; w < 8; w++) {
        L.q[i][0][w] = pack4(l0[4 * w], l0[4 * w + 1], l0[4 * w + 2], l0[4 * w + 3]);
        L.q[i][1][w] = pack4(l1[4 * w], l1[4 * w + 1], l1[4 * w + 2], l1[4 * w + 3]);
        L.q[i][2][w] = pack4(l2[4 * w], l2[4 * w + 1], l2[4 * w + 2], l2[4 * w + 3]);
    }
    L.seed[i][0] = -8 * s0;
    L.seed[i][1] = -8 * s1;
    L.seed[i][2] = -8 * s2;
}

// One block's contribution d_w * sum_j (q_j - 8) * x_j from its 5 raw words.
template <int NBL>
__device__ __forceinline__ float block_dot(const uint32_t (&w)[5], uint32_t sel, uint32_t dshift,
                                           const XLimbs<NBL> &L, int i) {
    int c0 = L.seed[i][0], c1 = L.seed[i][1], c2 = L.seed[i][2];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        uint32_t qs = __builtin_amdgcn_perm(w[j + 1], w[j], sel);
        int lo = (int)(qs & 0x0F0F0F0Fu);
        int hi = (int)((qs >> 4) & 0x0F0F0F0Fu);
        c0 = __builtin_amdgcn_sdot4(lo, L.q[i][0][j], c0, false);
        c0 = __builtin_amdgcn_sdot4(hi, L.q[i][0][j + 4], c0, false);
        c1 = __builtin_amdgcn_sdot4(lo, L.q[i][1][j], c1, false);
        c1 = __builtin_amdgcn_sdot4(hi, L.q[i][1][j + 4], c1, false);
        c2 = __builtin_amdgcn_sdot4(lo, L.q[i][2][j], c2, false);
        c2 = __builtin_amdgcn_sdot4(hi, L.q[i][2][j + 4], c2, false);
    }
    float dw = f16_bits_to_f32((w[0] >> dshift) & 0xffffu);
    float f = __builtin_fmaf((float)c2, kInv128, (float)c1);
    f = __builtin_fmaf(f, kInv128, (float)c0);
    return dw * (L.d[i] * f);
}

// S = K-slices per row (waves of a workgroup share rows when S > 1),
// NBL = blocks per lane per slice, R = rows per wave per iteration.
template <int NBL, int R>
__global__ __launch_bounds__(kWG) void gemv_q4_0_kernel(const uint8_t *__restrict__ W,
                                                        const float *__restrict__ x,
                                                        float *__restrict__ y, int n, int nb,
                                                        int S, int slice_blocks) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int s = wave % S;
    const int p = wave / S;
    const int P = (kWG / kWave) / S;
    __shared__ float red[kWG / kWave][R];

    XLimbs<NBL> L;
    int boff[NBL];
    bool valid[NBL];
#pragma unroll
    for (int i = 0; i < NBL; i++) {
        int local = lane + kWave * i;
        int b = s * slice_blocks + local;
        valid[i] = local < slice_blocks && b < nb;
        boff[i] = b * 18 - (lane & 1) * 2;  // 4-aligned start of the 20-byte window
        if (valid[i]) {
            quantize_block(x + (size_t)b * 32, L, i);
        } else {
#pragma unroll
            for (int l = 0; l < 3; l++) {
                L.seed[i][l] = 0;
#pragma unroll
                for (int w = 0; w < 8; w++) L.q[i][l][w] = 0;
            }
            L.d[i] = 0.f;
        }
    }
    // Even blocks: qs = bytes 2..17 of the window, d = low half of word 0.
    // Odd blocks: window starts 2 bytes early, qs = words 1..4, d = high half.
    const uint32_t sel = (lane & 1) ? 0x07060504u : 0x05040302u;
    const uint32_t dshift = (lane & 1) ? 16u : 0u;
    const size_t row_bytes = (size_t)nb * 18;
    const int rows_per_tile = P * R;
    const int tiles = (n + rows_per_tile - 1) / rows_per_tile;

    for (int tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
        const int row0 = tile * rows_per_tile + p * R;
        uint32_t wv[R][NBL][5];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = row0 + r;
#pragma unroll
            for (int i = 0; i < NBL; i++) {
                if (row < n && valid[i]) {
                    const uint32_t *src = reinterpret_cast<const uint32_t *>(
                        W + (size_t)row * row_bytes + boff[i]);
#pragma unroll
                    for (int j = 0; j < 5; j++) wv[r][i][j] = __builtin_nontemporal_load(src + j);
                } else {
#pragma unroll
                    for (int j = 0; j < 5; j++) wv[r][i][j] = 0u;  // d = 0: contributes 0
                }
            }
        }
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            float a = 0.f;
#pragma unroll
            for (int i = 0; i < NBL; i++) a += block_dot(wv[r][i], sel, dshift, L, i);
            acc[r] = wave_sum(a);
        }
        if (S == 1) {
            if (lane < R) {
                float v = acc[0];
#pragma unroll
                for (int r = 1; r < R; r++)
                    if (lane == r) v = acc[r];
                const int row = row0 + lane;
                if (row < n) y[row] = v;
            }
        } else {
            if (lane == 0) {
#pragma unroll
                for (int r = 0; r < R; r++) red[wave][r] = acc[r];
            }
            __syncthreads();
            if (s == 0 && lane < R) {
                float v = 0.f;
                for (int q = 0; q < S; q++) v += red[p * S + q][lane];
                const int row = row0 + lane;
                if (row < n) y[row] = v;
            }
            __syncthreads();
        }
    }
}

template <int NBL, int R>
int launch(hipStream_t st, const void *w, const float *x, float *y, int n, int nb, int S,
           int slice_blocks) {
    static int max_blocks_per_cu = 0;
    if (max_blocks_per_cu == 0) {
        int v = 0;
        SGQ_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, gemv_q4_0_kernel<NBL, R>, kWG,
                                                             0));
        max_blocks_per_cu = v > 0 ? v : 1;
    }
    const int P = (kWG / kWave) / S;
    const int tiles = (n + P * R - 1) / (P * R);
    int grid = device_info().cus * max_blocks_per_cu;
    if (grid > tiles) grid = tiles;
    hipLaunchKernelGGL((gemv_q4_0_kernel<NBL, R>), dim3(grid), dim3(kWG), 0, st,
                       static_cast<const uint8_t *>(w), x, y, n, nb, S, slice_blocks);
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}

}  // namespace

int launch_gemv_q4_0(hipStream_t st, const void *w, const float *x, float *y, uint32_t n,
                     uint32_t k) {
    SGQ_CHECK(k % 64 == 0 && k > 0, "gemv_q4_0: k=%u must be a positive multiple of 64", k);
    SGQ_CHECK(k <= 65536, "gemv_q4_0: k=%u exceeds 65536", k);
    SGQ_CHECK(n > 0 && n < (1u << 31), "gemv_q4_0: bad n=%u", n);
    SGQ_CHECK(((uintptr_t)w & 3) == 0, "gemv_q4_0: weights must be 4-byte aligned");
    SGQ_CHECK(((uintptr_t)x & 15) == 0, "gemv_q4_0: x must be 16-byte aligned");
    const int nb = (int)(k / 32);
    // Fewest K-slices that keep <= 3 blocks per lane; else 4 slices.
    int S = 1;
    while (S < 4 && (nb + S - 1) / S > 3 * kWave) S *= 2;
    int slice = (nb + S - 1) / S;
    slice += slice & 1;  // even: lane parity == block parity
    const int nbl = (slice + kWave - 1) / kWave;
    switch (nbl) {
        case 1: return launch<1, 4>(st, w, x, y, (int)n, nb, S, slice);
        case 2: return launch<2, 4>(st, w, x, y, (int)n, nb, S, slice);
        case 3: return launch<3, 4>(st, w, x, y, (int)n, nb, S, slice);
        case 4: return launch<4, 2>(st, w, x, y, (int)n, nb, S, slice);
        case 5:
        case 6: return launch<6, 1>(st, w, x, y, (int)n, nb, S, slice);
        default: return launch<8, 1>(st, w, x, y, (int)n, nb, S, slice);
    }
}

}  // namespace sgq
