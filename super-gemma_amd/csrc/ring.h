// Building blocks of the streamed Q4_0 GEMV shared by the standalone GEMV
// kernels and the persistent decode kernel: the limb block dot, the LDS
// ring geometry (a wave streams row slices into its own ring slots with
// global_load_lds_dwordx4), asm LDS reads that the compiler's waitcnt pass
// cannot drain the ring for, and a fixed-order DPP wave sum.
#pragma once
#include "limbs.h"

namespace sgq {
namespace {

// One block's contribution d_w · Σ_j (q_j − 8)·x_j from its 5 raw words (the
// 20-byte window holding its f16 scale and 16 nibble bytes).  Word w of a
// limb holds, nibble by nibble, the limb values of weights 4w, 16+4w, 4w+1,
// 17+4w, 4w+2, 18+4w, 4w+3, 19+4w: the order in which qs bytes 4w..4w+3's
// low/high nibbles appear in a 32-bit qs word.
template <int NBL>
__device__ __forceinline__ float block_dot(const uint32_t (&w)[5], uint32_t sel, uint32_t dshift,
                                           const XLimbs<NBL> &L, int i) {
    int t[4];
#pragma unroll
    for (int j = 0; j < 4; j++) t[j] = (int)(__builtin_amdgcn_perm(w[j + 1], w[j], sel) ^ 0x88888888u);
    // Horner over the limbs in one exact integer accumulator: the result is
    // Σ (q-8)·v with |v| <= 28672, so |c| <= 32·8·28672 < 2^23 (exact as
    // f32); ×16 is a shift.
    int ci = 0;
#pragma unroll
    for (int l = 0; l < kLimbs; l++) {
        if (l) ci *= 16;
#pragma unroll
        for (int j = 0; j < 4; j++) ci = __builtin_amdgcn_sdot8(t[j], L.q[i][l][j], ci, false);
    }
    const float c = (float)ci;
    const float dw = f16_bits_to_f32((w[0] >> dshift) & 0xffffu);
    return dw * (L.d[i] * c);
}

constexpr int kRStages = 6;                     // ring slots per wave
constexpr int kRLoads = 3;                      // 3 × 1 KB DMA per slot
constexpr int kRSlot = kRLoads * kWave * 16;    // 3072 B: row slice <= 170 blocks

// s_waitcnt immediate for gfx9: wait until at most `n` vector-memory ops are
// outstanding (vmcnt bits [3:0] and [15:14]); expcnt/lgkmcnt left at "any".
constexpr int vmcnt_imm(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8); }
// Cache policy of the weight stream's LDS DMA: nontemporal (the `nt` bit).
// Weights are read once per step, and a streaming read of 2 GiB through
// the same per-wave 3-slot ring runs at 6.8 TB/s with it against 5.9
// without (2048 workgroups; with 16-byte register loads: 7.1 against 6.2).
constexpr int kStreamPolicy = 2;
typedef __attribute__((address_space(1))) void gvoid_t;
typedef __attribute__((address_space(3))) void lvoid_t;

// Reads the NBL 20-byte block windows of a lane from a ring slot, all
// issued before one wait.  Written as asm so the compiler's waitcnt pass,
// which cannot tell these reads from slots still being filled by LDS DMA,
// does not force vmcnt(0) (a full drain of the ring) in front of them; the
// explicit vmcnt wait already orders them.  Outputs are early-clobber: the
// address registers must survive until the last read has issued.
#define SGQ_RD5(o, a)                                       \
    "ds_read_b32 %" #o "0, %" #a "\n"                      \
    "ds_read_b32 %" #o "1, %" #a " offset:4\n"             \
    "ds_read_b32 %" #o "2, %" #a " offset:8\n"             \
    "ds_read_b32 %" #o "3, %" #a " offset:12\n"            \
    "ds_read_b32 %" #o "4, %" #a " offset:16\n"
template <int NBL>
__device__ __forceinline__ void lds_read_blocks(const uint8_t *st, const int (&boff)[NBL],
                                                uint32_t (&w)[NBL][5]);
template <>
__device__ __forceinline__ void lds_read_blocks<1>(const uint8_t *st, const int (&boff)[1],
                                                   uint32_t (&w)[1][5]) {
    const uint32_t a0 = (uint32_t)(uintptr_t)(st + boff[0]);
    asm volatile(
        "ds_read_b32 %0, %5\n ds_read_b32 %1, %5 offset:4\n ds_read_b32 %2, %5 offset:8\n"
        "ds_read_b32 %3, %5 offset:12\n ds_read_b32 %4, %5 offset:16\n s_waitcnt lgkmcnt(0)"
        : "=&v"(w[0][0]), "=&v"(w[0][1]), "=&v"(w[0][2]), "=&v"(w[0][3]), "=&v"(w[0][4])
        : "v"(a0)
        : "memory");
}
template <>
__device__ __forceinline__ void lds_read_blocks<2>(const uint8_t *st, const int (&boff)[2],
                                                   uint32_t (&w)[2][5]) {
    const uint32_t a0 = (uint32_t)(uintptr_t)(st + boff[0]);
    const uint32_t a1 = (uint32_t)(uintptr_t)(st + boff[1]);
    asm volatile(
        "ds_read_b32 %0, %10\n ds_read_b32 %1, %10 offset:4\n ds_read_b32 %2, %10 offset:8\n"
        "ds_read_b32 %3, %10 offset:12\n ds_read_b32 %4, %10 offset:16\n"
        "ds_read_b32 %5, %11\n ds_read_b32 %6, %11 offset:4\n ds_read_b32 %7, %11 offset:8\n"
        "ds_read_b32 %8, %11 offset:12\n ds_read_b32 %9, %11 offset:16\n s_waitcnt lgkmcnt(0)"
        : "=&v"(w[0][0]), "=&v"(w[0][1]), "=&v"(w[0][2]), "=&v"(w[0][3]), "=&v"(w[0][4]),
          "=&v"(w[1][0]), "=&v"(w[1][1]), "=&v"(w[1][2]), "=&v"(w[1][3]), "=&v"(w[1][4])
        : "v"(a0), "v"(a1)
        : "memory");
}
template <>
__device__ __forceinline__ void lds_read_blocks<3>(const uint8_t *st, const int (&boff)[3],
                                                   uint32_t (&w)[3][5]) {
    const uint32_t a0 = (uint32_t)(uintptr_t)(st + boff[0]);
    const uint32_t a1 = (uint32_t)(uintptr_t)(st + boff[1]);
    const uint32_t a2 = (uint32_t)(uintptr_t)(st + boff[2]);
    asm volatile(
        "ds_read_b32 %0, %15\n ds_read_b32 %1, %15 offset:4\n ds_read_b32 %2, %15 offset:8\n"
        "ds_read_b32 %3, %15 offset:12\n ds_read_b32 %4, %15 offset:16\n"
        "ds_read_b32 %5, %16\n ds_read_b32 %6, %16 offset:4\n ds_read_b32 %7, %16 offset:8\n"
        "ds_read_b32 %8, %16 offset:12\n ds_read_b32 %9, %16 offset:16\n"
        "ds_read_b32 %10, %17\n ds_read_b32 %11, %17 offset:4\n ds_read_b32 %12, %17 offset:8\n"
        "ds_read_b32 %13, %17 offset:12\n ds_read_b32 %14, %17 offset:16\n s_waitcnt lgkmcnt(0)"
        : "=&v"(w[0][0]), "=&v"(w[0][1]), "=&v"(w[0][2]), "=&v"(w[0][3]), "=&v"(w[0][4]),
          "=&v"(w[1][0]), "=&v"(w[1][1]), "=&v"(w[1][2]), "=&v"(w[1][3]), "=&v"(w[1][4]),
          "=&v"(w[2][0]), "=&v"(w[2][1]), "=&v"(w[2][2]), "=&v"(w[2][3]), "=&v"(w[2][4])
        : "v"(a0), "v"(a1), "v"(a2)
        : "memory");
}
#undef SGQ_RD5
__device__ __forceinline__ void lds_write_f32(uint8_t *p, float v) {
    const uint32_t a = (uint32_t)(uintptr_t)p;
    asm volatile("ds_write_b32 %0, %1\n s_waitcnt lgkmcnt(0)" : : "v"(a), "v"(v) : "memory");
}
__device__ __forceinline__ float lds_read_f32(const uint8_t *p) {
    const uint32_t a = (uint32_t)(uintptr_t)p;
    float v;
    asm volatile("ds_read_b32 %0, %1\n s_waitcnt lgkmcnt(0)" : "=&v"(v) : "v"(a) : "memory");
    return v;
}

// Sum over the wave in a fixed order with DPP: row_shr 1/2/4/8 leave each
// 16-lane row's sum in its lane 15, row_bcast 15/31 carry them up, lane 63
// ends with the total (deterministic).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float v) {
    const int t = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xf,
                                              false);
    return v + __builtin_bit_cast(float, t);
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v = dpp_add<0x111, 0xf>(v);  // row_shr:1
    v = dpp_add<0x112, 0xf>(v);  // row_shr:2
    v = dpp_add<0x114, 0xf>(v);  // row_shr:4
    v = dpp_add<0x118, 0xf>(v);  // row_shr:8
    v = dpp_add<0x142, 0xa>(v);  // row_bcast:15
    v = dpp_add<0x143, 0xc>(v);  // row_bcast:31
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

}  // namespace
}  // namespace sgq
