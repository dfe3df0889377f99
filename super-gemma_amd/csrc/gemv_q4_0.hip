// Decode Q4_0 GEMV for gfx950: y[n] = W[n×k] · x[k], W in GGUF Q4_0 blocks
// (f16 d + 16 nibble bytes, 18 B), x and y fp32.
//
// Replaces gemv_q4_0 (crates/sg-gpu/shaders/gemv_q4_0.wgsl:52-112), whose
// semantics are y[n] = sum_b d_b * sum_j (q_j - 8) * x_j in f32.
//
// Design (HBM-bound, ~1.8 flop/B):
//  * VALU, not the MFMA, is the scarce unit next to an 8 TB/s weight stream:
//    at ~1 wave-instruction per 4 cycles per SIMD, an fp32 FMA form (nibble
//    split, int->f32, FMA: ~2.4 ops/weight) takes as long as the stream.
//    So x is split once per 32-block into four signed 4-bit limbs, the
//    base-16 digits of v = rint(x·(7/amax)·4096) (limbs.h; |error| ≤
//    amax·1.7e-5), and the inner loop is v_dot8_i32_i4 on the
//    weight nibbles themselves: qs ^ 0x88888888 turns every nibble q into
//    the signed 4-bit value q-8, so one XOR per 8 weights is the whole
//    unpack.  Per block: 4 perm + 4 xor + 16 dot8 + 3 Horner steps in one
//    exact integer accumulator (|c| <= 32·8·28672 < 2^23) + cvt + 2 mul.
//  * x limbs live in registers for the whole kernel: lane l of a wave always
//    owns blocks l, l+64, l+128 of its K-slice.
//  * Each lane reads its block as 20 bytes from a 4-byte-aligned address
//    (even blocks start 4-aligned, odd blocks 2 bytes past); v_perm_b32
//    realigns the 16 nibble bytes with a per-lane selector.
//  * Row sums: butterfly over the wave (fixed order: deterministic).
#include <mutex>

#include "ring.h"

namespace sgq {
namespace {

constexpr int kWG = 256;  // 4 waves
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}


template <int R, int NBL>
__device__ __forceinline__ void load_tile(uint32_t (&wv)[R][NBL][5], const uint8_t *__restrict__ W,
                                          size_t row_bytes, int row0, int n,
                                          const int (&boff)[NBL], const bool (&valid)[NBL]) {
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int row = row0 + r;
#pragma unroll
        for (int i = 0; i < NBL; i++) {
            if (row < n && valid[i]) {
                const uint32_t *src =
                    reinterpret_cast<const uint32_t *>(W + (size_t)row * row_bytes + boff[i]);
#pragma unroll
                for (int j = 0; j < 5; j++) wv[r][i][j] = src[j];
            } else {
#pragma unroll
                for (int j = 0; j < 5; j++) wv[r][i][j] = 0u;  // d = 0: contributes 0
            }
        }
    }
}

// Register path (any K % 64 == 0): S = K-slices per row (waves of a
// workgroup share rows when S > 1), NBL = blocks per lane per slice, R = rows
// per wave per tile.  Each lane quantizes its own blocks of x; the tile loop
// is software-pipelined (the next tile's weights load while this one
// computes).
template <int NBL, int R, typename TX, typename TY>
__global__ __launch_bounds__(kWG) void gemv_q4_0_kernel(const uint8_t *__restrict__ W,
                                                        const TX *__restrict__ x,
                                                        TY *__restrict__ y, int n, int nb,
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
            for (int l = 0; l < kLimbs; l++)
#pragma unroll
                for (int w = 0; w < 4; w++) L.q[i][l][w] = 0;
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
    const int G = gridDim.x;

    auto compute = [&](const uint32_t(&wv)[R][NBL][5], int tile) {
        const int row0 = tile * rows_per_tile + p * R;
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
                if (row < n) act_st(y, row, v);
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
                if (row < n) act_st(y, row, v);
            }
            __syncthreads();
        }
    };

    uint32_t wa[R][NBL][5], wb[R][NBL][5];
    int tile = blockIdx.x;
    if (tile < tiles) load_tile(wa, W, row_bytes, tile * rows_per_tile + p * R, n, boff, valid);
    while (tile < tiles) {
        if (tile + G < tiles)
            load_tile(wb, W, row_bytes, (tile + G) * rows_per_tile + p * R, n, boff, valid);
        compute(wa, tile);
        tile += G;
        if (tile >= tiles) break;
        if (tile + G < tiles)
            load_tile(wa, W, row_bytes, (tile + G) * rows_per_tile + p * R, n, boff, valid);
        compute(wb, tile);
        tile += G;
    }
}

// ---------------------------------------------------------------------------
// Streamed variant (K % 256 == 0, 16-byte aligned W).
//
// x arrives pre-split into limbs (BlockLimbs per 32-block, written once per
// x by gemv_prep_x_kernel, or by a producer kernel that fuses it), so the
// GEMV itself does no quantization and no LDS table.
//
// Each wave owns a private ring of LDS slots (ring_stages) and streams exactly
// the row slices it reduces with global_load_lds_dwordx4 (a lane moves 16 B
// straight into LDS; the data never occupies VGPRs).  The slots are filled
// before the loop; each is refilled with the slice ring_stages rounds ahead
// as soon as its words are in registers, so slices stream in while a row
// computes.  A wave waits only on its own vmcnt.  For K <= 5440 a row is one
// slice and waves never synchronize; for longer K the S = 2 or 4 waves of a
// workgroup take the S slices of the same row and combine partials through
// LDS in fixed order (after the loop, or with one barrier per row past 64
// rounds per wave).
// ---------------------------------------------------------------------------
// Waves per workgroup, by prologue and epilogue (the enums are declared in
// sgq_internal.h).  Eight waves (one workgroup per CU) for the norm and
// embedding prologues with plain row stores (QKV, the LM head): half the
// redundant prologue work per CU, 10.6 -> 9.1 us per QKV launch in the
// decode step; the table-fed call with the table copied into LDS once per
// workgroup instead of once per wave (config 1, 8 interleaved runs: median
// 12.40 against 13.3 us); and the x prologue of the typed call (full call at config 1
// 14.4-14.6 us with a separate limb kernel, 13.0-13.4 with the prologue in
// eight-wave workgroups, 13.5-14.6 in four-wave ones; its x loads issued
// ahead of the weight stream and waited for behind it: 12.95 -> 12.57 us).  Four elsewhere:
// eight made the gate/up launch (GeGLU
// epilogue, 32-unit limb blocks, so 336 workgroups on 256 CUs) 25.5 ->
// 29.2 us, and table-fed launches gain nothing.
constexpr int ring_waves(int pro, int epi) {
    return (pro == kProNorm || pro == kProEmbed || pro == kProX || pro == kProTableLds ||
            pro == kProSliceLds) && epi == kEpiRows ? 8 : 4;
}
// Ring slots per wave and waves per CU (the grid).  The one-slice plain
// launches (the limb table copied into LDS, or built from x in the
// prologue; row outputs: the typed and by-name GEMV at K <= 5440) run one
// slot per wave at 16 waves per CU: at K=5376, N=21504 the kernel took
// 12.1-12.35 against 12.6-13.35 us with two slots at 8 waves per CU
// (interleaved runs on three boxes), the same bytes in flight spread over
// twice the waves, which hides more of each row's compute.  Everything else
// keeps two slots at 8 waves per CU: the norm-prologue launches would
// repeat their prologue in twice the workgroups (decode step 233.1 -> 230.1
// tok/s), and one slot made the residual and GeGLU launches and the
// K-sliced rows (K=21504: 15.8-16.4 against 13.7-15.4 us) slower.  Fewer
// bytes in flight stream faster here: three slots at 8 waves per CU took
// 13.3-13.5 us at config 1, six 15.8 us.
constexpr bool ring_plain(int pro, int epi) {
    return (pro == kProTableLds || pro == kProSliceLds || pro == kProX) && epi == kEpiRows;
}
constexpr int ring_stages(int pro, int epi) { return ring_plain(pro, epi) ? 1 : 2; }
constexpr int ring_waves_per_cu(int pro, int epi) { return ring_plain(pro, epi) ? 16 : 8; }

// Row r of the concatenated targets -> (matrix, local row).
__device__ __forceinline__ int target_of(const GemvTargets &tg, int row, int *local) {
    int j = 0;
#pragma unroll
    for (int q = 0; q < kGemvMaxTargets - 1; q++)
        if (q < tg.count - 1 && row >= tg.end[q]) j = q + 1;
    *local = row - (j ? tg.end[j - 1] : 0);
    return j;
}

// DMA one row slice (<= 3072 B) into a ring slot.  `row` is wave-uniform
// (scalar); past-the-end rows are clamped to row 0 so every call issues
// exactly kRLoads loads.  doff: the lane's precomputed byte offsets within
// the slice (clamped to 0 past its end).
__device__ __forceinline__ void issue_slice(const GemvTargets &tg, uint8_t *slot, int row, int n,
                                            size_t row_bytes, int slice_off,
                                            const int (&doff)[kRLoads]) {
    int local;
    const int j = target_of(tg, row < n ? row : 0, &local);
    const uint8_t *src =
        static_cast<const uint8_t *>(tg.w[j]) + (size_t)local * row_bytes + slice_off;
#pragma unroll
    for (int i = 0; i < kRLoads; i++)
        __builtin_amdgcn_global_load_lds((gvoid_t *)(src + doff[i]),
                                         (lvoid_t *)(slot + i * kWave * 16), 16, 0,
                                         kStreamPolicy);
}

// x (fp32 or f16, nb blocks of 32) -> limb table: 8 lanes per 32-block,
// four values each (limbs_block8).
template <typename T>
__global__ __launch_bounds__(256) void gemv_prep_x_kernel(const T *__restrict__ x,
                                                          BlockLimbs *__restrict__ xl, int nb) {
    const int i = blockIdx.x * 256 + threadIdx.x;  // index of 4 values
    if (i >= nb * 8) return;                         // whole 8-lane groups exit together
    const float4 v = act_ld4(x, i);
    limbs_block8(v, i & 7, &xl[i >> 3]);
}

__device__ __forceinline__ void store_row(const GemvTargets &tg, int row, float v) {
    int local;
    const int j = target_of(tg, row, &local);
    if (tg.softcap > 0.f) v = tg.softcap * tanhf(v / tg.softcap);
    if (tg.half_out)
        act_st(reinterpret_cast<uint16_t *>(tg.y[j]), local, v);
    else
        tg.y[j][local] = v;
}

// LDS of the streamed kernel: the wave rings, then two rounds of row
// partials (one float per wave), cross-wave scratch, the row results of the
// residual epilogue (64 rounds per wave), then (prologues only) the x limb
// table.
constexpr int kGegluUnits = 32;  // units (gate/up row pairs) per workgroup (4 waves)
template <int WV, int ST>
struct RingLds {
    static constexpr int kRing = WV * ST * kRSlot;
    static constexpr int kRed = kRing;
    static constexpr int kScr = kRed + 2 * 4 * WV;
    static constexpr int kScrBytes = (kGegluUnits * 4 > 16 * WV ? kGegluUnits * 4 : 16 * WV);
    static constexpr int kRows = kScr + kScrBytes;
    static constexpr int kTab = kRows + WV * kWave * 4;
};
constexpr int ring_lds_tab(int wv, int st) {
    return wv * st * kRSlot + 2 * 4 * wv + (kGegluUnits * 4 > 16 * wv ? kGegluUnits * 4 : 16 * wv) +
           wv * kWave * 4;
}
constexpr int kMaxTabBlocks = 3 * kWave;  // one slice: <= 192 blocks

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void lds_write_f32x4(uint8_t *p, float4 v) {
    const uint32_t a = (uint32_t)(uintptr_t)p;
    const f32x4_t t = {v.x, v.y, v.z, v.w};
    asm volatile("ds_write_b128 %0, %1\n s_waitcnt lgkmcnt(0)" : : "v"(a), "v"(t) : "memory");
}
__device__ __forceinline__ float4 lds_read_f32x4(const uint8_t *p) {
    const uint32_t a = (uint32_t)(uintptr_t)p;
    f32x4_t v;
    asm volatile("ds_read_b128 %0, %1\n s_waitcnt lgkmcnt(0)" : "=&v"(v) : "v"(a) : "memory");
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void lds_write_u32(uint8_t *p, uint32_t v) {
    const uint32_t a = (uint32_t)(uintptr_t)p;
    asm volatile("ds_write_b32 %0, %1" : : "v"(a), "v"(v) : "memory");
}
// Workgroup barrier for LDS written with the asm stores above: waits for
// this wave's LDS traffic only (vector memory, i.e. the weight DMA, keeps
// streaming).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
}

// Values passed through an empty asm: to the compiler they are defined here,
// so a load behind them is waited for here (before the weight stream
// starts) and not at their first use, where the compiler, which cannot
// count the stream's LDS DMA together with ordinary loads, would wait for
// everything in flight.
__device__ __forceinline__ void settle(float &v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void settle(uint32_t &v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void settle(float4 &v) {
    asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w));
}

// An 8-lane group's limb block written as an LDS table entry (BlockLimbs
// layout) from its words (limbs_words8).  The words of all of a thread's
// blocks are computed before any of them is written: the asm stores are
// scheduling barriers, and each block is a long dependent chain (max over
// the group, reciprocal, rounding, byte transposes), so computing and
// storing block by block would run the chains one after another.
__device__ __forceinline__ void limb_words_to_lds(const uint32_t (&word)[kLimbs], float d, int g,
                                                  uint8_t *dst) {
    if (g < 4) {
#pragma unroll
        for (int l = 0; l < kLimbs; l++) lds_write_u32(dst + (l * 4 + g) * 4, word[l]);
        if (g == 0) lds_write_u32(dst + 64, __builtin_bit_cast(uint32_t, d));
    }
}

__device__ __forceinline__ float gelu_tanh_g(float x) {
    const float k = 0.7978845608028654f;
    return 0.5f * x * (1.f + tanhf(k * (x + 0.044715f * x * x * x)));
}

// Sum of float4s over the workgroup in a fixed order (every workgroup that
// sums the same inputs gets the same bits): lanes in DPP order, then the
// WV waves in order through `scr`.
template <int WV>
__device__ __forceinline__ float4 wg_sum4(float4 v, uint8_t *scr) {
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    v.x = wave_sum_dpp(v.x);
    v.y = wave_sum_dpp(v.y);
    v.z = wave_sum_dpp(v.z);
    v.w = wave_sum_dpp(v.w);
    if (lane == 0) lds_write_f32x4(scr + wave * 16, v);
    lds_barrier();
    float4 r = lds_read_f32x4(scr);
#pragma unroll
    for (int w = 1; w < WV; w++) {
        const float4 t = lds_read_f32x4(scr + w * 16);
        r.x += t.x, r.y += t.y, r.z += t.z, r.w += t.w;
    }
    lds_barrier();  // scr may be reused
    return r;
}

// Rows of up to kGemvMaxTargets matrices sharing x (e.g. Q/K/V, gate/up) are
// one concatenated row space: one launch, one x table.  Everything that
// depends only on the wave (its K-slice, its rows, the DMA sources) is
// computed in scalar registers; the VALU does the block dots and the DPP
// reduction.  Lanes past the slice's last block read a genuine block of the
// slot (block 0 or 1, so its scale is a finite f16) against zero limbs.
//
// PRO/EPI select the fused prologue and epilogue (kPro*, kEpi*).  The
// prologue's global loads are issued before the weight stream's first
// slices (vector memory completes in order, so anything loaded after the
// stream started would wait for it), and everything it puts in LDS goes
// through asm accesses, so that the compiler, which cannot tell the table
// from ring slots still being filled, does not drain the stream first.
template <int NBL, int PRO, int EPI>
__global__ __launch_bounds__(ring_waves(PRO, EPI) * kWave) void gemv_q4_0_ring_kernel(GemvTargets tg,
                                                              const BlockLimbs *__restrict__ xl,
                                                              int n, int nb, int S, int slice,
                                                              GemvFuse fz) {
    extern __shared__ __align__(16) uint8_t gemv_smem[];
    constexpr int WV = ring_waves(PRO, EPI);
    constexpr int kRWG = WV * kWave;
    constexpr int GS = ring_stages(PRO, EPI);  // ring slots per wave
    constexpr int kPreSlices = GS;             // slots filled before the loop
    using Lds = RingLds<WV, GS>;
    static_assert(Lds::kTab == ring_lds_tab(WV, GS), "LDS layout");
    static_assert(EPI != kEpiGeglu || WV * 8 == kGegluUnits, "8 GeGLU units per wave");
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    // kProSliceLds: the workgroup's waves share one K-slice (its table in
    // LDS) and take P = WV different rows; otherwise the S waves of a row
    // group take the row's S slices
    constexpr bool kSliceWG = PRO == kProSliceLds;
    constexpr bool kTabLds = PRO == kProTableLds || kSliceWG;
    static_assert(!kSliceWG || EPI == kEpiRows, "per-workgroup slices write split rows");
    const int s = kSliceWG ? (int)(blockIdx.x % S) : wave % S;  // K-slice of this wave
    const int rw = kSliceWG ? wave : wave / S;  // row within the workgroup's row group
    const int P = kSliceWG ? WV : (kRWG / kWave) / S;  // rows per workgroup iteration
    const int wgi = kSliceWG ? (int)(blockIdx.x / S) : (int)blockIdx.x;  // row group
    uint8_t *ring = gemv_smem + wave * (GS * kRSlot);
    uint8_t *red = gemv_smem + Lds::kRed;  // [2][waves] floats
    uint8_t *scr = gemv_smem + Lds::kScr;
    uint8_t *tab = gemv_smem + Lds::kTab;
    uint8_t *rows_s = gemv_smem + Lds::kRows;
    const size_t row_bytes = (size_t)nb * 18;
    const int b0 = s * slice;
    const int slice_blocks = min(slice, nb - b0);
    const int slice_off = b0 * 18;
    const int slice_bytes = slice_blocks * 18;
    const int G = (kSliceWG ? (int)gridDim.x / S : (int)gridDim.x) * P;  // rows per round
    const int r0 = wgi * P + rw;
    constexpr int kUnitsPerWave = kGegluUnits / (kRWG / kWave);
    const int u0 = blockIdx.x * kGegluUnits + wave * kUnitsPerWave;  // kEpiGeglu

    int doff[kRLoads];
#pragma unroll
    for (int i = 0; i < kRLoads; i++) {
        const int off = (i * kWave + lane) * 16;
        doff[i] = off + 16 > slice_bytes ? 0 : off;
    }
    // rounds of rows this workgroup owns (the same for all its waves); only
    // real rounds are fetched, so no wave waits on loads it never uses
    auto row_of = [&](int it) -> int { return r0 + it * G; };  // row of round `it`
    const int rows_rounds =
        EPI == kEpiGeglu ? 2 * kUnitsPerWave : (n - wgi * P + G - 1) / G;
    // the weight slice of round `it` into ring slot `slot`
    auto issue = [&](int it) {
        uint8_t *slot = ring + (it % GS) * kRSlot;
        if (EPI == kEpiGeglu) {
            const uint8_t *w = static_cast<const uint8_t *>((it & 1) ? tg.w[1] : tg.w[0]);
            const uint8_t *src = w + (size_t)(u0 + (it >> 1)) * row_bytes + slice_off;
#pragma unroll
            for (int i = 0; i < kRLoads; i++)
                __builtin_amdgcn_global_load_lds((gvoid_t *)(src + doff[i]),
                                                 (lvoid_t *)(slot + i * kWave * 16), 16, 0,
                                         kStreamPolicy);
        } else {
            issue_slice(tg, slot, row_of(it), n, row_bytes, slice_off, doff);
        }
    };

    // ---- prologue loads (before the stream) --------------------------------
    constexpr int kGroups = kRWG / 8;                         // 8-lane groups
    constexpr int kPB = (kMaxTabBlocks + kGroups - 1) / kGroups;  // blocks per group
    const int grp = threadIdx.x >> 3, ge = threadIdx.x & 7;
    float4 pv[kGemvMaxPartials / kWave];
    float4 av[kPB], bv[kPB], xo_in, xo_u;
    [[maybe_unused]] f32x4_t xq0 = {}, xq1 = {}, xq2 = {};  // kProX, fp32 x (asm loads)
    [[maybe_unused]] i32x2_t xh0 = {}, xh1 = {}, xh2 = {};  // kProX, f16 x (asm loads)
    uint32_t eq[kPB];  // kProEmbed: 4 nibble bytes of the lane's values
    float ed[kPB];
    const int H4 = nb * 8;  // float4s of x
    const int per4 = (H4 + gridDim.x - 1) / gridDim.x;
    const int xo_i = blockIdx.x * per4 + (int)threadIdx.x;  // this thread's x_out float4
    const bool xo_on = fz.x_out != nullptr && (int)threadIdx.x < per4 && xo_i < H4;
    // (branch-free: indices are clamped and the extra values ignored, so the
    // compiler can count exactly which loads each later wait needs)
    float s_pre = 1.f;
    if (PRO == kProNorm) {
        // Issued by asm and waited for before the stream's first slices: the
        // compiler never sees these loads, so it adds no wait of its own
        // that would cover the stream (it cannot count LDS DMA and ordinary
        // loads together and would wait for everything).  Indices are
        // clamped; values past the end are ignored below.
        if (fz.scale) s_pre = *fz.scale;
        const float *A = fz.A, *B = fz.B;
        const float *xi = fz.x_out ? fz.x_in : A, *xu = fz.x_out ? fz.u : A;
        // wave 0 reads all np partial sums (lane l: entries l + 64k) and
        // hands their total to the others through LDS
        uint32_t op[8];
#pragma unroll
        for (int k = 0; k < 8; k++) op[k] = (uint32_t)min(lane + kWave * k, fz.np - 1) * 16u;
        const uint32_t ox = (uint32_t)(xo_on ? xo_i : 0) * 16u;
        uint32_t ob[kPB];
#pragma unroll
        for (int k = 0; k < kPB; k++) ob[k] = (uint32_t)(min(grp + kGroups * k, nb - 1) * 8 + ge) * 16u;
        f32x4_t t0, t1, t2, t3, t4, t5, t6, t7, t8, t9;
        if (wave == 0) {
            asm volatile(
                "global_load_dwordx4 %0, %8, %16\n"
                "global_load_dwordx4 %1, %9, %16\n"
                "global_load_dwordx4 %2, %10, %16\n"
                "global_load_dwordx4 %3, %11, %16\n"
                "global_load_dwordx4 %4, %12, %16\n"
                "global_load_dwordx4 %5, %13, %16\n"
                "global_load_dwordx4 %6, %14, %16\n"
                "global_load_dwordx4 %7, %15, %16\n"
                : "=&v"(t0), "=&v"(t1), "=&v"(t2), "=&v"(t3), "=&v"(t4), "=&v"(t5), "=&v"(t6),
                  "=&v"(t7)
                : "v"(op[0]), "v"(op[1]), "v"(op[2]), "v"(op[3]), "v"(op[4]), "v"(op[5]),
                  "v"(op[6]), "v"(op[7]), "s"(fz.part)
                : "memory");
        } else {
            t0 = t1 = t2 = t3 = t4 = t5 = t6 = t7 = f32x4_t{0.f, 0.f, 0.f, 0.f};
        }
        asm volatile(
            "global_load_dwordx4 %0, %2, %3\n"
            "global_load_dwordx4 %1, %2, %4\n"
            : "=&v"(t8), "=&v"(t9)
            : "v"(ox), "s"(xi), "s"(xu)
            : "memory");
        static_assert((kPB == 6 || kPB == 3) && kGemvMaxPartials == 8 * kWave,
                      "asm prologue layout");
        f32x4_t a0, a1, a2, a3 = {}, a4 = {}, a5 = {}, c0, c1, c2, c3 = {}, c4 = {}, c5 = {};
        if constexpr (kPB == 3) {
            asm volatile(
                "global_load_dwordx4 %0, %6, %9\n"
                "global_load_dwordx4 %1, %7, %9\n"
                "global_load_dwordx4 %2, %8, %9\n"
                "global_load_dwordx4 %3, %6, %10\n"
                "global_load_dwordx4 %4, %7, %10\n"
                "global_load_dwordx4 %5, %8, %10\n"
                : "=&v"(a0), "=&v"(a1), "=&v"(a2), "=&v"(c0), "=&v"(c1), "=&v"(c2)
                : "v"(ob[0]), "v"(ob[1]), "v"(ob[2]), "s"(A), "s"(B)
                : "memory");
        } else
        asm volatile(
            "global_load_dwordx4 %0, %12, %18\n"
            "global_load_dwordx4 %1, %13, %18\n"
            "global_load_dwordx4 %2, %14, %18\n"
            "global_load_dwordx4 %3, %15, %18\n"
            "global_load_dwordx4 %4, %16, %18\n"
            "global_load_dwordx4 %5, %17, %18\n"
            "global_load_dwordx4 %6, %12, %19\n"
            "global_load_dwordx4 %7, %13, %19\n"
            "global_load_dwordx4 %8, %14, %19\n"
            "global_load_dwordx4 %9, %15, %19\n"
            "global_load_dwordx4 %10, %16, %19\n"
            "global_load_dwordx4 %11, %17, %19\n"
            : "=&v"(a0), "=&v"(a1), "=&v"(a2), "=&v"(a3), "=&v"(a4), "=&v"(a5), "=&v"(c0),
              "=&v"(c1), "=&v"(c2), "=&v"(c3), "=&v"(c4), "=&v"(c5)
            : "v"(ob[0]), "v"(ob[1]), "v"(ob[2]), "v"(ob[kPB > 3 ? 3 : 0]),
              "v"(ob[kPB > 4 ? 4 : 0]), "v"(ob[kPB > 5 ? 5 : 0]), "s"(A), "s"(B)
            : "memory");
        // the prologue's loads land first, then the stream starts: issued
        // together, the loads wait behind the whole GPU's first slices
        // (decode step 225.3 -> 226.2 tok/s)
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
#pragma unroll
        for (int j = 0; j < kPreSlices; j++) issue(j);
        auto f4 = [](f32x4_t v) { return make_float4(v.x, v.y, v.z, v.w); };
        pv[0] = f4(t0), pv[1] = f4(t1), pv[2] = f4(t2), pv[3] = f4(t3), pv[4] = f4(t4),
        pv[5] = f4(t5), pv[6] = f4(t6), pv[7] = f4(t7);
        xo_in = f4(t8), xo_u = f4(t9);
        av[0] = f4(a0), av[1] = f4(a1), av[2] = f4(a2);
        bv[0] = f4(c0), bv[1] = f4(c1), bv[2] = f4(c2);
        if constexpr (kPB > 3) {
            av[kPB > 3 ? 3 : 0] = f4(a3), av[kPB > 4 ? 4 : 0] = f4(a4), av[kPB > 5 ? 5 : 0] = f4(a5);
            bv[kPB > 3 ? 3 : 0] = f4(c3), bv[kPB > 4 ? 4 : 0] = f4(c4), bv[kPB > 5 ? 5 : 0] = f4(c5);
        }
    } else if (PRO == kProEmbed) {
        const uint8_t *er = fz.embd + (size_t)fz.step[4] * nb * 18;
#pragma unroll
        for (int k = 0; k < kPB; k++) {
            const int b = min(grp + kGroups * k, nb - 1);
            const uint8_t *blk = er + b * 18;
            const uint8_t *qs = blk + 2 + ((4 * ge) & 15);
            ed[k] = f16_bits_to_f32(blk[0] | (blk[1] << 8));
            eq[k] = (uint32_t)qs[0] | ((uint32_t)qs[1] << 8) | ((uint32_t)qs[2] << 16) |
                    ((uint32_t)qs[3] << 24);
            av[k] = reinterpret_cast<const float4 *>(fz.w)[b * 8 + ge];
        }
    } else if (kTabLds) {
        // the limb table (nb·80 B, or the workgroup's slice of it;
        // L2-resident, shared by every workgroup) into LDS by DMA, 16 B per
        // lane; lanes past its end repeat the last chunk into the slack
        // after it
        const int chunks = (kSliceWG ? slice_blocks : nb) * 5;
        const uint8_t *src = reinterpret_cast<const uint8_t *>(xl + (kSliceWG ? b0 : 0));
        for (int c = wave * kWave; c < chunks; c += kRWG)
            __builtin_amdgcn_global_load_lds((gvoid_t *)(src + min(c + lane, chunks - 1) * 16),
                                             (lvoid_t *)(tab + c * 16), 16, 0, 0);
    } else if (PRO == kProX) {
        static_assert(PRO != kProX || kPB == 3, "x load layout");
        uint32_t xo[kPB];
#pragma unroll
        for (int k = 0; k < kPB; k++) xo[k] = (uint32_t)(min(grp + kGroups * k, nb - 1) * 8 + ge);
        if (fz.x_half)
            asm volatile(
                "global_load_dwordx2 %0, %3, %6\n global_load_dwordx2 %1, %4, %6\n"
                "global_load_dwordx2 %2, %5, %6"
                : "=&v"(xh0), "=&v"(xh1), "=&v"(xh2)
                : "v"(xo[0] * 8u), "v"(xo[1] * 8u), "v"(xo[2] * 8u), "s"(fz.x_raw)
                : "memory");
        else
            asm volatile(
                "global_load_dwordx4 %0, %3, %6\n global_load_dwordx4 %1, %4, %6\n"
                "global_load_dwordx4 %2, %5, %6"
                : "=&v"(xq0), "=&v"(xq1), "=&v"(xq2)
                : "v"(xo[0] * 16u), "v"(xo[1] * 16u), "v"(xo[2] * 16u), "s"(fz.x_raw)
                : "memory");
    }
    // kEpiResid: lane j holds the per-row inputs of round j
    float ex = 0.f, ewp = 0.f, ewn = 0.f;
    // (asm loads, waited for with the table behind the stream's first
    // slices: a compiler-visible load waited for there would make the
    // compiler drain the stream with it)
    if (EPI == kEpiResid) {
        int row = r0 + lane * G;
        row = lane < rows_rounds && row < n ? row : 0;
        asm volatile(
            "global_load_dword %0, %3, %4\n global_load_dword %1, %3, %5\n"
            "global_load_dword %2, %3, %6"
            : "=&v"(ex), "=&v"(ewp), "=&v"(ewn)
            : "v"((uint32_t)row * 4u), "s"(fz.x_res), "s"(fz.w_post), "s"(fz.w_next)
            : "memory");
    }

    // The prologue's inputs are waited for before the stream starts (about
    // one L2/MALL round trip), then turned into limbs while the first slices
    // are in flight.
    if (PRO != kProTable) {
        if (PRO == kProEmbed) {
#pragma unroll
            for (int k = 0; k < kPB; k++) {
                settle(ed[k]);
                settle(eq[k]);
                settle(av[k]);
            }
        }
        static_assert(EPI != kEpiResid || PRO == kProTable || kTabLds,
                      "the residual epilogue's row loads are waited for with the table");
    }

    // kProTable: this lane's limb table entries (L2-resident), loaded by asm
    // before the stream so that one wait after the stream's first slices
    // covers them and leaves the slices in flight
    f32x4_t g00 = {}, g01 = {}, g02 = {}, g03 = {}, g10 = {}, g11 = {}, g12 = {}, g13 = {},
            g20 = {}, g21 = {}, g22 = {}, g23 = {};
    float gd0 = 0.f, gd1 = 0.f, gd2 = 0.f;
    if (PRO == kProTable) {
        static_assert(NBL <= 3, "table load layout");
        const BlockLimbs *t0 = xl + b0 + min(lane, slice_blocks - 1);
        const BlockLimbs *t1 = xl + b0 + min(lane + kWave, slice_blocks - 1);
        const BlockLimbs *t2 = xl + b0 + min(lane + 2 * kWave, slice_blocks - 1);
#define SGQ_LDBLK(A, Q0, Q1, Q2, Q3, D)                                                      \
    asm volatile("global_load_dwordx4 %0, %5, off\n global_load_dwordx4 %1, %5, off offset:16\n" \
                 "global_load_dwordx4 %2, %5, off offset:32\n"                                 \
                 "global_load_dwordx4 %3, %5, off offset:48\n global_load_dword %4, %5, off offset:64" \
                 : "=&v"(Q0), "=&v"(Q1), "=&v"(Q2), "=&v"(Q3), "=&v"(D)                       \
                 : "v"(A)                                                                    \
                 : "memory")
        SGQ_LDBLK(t0, g00, g01, g02, g03, gd0);
        if (NBL > 1) SGQ_LDBLK(t1, g10, g11, g12, g13, gd1);
        if (NBL > 2) SGQ_LDBLK(t2, g20, g21, g22, g23, gd2);
#undef SGQ_LDBLK
    }
    // ---- the stream starts ------------------------------------------------
    // (unconditional: a missing round loads row 0, which keeps the number of
    // loads in flight known to the compiler's wait counting)
    if (PRO != kProNorm) {  // (kProNorm started it above)
#pragma unroll
        for (int j = 0; j < kPreSlices; j++) issue(j);
    }
    asm volatile("" ::: "memory");

    XLimbs<NBL> L;
    int boff[NBL];
#pragma unroll
    for (int i = 0; i < NBL; i++) {
        const int lb = lane + kWave * i;
        boff[i] = lb < slice_blocks ? lb * 18 - (lane & 1) * 2 : (lane & 1) * 16;
    }
    if (PRO == kProTable) {
        // the wait names the loaded registers, so no copy of them can be
        // placed ahead of it
        asm volatile("s_waitcnt vmcnt(%18)"
                     : "+v"(g00), "+v"(g01), "+v"(g02), "+v"(g03), "+v"(g10), "+v"(g11),
                       "+v"(g12), "+v"(g13), "+v"(g20), "+v"(g21), "+v"(g22), "+v"(g23),
                       "+v"(gd0), "+v"(gd1), "+v"(gd2), "+v"(ex), "+v"(ewp), "+v"(ewn)
                     : "n"(kRLoads * kPreSlices)
                     : "memory");
        // (named vectors, not an array of them: see the LDS table read below)
        auto f4g = [](f32x4_t v) { return make_float4(v.x, v.y, v.z, v.w); };
        auto putg = [&](int i, float4 q0, float4 q1, float4 q2, float4 q3, float d) {
#define SGQ_PUTG(l, Q)                                    \
    L.q[i][l][0] = __builtin_bit_cast(int, Q.x);          \
    L.q[i][l][1] = __builtin_bit_cast(int, Q.y);          \
    L.q[i][l][2] = __builtin_bit_cast(int, Q.z);          \
    L.q[i][l][3] = __builtin_bit_cast(int, Q.w);
            SGQ_PUTG(0, q0) SGQ_PUTG(1, q1) SGQ_PUTG(2, q2) SGQ_PUTG(3, q3)
#undef SGQ_PUTG
            L.d[i] = lane + kWave * i < slice_blocks ? d : 0.f;
        };
        putg(0, f4g(g00), f4g(g01), f4g(g02), f4g(g03), gd0);
        if (NBL > 1) putg(1, f4g(g10), f4g(g11), f4g(g12), f4g(g13), gd1);
        if (NBL > 2) putg(2, f4g(g20), f4g(g21), f4g(g22), f4g(g23), gd2);
    } else {
        float rb_s = 1.f;  // scale of the values that go into the table
        float ra = 0.f, s_out = 1.f;
        if (PRO == kProNorm) {
            float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int k = 0; k < kGemvMaxPartials / kWave; k++)
                if (lane + k * kWave < fz.np)  // past np: a clamped duplicate
                    acc.x += pv[k].x, acc.y += pv[k].y, acc.z += pv[k].z, acc.w += pv[k].w;
            if (wave == 0) {
                const float4 t = make_float4(wave_sum_dpp(acc.x), wave_sum_dpp(acc.y),
                                             wave_sum_dpp(acc.z), wave_sum_dpp(acc.w));
                if (lane == 0) lds_write_f32x4(scr, t);
            }
            lds_barrier();
            const float4 P4 = lds_read_f32x4(scr);
            const float K = (float)(nb * 32);
            s_out = s_pre;
            ra = 1.0f / sqrtf(P4.x / K + fz.eps);
            const float sx = s_out * s_out * (P4.w + 2.f * ra * P4.y + ra * ra * P4.z);
            const float rb = 1.0f / sqrtf(sx / K + fz.eps);
            rb_s = rb * s_out;
            uint32_t wd[kPB][kLimbs];
            float dd[kPB];
#pragma unroll
            for (int k = 0; k < kPB; k++) {
                const float4 v = make_float4((av[k].x + ra * bv[k].x) * rb_s,
                                             (av[k].y + ra * bv[k].y) * rb_s,
                                             (av[k].z + ra * bv[k].z) * rb_s,
                                             (av[k].w + ra * bv[k].w) * rb_s);
                dd[k] = limbs_words8(v, ge, wd[k]);
            }
            // branch-free: groups past the last block redo the last block
            // (same values into the same entry)
#pragma unroll
            for (int k = 0; k < kPB; k++)
                limb_words_to_lds(wd[k], dd[k], ge, tab + min(grp + kGroups * k, nb - 1) * 80);
            if (xo_on)
                reinterpret_cast<float4 *>(fz.x_out)[xo_i] =
                    make_float4(s_out * (xo_in.x + ra * xo_u.x), s_out * (xo_in.y + ra * xo_u.y),
                                s_out * (xo_in.z + ra * xo_u.z), s_out * (xo_in.w + ra * xo_u.w));
        } else if (kTabLds) {
            // the table's DMA (and the residual epilogue's row loads) were
            // issued before the stream's first slices
            asm volatile("s_waitcnt vmcnt(%3)"
                         : "+v"(ex), "+v"(ewp), "+v"(ewn)
                         : "n"(kRLoads * kPreSlices)
                         : "memory");
        } else if (PRO == kProX) {
            // the x loads were issued before the stream's first slices; the
            // wait names their registers (as the table's above)
            asm volatile("s_waitcnt vmcnt(%6)"
                         : "+v"(xq0), "+v"(xq1), "+v"(xq2), "+v"(xh0), "+v"(xh1), "+v"(xh2)
                         : "n"(kRLoads * kPreSlices)
                         : "memory");
            if (fz.x_half) {
                auto h4 = [](i32x2_t v) {
                    const uint32_t a = (uint32_t)v.x, b = (uint32_t)v.y;
                    return make_float4(f16_bits_to_f32(a & 0xffffu), f16_bits_to_f32(a >> 16),
                                       f16_bits_to_f32(b & 0xffffu), f16_bits_to_f32(b >> 16));
                };
                av[0] = h4(xh0), av[1] = h4(xh1), av[2] = h4(xh2);
            } else {
                auto f4 = [](f32x4_t v) { return make_float4(v.x, v.y, v.z, v.w); };
                av[0] = f4(xq0), av[1] = f4(xq1), av[2] = f4(xq2);
            }
            uint32_t wd[kPB][kLimbs];
            float dd[kPB];
#pragma unroll
            for (int k = 0; k < kPB; k++) dd[k] = limbs_words8(av[k], ge, wd[k]);
#pragma unroll
            for (int k = 0; k < kPB; k++)
                if (grp + kGroups * k < nb) limb_words_to_lds(wd[k], dd[k], ge, tab + (grp + kGroups * k) * 80);
        } else {  // kProEmbed
            float4 x0[kPB];
            float ss = 0.f;
            const int sh = ge < 4 ? 0 : 4;
#pragma unroll
            for (int k = 0; k < kPB; k++) {
                const int b = grp + kGroups * k;
                x0[k] = make_float4(0.f, 0.f, 0.f, 0.f);
                if (b < nb) {
                    float e[4];
#pragma unroll
                    for (int u = 0; u < 4; u++)
                        e[u] = ed[k] * (float)((int)((eq[k] >> (8 * u + sh)) & 15u) - 8) *
                               fz.embed_scale;
                    x0[k] = make_float4(e[0], e[1], e[2], e[3]);
                    ss += x0[k].x * x0[k].x + x0[k].y * x0[k].y + x0[k].z * x0[k].z +
                          x0[k].w * x0[k].w;
                    const int i4 = b * 8 + ge;
                    if (fz.x_out && i4 >= blockIdx.x * per4 && i4 < (blockIdx.x + 1) * per4)
                        reinterpret_cast<float4 *>(fz.x_out)[i4] = x0[k];
                }
            }
            const float4 t = wg_sum4<WV>(make_float4(ss, 0.f, 0.f, 0.f), scr);
            const float r = 1.0f / sqrtf(t.x / (float)(nb * 32) + fz.eps);
            uint32_t wd[kPB][kLimbs];
            float dd[kPB];
#pragma unroll
            for (int k = 0; k < kPB; k++) {
                const float4 v = make_float4(x0[k].x * r * av[k].x, x0[k].y * r * av[k].y,
                                             x0[k].z * r * av[k].z, x0[k].w * r * av[k].w);
                dd[k] = limbs_words8(v, ge, wd[k]);
            }
#pragma unroll
            for (int k = 0; k < kPB; k++)
                if (grp + kGroups * k < nb) limb_words_to_lds(wd[k], dd[k], ge, tab + (grp + kGroups * k) * 80);
        }
        lds_barrier();
        // this lane's blocks from the LDS table (a lane past the slice reads
        // the last entry and gets scale 0): all reads issued, then one wait
        // that names their registers (named variables, not an array of
        // vectors, which has read back wrong components on this compiler)
        static_assert(NBL <= 3 && kLimbs == 4, "table read layout");
        f32x4_t r00 = {}, r01 = {}, r02 = {}, r03 = {}, r10 = {}, r11 = {}, r12 = {}, r13 = {},
                r20 = {}, r21 = {}, r22 = {}, r23 = {};
        float e0 = 0.f, e1 = 0.f, e2 = 0.f;
        const int tb0 = kSliceWG ? 0 : b0, tlast = kSliceWG ? slice_blocks - 1 : nb - 1;
        const uint32_t ta0 = (uint32_t)(uintptr_t)(tab + min(tb0 + lane, tlast) * 80);
        const uint32_t ta1 = (uint32_t)(uintptr_t)(tab + min(tb0 + lane + kWave, tlast) * 80);
        const uint32_t ta2 = (uint32_t)(uintptr_t)(tab + min(tb0 + lane + 2 * kWave, tlast) * 80);
#define SGQ_RDBLK(A, Q0, Q1, Q2, Q3, D)                                                      \
    asm volatile("ds_read_b128 %0, %5\n ds_read_b128 %1, %5 offset:16\n"                      \
                 "ds_read_b128 %2, %5 offset:32\n ds_read_b128 %3, %5 offset:48\n"            \
                 "ds_read_b32 %4, %5 offset:64"                                              \
                 : "=&v"(Q0), "=&v"(Q1), "=&v"(Q2), "=&v"(Q3), "=&v"(D)                       \
                 : "v"(A)                                                                    \
                 : "memory")
        SGQ_RDBLK(ta0, r00, r01, r02, r03, e0);
        if (NBL > 1) SGQ_RDBLK(ta1, r10, r11, r12, r13, e1);
        if (NBL > 2) SGQ_RDBLK(ta2, r20, r21, r22, r23, e2);
#undef SGQ_RDBLK
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(r00), "+v"(r01), "+v"(r02), "+v"(r03), "+v"(r10), "+v"(r11),
                       "+v"(r12), "+v"(r13), "+v"(r20), "+v"(r21), "+v"(r22), "+v"(r23),
                       "+v"(e0), "+v"(e1), "+v"(e2)
                     :
                     : "memory");
        auto f4 = [](f32x4_t v) { return make_float4(v.x, v.y, v.z, v.w); };
        auto put = [&](int i, float4 q0, float4 q1, float4 q2, float4 q3, float d) {
#define SGQ_PUT(l, Q)                                     \
    L.q[i][l][0] = __builtin_bit_cast(int, Q.x);          \
    L.q[i][l][1] = __builtin_bit_cast(int, Q.y);          \
    L.q[i][l][2] = __builtin_bit_cast(int, Q.z);          \
    L.q[i][l][3] = __builtin_bit_cast(int, Q.w);
            SGQ_PUT(0, q0) SGQ_PUT(1, q1) SGQ_PUT(2, q2) SGQ_PUT(3, q3)
#undef SGQ_PUT
            L.d[i] = lane + kWave * i < slice_blocks ? d : 0.f;
        };
        put(0, f4(r00), f4(r01), f4(r02), f4(r03), e0);
        if (NBL > 1) put(1, f4(r10), f4(r11), f4(r12), f4(r13), e1);
        if (NBL > 2) put(2, f4(r20), f4(r21), f4(r22), f4(r23), e2);
    }

    // lb even: qs = bytes 2..17 of the window, d = low half of word 0;
    // lb odd: the window starts 2 bytes early, qs = words 1..4, d = high half.
    const uint32_t sel = (lane & 1) ? 0x07060504u : 0x05040302u;
    const uint32_t dshift = (lane & 1) ? 16u : 0u;
    float gate = 0.f;                              // kEpiGeglu
    float held = 0.f;                              // kEpiRows, deferred stores
    // K-slices of plain rows combined after the loop (the row-partials area
    // holds 64 rounds per wave); more rounds keep one barrier per row
    const bool defer = EPI == kEpiRows && !kSliceWG && S > 1 && !tg.split_out && rows_rounds <= kWave;
    for (int it = 0; it < rows_rounds; it++) {
        // wait for round `it`: the slices issued after it may stay in flight
        static_assert(GS >= 1 && GS <= 6, "the wait switch covers 0..5 rounds ahead");
        switch (min(GS - 1, rows_rounds - 1 - it)) {
            case 5: __builtin_amdgcn_s_waitcnt(vmcnt_imm(kRLoads * 5)); break;
            case 4: __builtin_amdgcn_s_waitcnt(vmcnt_imm(kRLoads * 4)); break;
            case 3: __builtin_amdgcn_s_waitcnt(vmcnt_imm(kRLoads * 3)); break;
            case 2: __builtin_amdgcn_s_waitcnt(vmcnt_imm(kRLoads * 2)); break;
            case 1: __builtin_amdgcn_s_waitcnt(vmcnt_imm(kRLoads * 1)); break;
            default: __builtin_amdgcn_s_waitcnt(vmcnt_imm(0)); break;
        }
        float a = 0.f;
        uint32_t wv[NBL][5];
        lds_read_blocks<NBL>(ring + (it % GS) * kRSlot, boff, wv);
        // the slot's words are in registers: refill it now, so that all
        // GS slots stream while this row computes
        if (it + GS < rows_rounds) issue(it + GS);
#pragma unroll
        for (int i = 0; i < NBL; i++) a += block_dot(wv[i], sel, dshift, L, i);
        a = wave_sum_dpp(a);
        if (EPI == kEpiGeglu) {
            if ((it & 1) == 0) {
                gate = a;
            } else if (lane == 0) {
                lds_write_u32(scr + (wave * kUnitsPerWave + (it >> 1)) * 4,
                              __builtin_bit_cast(uint32_t, gelu_tanh_g(gate) * a));
            }
            continue;
        }
        if (EPI == kEpiResid) {
            // kept for the epilogue after the loop: slot (row group, round,
            // K-slice), so the K-slices of a row need no barrier per row
            if (lane == 0)
                lds_write_u32(rows_s + ((rw * kWave + it) * S + s) * 4, __builtin_bit_cast(uint32_t, a));
            continue;
        }
        if (defer) {
            // the K-slice partials of round `it` kept for after the loop
            // (as the residual epilogue does): no barrier per row
            if (lane == 0)
                lds_write_u32(rows_s + ((rw * kWave + it) * S + s) * 4, __builtin_bit_cast(uint32_t, a));
            continue;
        }
        bool have = true;
        if (!kSliceWG && S > 1 && !(EPI == kEpiRows && tg.split_out)) {
            // one barrier per row: partials alternate between two slots, and
            // a slot is rewritten only after the next row's barrier, which
            // the reading wave reaches after its reads
            uint8_t *rb = red + (it & 1) * 4 * WV;
            if (lane == 0) lds_write_f32(rb + wave * 4, a);
            __builtin_amdgcn_s_barrier();
            have = s == 0;
            if (have) {
                float v = 0.f;
                for (int q = 0; q < S; q++) v += lds_read_f32(rb + (rw * S + q) * 4);
                a = v;
            }
        }
        // rows are stored 64 rounds at a time (lane j: round it0 + j), not
        // one store per row: a store inside the loop counts in vmcnt and
        // would make the next slot's wait cover part of a later slice
        if (have && lane == (it & (kWave - 1))) held = a;
        if ((it & (kWave - 1)) == kWave - 1 || it == rows_rounds - 1) {
            const int it0 = it & ~(kWave - 1);
            const int rowl = row_of(it0 + lane);
            if (have && lane <= (it & (kWave - 1)) && rowl < n) {
                if (S > 1 && tg.split_out)
                    tg.y[0][(size_t)s * n + rowl] = held;
                else
                    store_row(tg, rowl, held);
            }
        }
    }
    if (defer) {
        // lane j of the first wave of each row group finishes round j's row:
        // the K-slices summed in order
        lds_barrier();
        const int row = r0 + lane * G;
        if (s == 0 && lane < rows_rounds && row < n) {
            float o = 0.f;
            for (int q = 0; q < S; q++) o += lds_read_f32(rows_s + ((rw * kWave + lane) * S + q) * 4);
            store_row(tg, row, o);
        }
    }
    if (EPI == kEpiResid) {
        // lane j of the first wave of each row group finishes round j's row:
        // the K-slices summed in order, u = o·w_post, A = x·w_next,
        // B = u·w_next; then the partial sums (lanes in DPP order, waves in
        // order)
        lds_barrier();
        float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
        const int row = r0 + lane * G;
        if (s == 0 && lane < rows_rounds && row < n) {
            float o = 0.f;
            for (int q = 0; q < S; q++) o += lds_read_f32(rows_s + ((rw * kWave + lane) * S + q) * 4);
            const float u = o * ewp;
            fz.u_out[row] = u;
            fz.A_out[row] = ex * ewn;
            fz.B_out[row] = u * ewn;
            t = make_float4(o * o, ex * u, u * u, ex * ex);
        }
        t = make_float4(wave_sum_dpp(t.x), wave_sum_dpp(t.y), wave_sum_dpp(t.z), wave_sum_dpp(t.w));
        if (lane == 0) lds_write_f32x4(scr + wave * 16, t);
        lds_barrier();
        if (threadIdx.x == 0) {
            float4 r = lds_read_f32x4(scr);
#pragma unroll
            for (int w = 1; w < WV; w++) {
                const float4 q = lds_read_f32x4(scr + w * 16);
                r.x += q.x, r.y += q.y, r.z += q.z, r.w += q.w;
            }
            fz.part_out[blockIdx.x] = r;
        }
    } else if (EPI == kEpiGeglu) {
        lds_barrier();
        // 8 threads per 32-unit limb block
        if (threadIdx.x < kGegluUnits / 4) {
            const float4 h = lds_read_f32x4(scr + threadIdx.x * 16);
            limbs_block8(h, (int)threadIdx.x & 7,
                         &fz.hl[blockIdx.x * (kGegluUnits / 32) + (threadIdx.x >> 3)]);
        }
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // nothing should be left; LDS is released at exit
}

constexpr int lds_bytes(int pro, int epi, int nb) {
    return ring_lds_tab(ring_waves(pro, epi), ring_stages(pro, epi)) +
           (pro != kProTable ? nb * 80 : 0) +
           (pro == kProTableLds || pro == kProSliceLds ? kWave * 16 : 0);
}

template <int NBL, int PRO, int EPI>
int ring_attr() {
    static bool attr = false;
    if (!attr) {
        SGQ_HIP(hipFuncSetAttribute((const void *)gemv_q4_0_ring_kernel<NBL, PRO, EPI>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize,
                                    PRO == kProTableLds ? 80 * 1024
                                                        : lds_bytes(PRO, EPI, kMaxTabBlocks)));
        attr = true;
    }
    return SGQ_OK;
}

int ring_grid(int n, int S, int pro, int epi) {
    if (epi == kEpiGeglu) return n / kGegluUnits;
    const int wv = ring_waves(pro, epi);
    int grid = device_info().cus * (ring_waves_per_cu(pro, epi) / wv);
    if (pro == kProSliceLds) {  // S workgroups per row group, one per K-slice
        const int max_grid = (n + wv - 1) / wv * S;
        grid = grid > max_grid ? max_grid : grid;
        return grid / S * S;
    }
    const int P = wv / S;
    const int max_grid = (n + P - 1) / P;
    return grid > max_grid ? max_grid : grid;
}

template <int NBL, int PRO, int EPI>
int launch_ring(hipStream_t st, const GemvTargets &tg, const BlockLimbs *xl, int n, int nb, int S,
                int slice, const GemvFuse &fz) {
    if (int rc = ring_attr<NBL, PRO, EPI>()) return rc;
    const int grid = ring_grid(n, S, PRO, EPI);
    hipLaunchKernelGGL((gemv_q4_0_ring_kernel<NBL, PRO, EPI>), dim3(grid),
                       dim3(ring_waves(PRO, EPI) * kWave),
                       lds_bytes(PRO, EPI, PRO == kProSliceLds ? slice : nb), st, tg, xl, n,
                       nb, S, slice, fz);
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}

template <int NBL, int R, typename TX, typename TY>
int launch(hipStream_t st, const void *w, const TX *x, TY *y, int n, int nb, int S,
           int slice_blocks) {
    static int max_blocks_per_cu = 0;
    if (max_blocks_per_cu == 0) {
        int v = 0;
        SGQ_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, gemv_q4_0_kernel<NBL, R, TX, TY>,
                                                             kWG, 0));
        max_blocks_per_cu = v > 0 ? v : 1;
    }
    const int P = (kWG / kWave) / S;
    const int tiles = (n + P * R - 1) / (P * R);
    // Every workgroup walks the same number of tiles (no ragged last round).
    const int max_grid = device_info().cus * max_blocks_per_cu;
    const int rounds = (tiles + max_grid - 1) / max_grid;
    const int grid = (tiles + rounds - 1) / rounds;
    hipLaunchKernelGGL((gemv_q4_0_kernel<NBL, R, TX, TY>), dim3(grid), dim3(kWG), 0, st,
                       static_cast<const uint8_t *>(w), x, y, n, nb, S, slice_blocks);
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}

}  // namespace

// Streamed path geometry for K (x limbs in a table): S K-slices of `slice`
// blocks, or false when K is outside it (K % 256 != 0 or a slice > 3 KB).
static bool ring_geometry(int nb, int *S_out, int *slice_out) {
    if (nb % 8 != 0) return false;
    int S = 1;
    while (S < 4 && (nb + S - 1) / S > kRSlot / 18) S *= 2;
    int slice = (nb + S - 1) / S;
    slice = (slice + 7) & ~7;  // 144-byte multiple: 16-byte aligned slice starts
    if (slice * 18 > kRSlot || slice > 3 * kWave) return false;
    *S_out = S;
    *slice_out = slice;
    return true;
}

template <int PRO, int EPI>
static int launch_ring_nbl(hipStream_t st, const GemvTargets &tg, const BlockLimbs *xl, int n,
                           int nb, int S, int slice, const GemvFuse &fz) {
    const int nbl = (slice + kWave - 1) / kWave;
    if (nbl == 1) return launch_ring<1, PRO, EPI>(st, tg, xl, n, nb, S, slice, fz);
    if (nbl == 2) return launch_ring<2, PRO, EPI>(st, tg, xl, n, nb, S, slice, fz);
    return launch_ring<3, PRO, EPI>(st, tg, xl, n, nb, S, slice, fz);
}

static int launch_ring_any(hipStream_t st, const GemvTargets &tg, const BlockLimbs *xl, int n,
                           int nb, int S, int slice, int pro = kProTable, int epi = kEpiRows,
                           const GemvFuse &fz = GemvFuse{}) {
    if (pro == kProTable && epi == kEpiRows)
        return launch_ring_nbl<kProTable, kEpiRows>(st, tg, xl, n, nb, S, slice, fz);
    if (pro == kProNorm && epi == kEpiRows)
        return launch_ring_nbl<kProNorm, kEpiRows>(st, tg, xl, n, nb, S, slice, fz);
    if (pro == kProEmbed && epi == kEpiRows)
        return launch_ring_nbl<kProEmbed, kEpiRows>(st, tg, xl, n, nb, S, slice, fz);
    if (pro == kProX && epi == kEpiRows)
        return launch_ring_nbl<kProX, kEpiRows>(st, tg, xl, n, nb, S, slice, fz);
    if (pro == kProTableLds && epi == kEpiRows)
        return launch_ring_nbl<kProTableLds, kEpiRows>(st, tg, xl, n, nb, S, slice, fz);
    if (pro == kProTableLds && epi == kEpiResid)
        return launch_ring_nbl<kProTableLds, kEpiResid>(st, tg, xl, n, nb, S, slice, fz);
    if (pro == kProSliceLds && epi == kEpiRows)
        return launch_ring_nbl<kProSliceLds, kEpiRows>(st, tg, xl, n, nb, S, slice, fz);
    if (pro == kProNorm && epi == kEpiGeglu)
        return launch_ring_nbl<kProNorm, kEpiGeglu>(st, tg, xl, n, nb, S, slice, fz);
    if (pro == kProTable && epi == kEpiResid)
        return launch_ring_nbl<kProTable, kEpiResid>(st, tg, xl, n, nb, S, slice, fz);
    return fail(SGQ_ERR_VALIDATION, "gemv (fused): prologue %d with epilogue %d not built", pro,
                epi);
}

template <int PRO, int EPI>
static int attr_nbl() {
    int rc = ring_attr<1, PRO, EPI>();
    if (!rc) rc = ring_attr<2, PRO, EPI>();
    if (!rc) rc = ring_attr<3, PRO, EPI>();
    return rc;
}

int gemv_prepare() {
    int rc = attr_nbl<kProTable, kEpiRows>();
    if (!rc) rc = attr_nbl<kProNorm, kEpiRows>();
    if (!rc) rc = attr_nbl<kProEmbed, kEpiRows>();
    if (!rc) rc = attr_nbl<kProX, kEpiRows>();
    if (!rc) rc = attr_nbl<kProTableLds, kEpiRows>();
    if (!rc) rc = attr_nbl<kProTableLds, kEpiResid>();
    if (!rc) rc = attr_nbl<kProSliceLds, kEpiRows>();
    if (!rc) rc = attr_nbl<kProNorm, kEpiGeglu>();
    if (!rc) rc = attr_nbl<kProTable, kEpiResid>();
    return rc;
}

int gemv_fused_grid(uint32_t n, uint32_t k, int epi, int pro) {
    int S, slice;
    if (k % 256 != 0 || k == 0 || k > 65536 || !ring_geometry((int)(k / 32), &S, &slice)) return 0;
    return ring_grid((int)n, S, pro, epi);  // (the residual epilogue's launches)
}

int launch_gemv_fused(hipStream_t st, const GemvTargets &tg, const void *xl, uint32_t k, int pro,
                      int epi, const GemvFuse &fz) {
    SGQ_CHECK(k % 256 == 0 && k > 0 && k <= 65536, "gemv (fused): k=%u must be a multiple of 256", k);
    SGQ_CHECK(tg.count >= 1 && tg.count <= kGemvMaxTargets, "gemv (fused): %d targets", tg.count);
    for (int j = 0; j < tg.count; j++)
        SGQ_CHECK(((uintptr_t)tg.w[j] & 15) == 0, "gemv (fused): weights must be 16-byte aligned");
    int S, slice;
    const int nb = (int)(k / 32);
    SGQ_CHECK(ring_geometry(nb, &S, &slice), "gemv (fused): k=%u outside the streamed geometry", k);
    SGQ_CHECK(pro == kProTable || pro == kProTableLds || S == 1,
              "gemv (fused): prologues need k <= %d", kRSlot / 18 * 32);
    SGQ_CHECK(pro != kProTableLds || lds_bytes(pro, epi, nb) <= 80 * 1024,
              "gemv (fused): k=%u: the limb table does not fit two workgroups' LDS", k);
    SGQ_CHECK((pro != kProTable && pro != kProTableLds) || xl != nullptr, "gemv (fused): no limb table");
    SGQ_CHECK(pro != kProNorm || (fz.part && fz.np > 0 && fz.np <= kGemvMaxPartials && fz.A &&
                                  fz.B && (!fz.x_out || (fz.x_in && fz.u))),
              "gemv (fused): norm prologue inputs");
    SGQ_CHECK(pro != kProEmbed || (fz.embd && fz.step && fz.w), "gemv (fused): embed inputs");
    SGQ_CHECK(pro != kProX || fz.x_raw, "gemv (fused): x prologue input");
    int n = tg.end[tg.count - 1];
    if (epi == kEpiGeglu) {
        SGQ_CHECK(tg.count == 2 && tg.end[0] > 0 && tg.end[1] == 2 * tg.end[0] &&
                      tg.end[0] % kGegluUnits == 0 && fz.hl,
                  "gemv (fused): GeGLU needs gate/up of equal rows, a multiple of %d", kGegluUnits);
        n = tg.end[0];
    }
    if (epi == kEpiResid) {
        SGQ_CHECK(tg.count == 1 && !tg.split_out && tg.softcap == 0.f && fz.x_res && fz.w_post &&
                      fz.w_next && fz.u_out && fz.A_out && fz.B_out && fz.part_out,
                  "gemv (fused): residual epilogue inputs");
        const int G = ring_grid(n, S, pro, epi) * (ring_waves(pro, epi) / S);
        SGQ_CHECK((n + G - 1) / G <= kWave, "gemv (fused): more than %d rows per wave", kWave);
    }
    SGQ_CHECK(!tg.split_out || (tg.count == 1 && tg.softcap == 0.f && epi == kEpiRows),
              "gemv (fused): split output needs one target and no softcap");
    SGQ_CHECK(!tg.half_out || (!tg.split_out && epi == kEpiRows),
              "gemv (fused): f16 output needs plain row stores");
    return launch_ring_any(st, tg, static_cast<const BlockLimbs *>(xl), n, nb, S, slice, pro, epi,
                           fz);
}

namespace {
template <typename T>
int quant_limbs_t(hipStream_t st, const T *x, void *xl, uint32_t k) {
    SGQ_CHECK(k % 32 == 0 && k > 0, "quant_limbs: k=%u must be a multiple of 32", k);
    SGQ_CHECK(((uintptr_t)x & (4 * sizeof(T) - 1)) == 0 && ((uintptr_t)xl & 15) == 0,
              "quant_limbs: misaligned");
    const int nb = (int)(k / 32);
    hipLaunchKernelGGL(gemv_prep_x_kernel<T>, dim3((nb * 8 + 255) / 256), dim3(256), 0, st, x,
                       static_cast<BlockLimbs *>(xl), nb);
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}
}  // namespace

int launch_quant_limbs(hipStream_t st, const float *x, void *xl, uint32_t k) {
    return quant_limbs_t(st, x, xl, k);
}
int launch_quant_limbs(hipStream_t st, const uint16_t *x, void *xl, uint32_t k) {
    return quant_limbs_t(st, x, xl, k);
}

int gemv_slices(uint32_t k) {
    int S, slice;
    if (k % 256 != 0 || k == 0 || k > 65536 || !ring_geometry((int)(k / 32), &S, &slice)) return 0;
    return S;
}

int launch_gemv_limbs(hipStream_t st, const GemvTargets &tg, const void *xl, uint32_t k) {
    SGQ_CHECK(tg.count >= 1 && tg.count <= kGemvMaxTargets, "gemv: %d targets", tg.count);
    SGQ_CHECK(k % 256 == 0 && k > 0 && k <= 65536, "gemv (limbs): k=%u must be a multiple of 256", k);
    for (int j = 0; j < tg.count; j++) {
        SGQ_CHECK(((uintptr_t)tg.w[j] & 15) == 0, "gemv (limbs): weights must be 16-byte aligned");
        SGQ_CHECK(tg.end[j] > (j ? tg.end[j - 1] : 0), "gemv (limbs): empty target %d", j);
    }
    int S, slice;
    const int nb = (int)(k / 32);
    SGQ_CHECK(ring_geometry(nb, &S, &slice), "gemv (limbs): k=%u outside the streamed geometry", k);
    SGQ_CHECK(!tg.split_out || (tg.count == 1 && tg.softcap == 0.f),
              "gemv (limbs): split output needs one target and no softcap");
    SGQ_CHECK(!tg.half_out || !tg.split_out, "gemv (limbs): f16 output with split output");
    if (S == 1)  // one K-slice: the table goes to LDS once per workgroup
        return launch_ring_any(st, tg, static_cast<const BlockLimbs *>(xl), tg.end[tg.count - 1],
                               nb, S, slice, kProTableLds, kEpiRows);
    // split rows: one K-slice per workgroup and its part of the table in LDS
    // (K=21504, N=5376: 12.4-13.2 against 14.0-14.8 us with the S waves of
    // a row group taking the row's S slices, bit-identical partials)
    if (tg.split_out)
        return launch_ring_any(st, tg, static_cast<const BlockLimbs *>(xl), tg.end[tg.count - 1],
                               nb, S, slice, kProSliceLds, kEpiRows);
    // K-sliced rows combined in the launch: the whole table in LDS when two
    // workgroups' copies fit the CU (K <= 21504 or so; K=21504, N=5376:
    // 13.4-14.5 -> 12.8-13.0 us)
    if (lds_bytes(kProTableLds, kEpiRows, nb) <= 80 * 1024)
        return launch_ring_any(st, tg, static_cast<const BlockLimbs *>(xl), tg.end[tg.count - 1],
                               nb, S, slice, kProTableLds, kEpiRows);
    return launch_ring_any(st, tg, static_cast<const BlockLimbs *>(xl), tg.end[tg.count - 1], nb,
                           S, slice);
}

namespace {
template <typename TX, typename TY>
int gemv_q4_0_t(hipStream_t st, const void *w, const TX *x, TY *y, uint32_t n, uint32_t k,
                void *workspace) {
    SGQ_CHECK(k % 64 == 0 && k > 0, "gemv_q4_0: k=%u must be a positive multiple of 64", k);
    SGQ_CHECK(k <= 65536, "gemv_q4_0: k=%u exceeds 65536", k);
    SGQ_CHECK(n > 0 && n < (1u << 31), "gemv_q4_0: bad n=%u", n);
    SGQ_CHECK(((uintptr_t)w & 3) == 0, "gemv_q4_0: weights must be 4-byte aligned");
    SGQ_CHECK(((uintptr_t)x & (4 * sizeof(TX) - 1)) == 0, "gemv_q4_0: x must be %zu-byte aligned",
              4 * sizeof(TX));
    const int nb = (int)(k / 32);
    // Streamed path: 16-byte aligned rows (K % 256 == 0), row slices of
    // <= 170 blocks; x limbs built in the kernel's prologue (one slice per
    // row) or prepared once into the workspace (2 or 4 slices).
    int S, slice;
    if (((uintptr_t)w & 15) == 0 && workspace != nullptr && ring_geometry(nb, &S, &slice)) {
        GemvTargets tg{};
        tg.w[0] = w;
        tg.y[0] = reinterpret_cast<float *>(y);
        tg.half_out = sizeof(TY) == 2;
        tg.end[0] = (int)n;
        tg.count = 1;
        if (S == 1) {  // one K-slice: every workgroup builds the limb table itself
            GemvFuse fz{};
            fz.x_raw = x;
            fz.x_half = sizeof(TX) == 2;
            return launch_ring_any(st, tg, nullptr, (int)n, nb, S, slice, kProX, kEpiRows, fz);
        }
        int rc = launch_quant_limbs(st, x, workspace, k);
        if (rc) return rc;
        return launch_gemv_limbs(st, tg, workspace, k);
    }
    // Register path (any K % 64 == 0): each wave quantizes its own blocks.
    S = 1;
    while (S < 4 && (nb + S - 1) / S > 3 * kWave) S *= 2;
    slice = (nb + S - 1) / S;
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
}  // namespace

int launch_gemv_q4_0(hipStream_t st, const void *w, const float *x, float *y, uint32_t n,
                     uint32_t k, void *workspace) {
    return gemv_q4_0_t(st, w, x, y, n, k, workspace);
}
int launch_gemv_q4_0(hipStream_t st, const void *w, const uint16_t *x, uint16_t *y, uint32_t n,
                     uint32_t k, void *workspace) {
    return gemv_q4_0_t(st, w, x, y, n, k, workspace);
}

}  // namespace sgq

// ---------------------------------------------------------------------------
// Allocation-free form of sgq_gemv_q4_0 for callers that cannot allocate
// device memory (code under HIP graph capture, tight serving loops): the x
// limb table lives in a file-scope device array instead of a context's
// workspace.  The array's host-side name is not a device address; its
// address is looked up once per device with hipGetSymbolAddress and only
// that pointer is handed to kernels.
// ---------------------------------------------------------------------------
namespace sgq {
namespace {

constexpr size_t kNoAllocScratchBytes = kGemvWorkspace;  // limbs for K <= 65536
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
// Per device: the scratch array's address, an event recorded after each
// eager call (its completion says the array is free again) and the stream
// of that call (compared, never used).
struct ScratchState {
    void *ptr = nullptr;
    hipEvent_t done = nullptr;
    hipStream_t last = nullptr;
    bool used = false;
};
ScratchState g_scratch[kMaxDevices];

// Set-up on a device's first call: the current device's copy of `scratch`
// and its completion event.
int scratch_for_current_device(ScratchState **out) {
    int dev = -1;
    SGQ_HIP(hipGetDevice(&dev));
    SGQ_CHECK(dev >= 0 && dev < kMaxDevices, "gemv_q4_0_noalloc: device %d out of range", dev);
    ScratchState &sc = g_scratch[dev];
    if (sc.ptr == nullptr) {
        void *p = nullptr;
        SGQ_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        SGQ_CHECK(p != nullptr, "gemv_q4_0_noalloc: no device address for the scratch array");
        SGQ_HIP(hipEventCreateWithFlags(&sc.done, hipEventDisableTiming));
        sc.ptr = p;
    }
    *out = &sc;
    return SGQ_OK;
}

}  // namespace
}  // namespace sgq

extern "C" int sgq_gemv_q4_0_noalloc(void *hip_stream, const void *w, const float *x, float *y,
                                     uint32_t n, uint32_t k) {
    using namespace sgq;
    if (!w || !x || !y) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    SGQ_CHECK(k % 64 == 0 && k > 0 && k <= 65536,
              "gemv_q4_0_noalloc: k=%u must be a positive multiple of 64 and <= 65536 "
              "(the %zu-byte scratch array holds the x limbs of at most 65536 values)",
              k, kNoAllocScratchBytes);
    SGQ_CHECK((size_t)(k / 32) * sizeof(BlockLimbs) <= kNoAllocScratchBytes,
              "gemv_q4_0_noalloc: k=%u needs %zu scratch bytes, %zu available", k,
              (size_t)(k / 32) * sizeof(BlockLimbs), kNoAllocScratchBytes);
    const hipStream_t st = static_cast<hipStream_t>(hip_stream);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    ScratchState *sc = nullptr;
    if (int rc = scratch_for_current_device(&sc)) return rc;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    SGQ_HIP(hipStreamIsCapturing(st, &cap));
    const bool eager = cap == hipStreamCaptureStatusNone;
    // Calls on one stream are ordered; a call on another stream while the
    // previous eager call may still be running would share the array with it
    if (eager && sc->used && st != sc->last) {
        const hipError_t q = hipEventQuery(sc->done);
        if (q == hipErrorNotReady)
            return fail(SGQ_ERR_VALIDATION,
                        "gemv_q4_0_noalloc: the previous call, on another stream, may still be "
                        "running and shares this device's scratch array; synchronize it first");
        if (q != hipSuccess) return check_hip(q, "hipEventQuery");
    }
    if (int rc = launch_gemv_q4_0(st, w, x, y, n, k, sc->ptr)) return rc;
    if (eager) {
        SGQ_HIP(hipEventRecord(sc->done, st));
        sc->last = st;
        sc->used = true;
    }
    return SGQ_OK;
}

