// Prefill int8 MMQ GEMM for gfx950: Y[m×n] = Xq[m×k] · W[n×k]^T with the
// per-32-block rescale of the reference's gemm_q4_0_i8 family
// (crates/sg-gpu/shaders/gemm_q4_0_i8.wgsl:153-393; FFN-down variant
// gemm_q4_0_i8_bb_pfd.wgsl): for every block b,
//     Y[m,n] += (d_a[m,b] * d_w[n,b]) * f32( sum_j xq[m,32b+j] * (wq[n,32b+j]-8) )
// where the i32 block dot is exact and the scale product of two f16 values
// is exact in f32.
//
// Design:
//  * One v_mfma_i32_32x32x32_i8 is exactly one Q4_0 block (K = 32) of a
//    32×32 output tile: lane (r, h) = (lane%32, lane/32) feeds 16 K-bytes
//    [16h, 16h+16) of row/column r.  For the weights that half is the low
//    (h = 0) or high (h = 1) nibbles of the block's 16 qs bytes, so the
//    logical K order of q4_0.rs:31-42 falls out with no shuffle.
//  * Workgroup = 4 waves (2×2), tile 128×128, each wave 64×64 = 2×2 MFMA
//    tiles.  A K-stage is 4 blocks (128 K): activations (int8) and weights
//    (unpacked once per workgroup to int8 q-8 by the loading thread) go to
//    LDS, rows padded to 144 B so the 16-byte fragment reads of 8 lanes hit
//    32 distinct banks.  Double-buffered: stage s+1's global loads are in
//    flight while stage s computes; one barrier per stage.
//  * Rescale: the scale products d_a·d_w of a 32×32 tile come from the
//    matrix cores too — one v_mfma_f32_32x32x8_f16 whose only non-zero K
//    term is (d_a[row], d_w[col]) gives the exact outer product (f16·f16 is
//    exact in f32) in the accumulator layout of the int8 MFMA (the K=8 form
//    costs the matrix cores less than the K=16 one: config 2 571 -> 620-627
//    TOP/s, M = 4096 750 -> 786, with half the operand registers).  The VALU is
//    left with one cvt and one FMA per output element and block, and that —
//    not the MFMA — still bounds the kernel (a wave64 VALU op costs 4
//    cycles against 32 for an MFMA covering 1024 elements).
//  * Tile order is XCD-aware: consecutive workgroup ids land on different
//    XCDs (each with its own L2), so ids are remapped so that every XCD
//    walks a contiguous range of N-tiles with all their M-tiles, and a
//    weight strip is fetched from HBM once per XCD; with many M-tiles the
//    XCD takes them 8 at a time across its N-tiles.
//  * Split-K (slices of the block range, factor 1/2/4/8) writes fp32
//    partial tiles; a second kernel sums them in fixed order s = 0..S-1.
#include "sgq_internal.h"

namespace sgq {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, KB = 4;   // tile rows, cols, blocks per stage
constexpr int ROWB = KB * 32 + 16;          // padded LDS row bytes (144)
constexpr int kMWG = 256;
#ifndef SGQ_MMQ_WG_PER_CU
#define SGQ_MMQ_WG_PER_CU 2
#endif

struct Stage {
    int8_t a[BM * ROWB];      // activations, [row][k]
    int8_t b[BN * ROWB];      // weights (q-8), [col][k]
    uint16_t da[BM][KB];      // activation scales (f16 bits), [row][block]
    uint16_t dw[BN][KB];      // weight scales (f16 bits), [col][block]
};

__device__ __forceinline__ uint32_t unpack_lo(uint32_t q) {
    return ((q & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;  // nibble-8 as int8
}
__device__ __forceinline__ uint32_t unpack_hi(uint32_t q) {
    return (((q >> 4) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
}

struct Prefetch {
    v4i a[4];          // 64 activation bytes: row = tid/2, k-half = tid%2 (native
                       // vectors: HIP's uint4 is a struct, copied through scratch)
    uint32_t w[9];     // two Q4_0 blocks (36 bytes): col = tid/2, blocks 2*(tid%2)+{0,1}
    uint16_t da[4];    // threads < 128: 4 block scales of row tid
};

__device__ __forceinline__ void load_stage(Prefetch &pf, const int8_t *__restrict__ xq,
                                           const uint16_t *__restrict__ xs,
                                           const uint8_t *__restrict__ W, int m, int n, int k,
                                           int nb, int m0, int n0, int b0, int b_end) {
    const int t = threadIdx.x;
    {   // activations: 64 contiguous bytes
        const int row = t >> 1, half = t & 1;
        const int gm = m0 + row;
        const int kb = b0 * 32 + half * 64;  // first K index of this thread's 64 bytes
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int kk = kb + i * 16;
            if (gm < m && kk < b_end * 32)
                pf.a[i] = *reinterpret_cast<const v4i *>(xq + (size_t)gm * k + kk);
            else
                pf.a[i] = v4i{0, 0, 0, 0};
        }
    }
    {   // weights: two blocks, 36 bytes, 4-aligned (b0 and the pair index are even)
        const int col = t >> 1, pair = t & 1;
        const int gn = n0 + col;
        const int b = b0 + 2 * pair;
        if (gn < n && b < b_end) {
            const uint32_t *src =
                reinterpret_cast<const uint32_t *>(W + ((size_t)gn * nb + b) * 18);
            const bool two = b + 1 < b_end;
#pragma unroll
            for (int j = 0; j < 9; j++)
                pf.w[j] = (j < 5 || two) ? src[j] : 0u;
        } else {
#pragma unroll
            for (int j = 0; j < 9; j++) pf.w[j] = 0u;
        }
    }
    if (t < BM) {
        const int gm = m0 + t;
#pragma unroll
        for (int i = 0; i < KB; i++) {
            const int b = b0 + i;
            pf.da[i] = (gm < m && b < b_end) ? xs[(size_t)gm * nb + b] : (uint16_t)0;
        }
    }
}

// Aligned shapes (m % BM == 0, n % BN == 0, nb % KB == 0): no bounds
// checks; each thread's three sources are base pointers that advance by a
// constant per stage, and the 4 block scales of a row are one 8-byte load.
struct AlignedSrc {
    const int8_t *a;      // row t/2 of the tile, byte 64·(t%2) of block 0
    const uint32_t *w;    // column t/2, block 2·(t%2)
    const uint2 *da;      // row t (t < BM): scales of blocks 0..3
};

__device__ __forceinline__ AlignedSrc aligned_src(const int8_t *__restrict__ xq,
                                                  const uint16_t *__restrict__ xs,
                                                  const uint8_t *__restrict__ W, int k, int nb,
                                                  int m0, int n0) {
    const int t = threadIdx.x;
    AlignedSrc s;
    s.a = xq + (size_t)(m0 + (t >> 1)) * k + (t & 1) * 64;
    s.w = reinterpret_cast<const uint32_t *>(W + ((size_t)(n0 + (t >> 1)) * nb + 2 * (t & 1)) * 18);
    s.da = reinterpret_cast<const uint2 *>(xs + (size_t)(m0 + (t & (BM - 1))) * nb);
    return s;
}

__device__ __forceinline__ void load_stage_al(Prefetch &pf, const AlignedSrc &src, int b0) {
    const v4i *a = reinterpret_cast<const v4i *>(src.a + b0 * 32);
#pragma unroll
    for (int i = 0; i < 4; i++) pf.a[i] = a[i];
    const uint32_t *w = src.w + (b0 * 18) / 4;  // b0 % 4 == 0: 72 B per stage
    // plain loads: a weight strip serves every M-tile of its column group
    // (from L2); with the nontemporal hint config 2 ran at 526-530 against
    // 573-579 TOP/s and M = 4096 at 676 against 758-763
#pragma unroll
    for (int j = 0; j < 9; j++) pf.w[j] = w[j];
    if (threadIdx.x < BM) {
        const uint2 d = src.da[b0 / 4];
        pf.da[0] = (uint16_t)(d.x & 0xffffu);
        pf.da[1] = (uint16_t)(d.x >> 16);
        pf.da[2] = (uint16_t)(d.y & 0xffffu);
        pf.da[3] = (uint16_t)(d.y >> 16);
    }
}

__device__ __forceinline__ void store_stage(const Prefetch &pf, Stage &S) {
    const int t = threadIdx.x;
    {
        const int row = t >> 1, half = t & 1;
#pragma unroll
        for (int i = 0; i < 4; i++)
            *reinterpret_cast<v4i *>(&S.a[row * ROWB + half * 64 + i * 16]) = pf.a[i];
    }
    {
        const int col = t >> 1, pair = t & 1;
        // Block A: d in low half of w0, qs bytes = w0.hi .. w4.lo
        uint32_t qa[4], qb[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            qa[j] = __builtin_amdgcn_alignbyte(pf.w[j + 1], pf.w[j], 2);
            qb[j] = pf.w[5 + j];
        }
        int8_t *dst = &S.b[col * ROWB + pair * 64];
        uint4 lo, hi;
        lo = make_uint4(unpack_lo(qa[0]), unpack_lo(qa[1]), unpack_lo(qa[2]), unpack_lo(qa[3]));
        hi = make_uint4(unpack_hi(qa[0]), unpack_hi(qa[1]), unpack_hi(qa[2]), unpack_hi(qa[3]));
        *reinterpret_cast<uint4 *>(dst) = lo;
        *reinterpret_cast<uint4 *>(dst + 16) = hi;
        lo = make_uint4(unpack_lo(qb[0]), unpack_lo(qb[1]), unpack_lo(qb[2]), unpack_lo(qb[3]));
        hi = make_uint4(unpack_hi(qb[0]), unpack_hi(qb[1]), unpack_hi(qb[2]), unpack_hi(qb[3]));
        *reinterpret_cast<uint4 *>(dst + 32) = lo;
        *reinterpret_cast<uint4 *>(dst + 48) = hi;
        // the two blocks' scales: low half of word 0, high half of word 4
        *reinterpret_cast<uint32_t *>(&S.dw[col][2 * pair]) =
            (pf.w[0] & 0xffffu) | (pf.w[4] & 0xffff0000u);
    }
    if (t < BM) {
#pragma unroll
        for (int i = 0; i < KB; i++) S.da[t][i] = pf.da[i];
    }
}

// Tile of the jl-th workgroup slot of XCD x (workgroup b runs on XCD b % 8,
// jl = b / 8; tiles % 8 == 0, else x = 0 and jl = b).  XCD-aware order:
// every XCD walks a contiguous range of the tiles.
constexpr int kXcds = 8, kGroupM = 8;
__device__ __forceinline__ void mmq_tile(int x, int jl, int mt, int nt, int *tm, int *tn) {
    const int tiles = mt * nt;
    if (nt % kXcds == 0 && mt % kGroupM == 0) {
        // XCD x owns N-tiles [x·nt/8, (x+1)·nt/8) with every M-tile, walked in
        // groups of 8 M-tiles across all its N-tiles: the XCD's resident
        // tiles (64) then share 8 activation panels and 8 weight strips in
        // its L2 instead of all M-tiles' panels and 2 strips (M = 4096: 646
        // -> 656 TOP/s, the 4096-token prefill +1.3-2%; 16 M-tiles per group
        // measured as the plain order)
        const int ntx = nt / kXcds, gs = kGroupM * ntx;
        const int g = jl / gs, r = jl % gs;
        *tm = g * kGroupM + r % kGroupM;
        *tn = x * ntx + r / kGroupM;
    } else if (tiles % kXcds == 0 && mt % kGroupM == 0) {
        // N-tiles not a multiple of 8: the same grouped order over the whole
        // grid, each XCD a contiguous eighth of it (the down projection at
        // M = 4096, K = 21504: 614-627 -> 634-642 TOP/s)
        const int j = x * (tiles / kXcds) + jl, gs = kGroupM * nt;
        const int g = j / gs, r = j % gs;
        *tm = g * kGroupM + r % kGroupM;
        *tn = r / kGroupM;
    } else {
        const int id = tiles % kXcds == 0 ? x * (tiles / kXcds) + jl : jl;
        *tn = id / mt, *tm = id % mt;
    }
}

// Tail split (split = 1 only): when the tiles are more than whole rounds of
// the resident workgroups, each XCD computes its first tail_fx tiles whole
// and splits each of its remaining tiles over K into tail_st parts, one
// workgroup each, so the last round is full; the parts go to tailp as
// 128×128 fp32 tiles (slot = x·(tiles/8 − tail_fx) + tail tile, part) and
// mmq_tail_reduce_kernel sums them in part order.
struct TailSplit {
    int fx, st;    // whole tiles per XCD, parts per tail tile (0: off)
    float *part;
};

// HOUT: the output is f16 (uint16_t bits, each sum rounded to nearest even:
// the reference's y binding, gemm_q4_0_i8.wgsl:63); else fp32.  TAIL: the
// tail split is built in (a separate kernel, so the others keep their code).
template <bool AL, bool HOUT, bool TAIL = false>
__global__ __launch_bounds__(kMWG, SGQ_MMQ_WG_PER_CU) void mmq_kernel(const uint8_t *__restrict__ W,
                                                      const int8_t *__restrict__ xq,
                                                      const uint16_t *__restrict__ xs,
                                                      void *__restrict__ out_, int m, int n,
                                                      int k, int mt, int nt, int split,
                                                      TailSplit ts) {
    extern __shared__ __align__(16) uint8_t smem[];
    Stage *stages = reinterpret_cast<Stage *>(smem);

    // XCD-aware tile order (see header).
    const int tiles = mt * nt;
    const bool by_xcd = tiles % kXcds == 0;
    const int x = by_xcd ? (int)(blockIdx.x % kXcds) : 0;
    int jl = by_xcd ? (int)(blockIdx.x / kXcds) : (int)blockIdx.x;
    int z = blockIdx.y;
    int tail_slot = -1;
    if (TAIL && jl >= ts.fx) {
        const int k2 = jl - ts.fx, lx = tiles / kXcds - ts.fx;
        jl = ts.fx + k2 / ts.st;
        z = k2 % ts.st;
        split = ts.st;
        tail_slot = x * lx + k2 / ts.st;
    }
    int tm, tn;
    mmq_tile(x, jl, mt, nt, &tm, &tn);
    const int m0 = tm * BM, n0 = tn * BN;

    const int nb = k / 32;
    const int b_beg = (int)((long)nb * z / split) & ~(KB - 1);
    const int b_end = z + 1 == split ? nb : ((int)((long)nb * (z + 1) / split) & ~(KB - 1));
    const int n_stages = (b_end - b_beg + KB - 1) / KB;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int r = lane & 31, h = lane >> 5;

    float acc[2][2][16];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
            for (int i = 0; i < 16; i++) acc[a][b][i] = 0.f;

    // register prefetch one stage ahead: stage s+1's global loads are in
    // flight while stage s computes (four blocks of MFMAs and rescales),
    // then go to the other LDS buffer
    Prefetch pf;
    AlignedSrc src{};
    if (AL) src = aligned_src(xq, xs, W, k, nb, m0, n0);
    auto load = [&](Prefetch &p, int b0) {
        if (AL)
            load_stage_al(p, src, b0);
        else
            load_stage(p, xq, xs, W, m, n, k, nb, m0, n0, b0, b_end);
    };
    if (n_stages > 0) {
        load(pf, b_beg);
        store_stage(pf, stages[0]);
    }
    __syncthreads();

    // LDS operands of one block: int8 fragments of the wave's two row and
    // two column tiles
    struct Ops {
        v4i af[2], bf[2];
    };
    // the f16 scale bits of the wave's two row and two column tiles for the
    // stage's four blocks (two per word), read once per stage; zero in the
    // lanes (h = 1) whose K terms of the scale MFMA are zero
    uint2 sa4[2], sb4[2];
    auto ld_scales = [&](const Stage &S) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const uint2 a = *reinterpret_cast<const uint2 *>(&S.da[wm * 64 + i * 32 + r][0]);
            const uint2 b = *reinterpret_cast<const uint2 *>(&S.dw[wn * 64 + i * 32 + r][0]);
            sa4[i] = h == 0 ? a : make_uint2(0u, 0u);
            sb4[i] = h == 0 ? b : make_uint2(0u, 0u);
        }
    };
    auto ld_ops = [&](const Stage &S, int blk, Ops &o) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            o.af[i] = *reinterpret_cast<const v4i *>(
                &S.a[(wm * 64 + i * 32 + r) * ROWB + blk * 32 + h * 16]);
            o.bf[i] = *reinterpret_cast<const v4i *>(
                &S.b[(wn * 64 + i * 32 + r) * ROWB + blk * 32 + h * 16]);
        }
    };
    // Scale operands: lane (r, h = 0) holds K term 0 = d of its row (A) /
    // column (B); every other K term is zero.  Kept across blocks, so only
    // the first word of each is rewritten per block (the zero words stay in
    // their registers).
    v2i asv[2] = {}, bsv[2] = {};
    // One block on the wave's 2×2 tiles.  Tile t's MFMAs are issued before
    // tile t-1's rescale, so the matrix cores work while the VALU converts.
    // wa / wb: the scale words of the block pair (blocks 2p, 2p + 1), hi =
    // the pair's second block
    auto block = [&](const Ops &o, const uint32_t (&wa)[2], const uint32_t (&wb)[2], bool hi) {
        h4 as[2], bs[2];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            asv[i][0] = (int)(hi ? wa[i] >> 16 : wa[i] & 0xffffu);
            bsv[i][0] = (int)(hi ? wb[i] >> 16 : wb[i] & 0xffffu);
            as[i] = __builtin_bit_cast(h4, asv[i]);
            bs[i] = __builtin_bit_cast(h4, bsv[i]);
        }
        v16i d[2];
        f32x16 sc[2];
        const v16i zero = {};
        const f32x16 fzero = {};
#pragma unroll
        for (int t = 0; t <= 4; t++) {
            if (t < 4) {
                const int i = t >> 1, j = t & 1;
                d[t & 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.af[i], o.bf[j], zero, 0, 0, 0);
                sc[t & 1] = __builtin_amdgcn_mfma_f32_32x32x8f16(as[i], bs[j], fzero, 0, 0, 0);
            }
            if (t > 0) {
                const int u = t - 1, i = u >> 1, j = u & 1;
#pragma unroll
                for (int q = 0; q < 16; q++)
                    acc[i][j][q] = __builtin_fmaf((float)d[u & 1][q], sc[u & 1][q], acc[i][j][q]);
            }
        }
    };
    auto step = [&](int s) {
        if (s + 1 < n_stages) load(pf, b_beg + (s + 1) * KB);
        const Stage &S = stages[s & 1];
        // the next block's LDS operands load while this block computes
        // (two blocks per iteration, so both operand sets keep fixed registers)
        Ops o0, o1;
        ld_ops(S, 0, o0);
        ld_scales(S);
#pragma unroll 1
        for (int bp = 0; bp < KB; bp += 2) {
            ld_ops(S, bp + 1, o1);
            asm volatile("" ::: "memory");  // keeps the reads above the block's MFMAs
            uint32_t wa[2], wb[2];
#pragma unroll
            for (int i = 0; i < 2; i++) {
                wa[i] = bp == 0 ? sa4[i].x : sa4[i].y;
                wb[i] = bp == 0 ? sb4[i].x : sb4[i].y;
            }
            block(o0, wa, wb, false);
            ld_ops(S, min(bp + 2, KB - 1), o0);
            asm volatile("" ::: "memory");
            block(o1, wa, wb, true);
        }
        if (s + 1 < n_stages) store_stage(pf, stages[(s + 1) & 1]);
        __syncthreads();
    };
    for (int s = 0; s < n_stages; s++) step(s);

    float *dst = static_cast<float *>(out_) + (size_t)z * m * n;
    uint16_t *dsth = static_cast<uint16_t *>(out_);
    if (TAIL && tail_slot >= 0) {  // a K-part of a tail tile: tile-local rows of 128
        float *tp = ts.part + ((size_t)tail_slot * ts.st + z) * (BM * BN);
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int q = 0; q < 16; q++)
                    tp[(wm * 64 + i * 32 + 8 * (q / 4) + 4 * h + (q % 4)) * BN + wn * 64 + j * 32 +
                       r] = acc[i][j][q];
        return;
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int col = n0 + wn * 64 + j * 32 + r;
            if (!AL && col >= n) continue;
#pragma unroll
            for (int q = 0; q < 16; q++) {
                const int row = m0 + wm * 64 + i * 32 + 8 * (q / 4) + 4 * h + (q % 4);
                if (AL || row < m) {
                    if (HOUT)
                        dsth[(size_t)row * n + col] = f32_to_f16_bits(acc[i][j][q]);
                    else
                        dst[(size_t)row * n + col] = acc[i][j][q];
                }
            }
        }
}

__global__ void splitk_reduce_kernel(const float4 *__restrict__ part, float4 *__restrict__ y,
                                     uint64_t n4, int split) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4;
         i += (uint64_t)gridDim.x * blockDim.x) {
        float4 a = part[i];
        for (int s = 1; s < split; s++) {
            const float4 b = part[(uint64_t)s * n4 + i];
            a.x += b.x;
            a.y += b.y;
            a.z += b.z;
            a.w += b.w;
        }
        y[i] = a;
    }
}

// y of the tail tiles: the tail_st parts summed in part order (float4 per
// thread, one 128×128 tile per 16 workgroups of 256 threads).
__global__ __launch_bounds__(256) void mmq_tail_reduce_kernel(TailSplit ts, float *__restrict__ y,
                                                              int n, int mt, int nt) {
    const int tiles = mt * nt, lx = tiles / kXcds - ts.fx;
    const int slot = blockIdx.x / 16;  // tail tile
    const int e = (blockIdx.x % 16) * 256 + threadIdx.x;  // float4 within the tile
    const int x = slot / lx, jl = ts.fx + slot % lx;
    int tm, tn;
    mmq_tile(x, jl, mt, nt, &tm, &tn);
    const float4 *p = reinterpret_cast<const float4 *>(ts.part + (size_t)slot * ts.st * (BM * BN));
    float4 a = p[e];
    for (int zz = 1; zz < ts.st; zz++) {
        const float4 b = p[(size_t)zz * (BM * BN / 4) + e];
        a.x += b.x;
        a.y += b.y;
        a.z += b.z;
        a.w += b.w;
    }
    const int row = e / (BN / 4), c4 = e % (BN / 4);
    *reinterpret_cast<float4 *>(y + (size_t)(tm * BM + row) * n + tn * BN + 4 * c4) = a;
}

}  // namespace

namespace {
template <bool HOUT>
int gemm_t(hipStream_t st, const void *w, const int8_t *xq, const uint16_t *xs, void *y,
           uint32_t m, uint32_t n, uint32_t k, uint32_t split_k, float *partials) {
    SGQ_CHECK(k % 64 == 0 && k > 0, "gemm_q4_0_q8: k=%u must be a positive multiple of 64", k);
    SGQ_CHECK(m > 0 && n > 0, "gemm_q4_0_q8: empty shape");
    SGQ_CHECK(split_k == 1 || split_k == 2 || split_k == 4 || split_k == 8,
              "gemm_q4_0_q8: split_k=%u not in {1,2,4,8}", split_k);
    SGQ_CHECK(split_k == 1 || partials != nullptr, "gemm_q4_0_q8: split_k>1 needs partials");
    SGQ_CHECK(!HOUT || split_k == 1, "gemm_q4_0_q8: f16 output is not built with split-K");
    SGQ_CHECK(k % 16 == 0 && ((uintptr_t)xq & 15) == 0, "gemm_q4_0_q8: xq must be 16-byte aligned");
    SGQ_CHECK(((uintptr_t)w & 3) == 0, "gemm_q4_0_q8: weights must be 4-byte aligned");
    SGQ_CHECK((uint64_t)m * n < (1ull << 31) * 4, "gemm_q4_0_q8: output too large");
    SGQ_CHECK(split_k == 1 || (m * (uint64_t)n) % 4 == 0, "gemm_q4_0_q8: m*n must be a multiple of 4 for split-K");
    static bool attr = false;
    const size_t lds = 2 * sizeof(Stage);
    if (!attr) {
        SGQ_HIP(hipFuncSetAttribute((const void *)mmq_kernel<false, HOUT>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        SGQ_HIP(hipFuncSetAttribute((const void *)mmq_kernel<true, HOUT>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        SGQ_HIP(hipFuncSetAttribute((const void *)mmq_kernel<true, false, true>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        attr = true;
    }
    const int mt = (int)((m + BM - 1) / BM), nt = (int)((n + BN - 1) / BN);
    void *dst = split_k == 1 ? y : static_cast<void *>(partials);
    // every split's block range is a multiple of KB when nb is (the split
    // bounds are rounded down to KB)
    const bool aligned = m % BM == 0 && n % BN == 0 && (k / 32) % KB == 0 &&
                         ((uintptr_t)xs & 7) == 0;
    // Tail split: aligned fp32 output, split_k = 1 and a partials buffer
    // (m·n floats always suffice: the parts are at most one round of tiles)
    TailSplit ts{0, 0, partials};
    const int tiles = mt * nt, slots_x = device_info().cus * SGQ_MMQ_WG_PER_CU / kXcds;
    // (only below two whole rounds: at M = 4096, N = 21504, with a tail of
    // half a round split in 2, the launch measured 1.3% slower)
    if (aligned && !HOUT && split_k == 1 && partials != nullptr && tiles % kXcds == 0 &&
        slots_x > 0 && tiles / kXcds > slots_x && tiles / kXcds < 2 * slots_x) {
        const int tx = tiles / kXcds, fx = tx / slots_x * slots_x, lx = tx - fx;
        const int parts = lx > 0 ? std::min(4, slots_x / lx) : 0;
        if (parts >= 2 && (int)(k / 32) / parts >= 4 * KB) ts.fx = fx, ts.st = parts;
    }
    const int grid_x = ts.st ? kXcds * (ts.fx + (tiles / kXcds - ts.fx) * ts.st) : tiles;
    if (ts.st)
        hipLaunchKernelGGL((mmq_kernel<true, false, true>), dim3(grid_x, split_k), dim3(kMWG), lds,
                           st, static_cast<const uint8_t *>(w), xq, xs, dst, (int)m, (int)n,
                           (int)k, mt, nt, (int)split_k, ts);
    else if (aligned)
        hipLaunchKernelGGL((mmq_kernel<true, HOUT>), dim3(grid_x, split_k), dim3(kMWG), lds, st,
                           static_cast<const uint8_t *>(w), xq, xs, dst, (int)m, (int)n, (int)k,
                           mt, nt, (int)split_k, ts);
    else
        hipLaunchKernelGGL((mmq_kernel<false, HOUT>), dim3(grid_x, split_k), dim3(kMWG), lds, st,
                           static_cast<const uint8_t *>(w), xq, xs, dst, (int)m, (int)n, (int)k,
                           mt, nt, (int)split_k, ts);
    SGQ_HIP(hipGetLastError());
    if (ts.st) {
        const int tail_tiles = kXcds * (tiles / kXcds - ts.fx);
        hipLaunchKernelGGL(mmq_tail_reduce_kernel, dim3(tail_tiles * 16), dim3(256), 0, st, ts,
                           static_cast<float *>(y), (int)n, mt, nt);
        SGQ_HIP(hipGetLastError());
    }
    if (split_k > 1) {
        const uint64_t n4 = (uint64_t)m * n / 4;
        uint64_t g = (n4 + 255) / 256;
        if (g > (uint64_t)device_info().cus * 8) g = (uint64_t)device_info().cus * 8;
        hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)g), dim3(256), 0, st,
                           reinterpret_cast<const float4 *>(partials),
                           static_cast<float4 *>(y), n4, (int)split_k);
        SGQ_HIP(hipGetLastError());
    }
    return SGQ_OK;
}

}  // namespace

int launch_gemm_q4_0_q8(hipStream_t st, const void *w, const int8_t *xq, const uint16_t *xs,
                        float *y, uint32_t m, uint32_t n, uint32_t k, uint32_t split_k,
                        float *partials) {
    return gemm_t<false>(st, w, xq, xs, y, m, n, k, split_k, partials);
}
int launch_gemm_q4_0_q8(hipStream_t st, const void *w, const int8_t *xq, const uint16_t *xs,
                        uint16_t *y, uint32_t m, uint32_t n, uint32_t k) {
    return gemm_t<true>(st, w, xq, xs, y, m, n, k, 1, nullptr);
}

}  // namespace sgq
