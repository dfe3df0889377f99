// Prefill flash attention over a Q8_0 KV cache for gfx950 (causal, optional
// sliding window).
//
// Semantics: attn_prefill_global_flash_* / attn_prefill_sliding_ring
// (crates/sg-gpu/shaders/attn_prefill_global_flash_sp_q8.wgsl:65-183,
// attn_prefill_sliding_ring.wgsl:53-152): query i of the chunk sits at
// position q0+i and attends keys p with p <= q0+i and, with a window W,
// p > q0+i-W; out = softmax(scale · q·kᵀ)·v per query head, GQA head h
// reading kv head h/(n_q/n_kv).  K and V come from Q8_0 pages (int8
// [row × n_kv × 128] + f16 scales per 32) in two ranges, as in
// attn_prefill_sliding_ring.wgsl: keys before q0 from the cache (slot =
// position, or position mod ring for a sliding ring), keys from q0 on from
// the chunk's own pages (row = position - q0) when those are given, else
// from the cache too.  They are dequantized to f16 as in the reference's
// _sp_q8 variant; P is rounded to f16 for PV, as in the reference.  The
// head_dim-256/512 kernel (attn_prefill_wide_kernel, below) also reads the
// reference's other page formats: f16 K/V, int8 q with Q8_0 K, int8 V with
// key-blocked scales (PfFmt).
//
// Design (MFMA-bound: 4·hd flops per query-key pair against 2·hd·1 B of
// K/V per key per query tile):
//  * Workgroup = 4 waves per query head of one kv head (GQA: 8 waves for
//    two) = 128 queries of each.  K and V are dequantized by all threads
//    into LDS tiles of kLT keys (K as [key][dim], V transposed as
//    [dim][key], rows padded), used by all of the workgroup's queries, and
//    computed as 64-key tiles: one barrier pair per LDS tile.
//  * Each wave computes Sᵀ = K·Qᵀ for its 32 queries with
//    v_mfma_f32_32x32x16_f16 (8 per 32 keys): in that layout lane l owns
//    query column l%32, so the online softmax needs one cross-half shuffle,
//    and the probabilities are already in the B-operand layout of
//    Oᵀ = Vᵀ·Pᵀ (4 dim blocks × 2 key chunks of 16 per 32 keys) — no LDS
//    round trip for P.  Oᵀ stays in registers (4 × 16 fp32 per lane).
//  * Causal: tiles run heaviest-first (last query tile first); the head
//    groups are spread over the XCDs so each XCD's L2 keeps its K/V pages.
#include "sgq_internal.h"

namespace sgq {
namespace {

#ifndef SGQ_PREFILL_PAIR_HEADS
#define SGQ_PREFILL_PAIR_HEADS 1
#endif
constexpr bool kPrefillPairHeads = SGQ_PREFILL_PAIR_HEADS;  // two query heads per workgroup
constexpr int kHD = 128;
constexpr int kQT = 128;           // queries per workgroup (4 waves × 32)
constexpr int kKT = 64;            // keys per compute tile
#ifndef SGQ_PF_SUBTILES
#define SGQ_PF_SUBTILES 4
#endif
constexpr int kSub = SGQ_PF_SUBTILES;  // compute tiles per LDS tile (per barrier pair)
constexpr int kLT = kSub * kKT;       // keys per LDS tile
constexpr int kKRow = kHD + 8;     // K tile row in LDS (f16), padded
// Vᵀ tile row in LDS (f16): 130 dwords, so the 32 rows one PV read spans
// start 2 banks apart (conflict-free 8-byte reads).  Columns are swizzled in
// units of 4 keys (8 bytes): unit u of a row of dim block b is stored at
// u ^ 8b, so the four blocks' row writes of one key range (the rows 32b + j
// share their bank offset) land on disjoint banks.
constexpr int kVRow = kLT + 4;
__device__ __forceinline__ int vt_col(int key, int b) { return ((key >> 2) ^ (8 * b)) * 4 + (key & 3); }
constexpr float kNegBig = -3.0e38f;

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int v4i_p __attribute__((ext_vector_type(4)));
typedef int v16i_p __attribute__((ext_vector_type(16)));

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// Bytes (sel picks two of the four) of a word of int8 quants -> their exact
// f16 values: 1024 + (q + 128) by a permute against 0x64, then -1152.
__device__ __forceinline__ h2 i8_pair_f16(uint32_t w, uint32_t sel) {
    const h2 bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    return __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, w ^ 0x80808080u, sel)) + bias;
}

// A pointer pinned in scalar registers: stops the compiler from turning a
// per-lane choice between two kernel-argument pointers into a vector load
// of the chosen pointer (a dependent load before every K/V fetch).
template <typename T>
__device__ __forceinline__ T *sgpr_ptr(T *p) {
    asm volatile("" : "+s"(p));
    return p;
}
// A load through the global address space (global_load, counted by vmcnt
// only; the generic pointer sgpr_ptr returns would give a flat load, which
// every LDS wait also waits for).
template <typename T>
__device__ __forceinline__ T gload(const T *p) {
    return *(const __attribute__((address_space(1))) T *)(p);
}

struct KvSource {
    const int8_t *kq, *vq;      // cache pages
    const uint16_t *ks, *vs;
    int ring;                   // ring slots (0: linear cache)
    const int8_t *ckq, *cvq;    // the chunk's pages (rows = position - q0), or null
    const uint16_t *cks, *cvs;
};

// IPV (int8 PV, attn_prefill_global_flash_sp_ipv.wgsl): V stays int8 in LDS
// (transposed, [dim][key]) with its key-blocked scales, P is quantized per
// (query, 32-key block) and Oᵀ += Vᵀ·Pᵀ runs as one v_mfma_i32_32x32x32_i8
// per block and 32 dims, rescaled by p_scale ⊗ v_scale; linear cache,
// causal, no window (tiles start at key 0, so every 32-key MFMA block is a
// V scale block).
constexpr int kVRowB = kLT + 16;   // int8 Vᵀ tile row (IPV), padded
static_assert(kHD * kVRowB + (kLT / 32) * kHD * 4 <= kHD * kVRow * 2, "IPV tiles fit the Vᵀ LDS");

template <int HPW, bool IPV = false>
__global__ __launch_bounds__(256 * HPW) void attn_prefill_kernel(
    const float *__restrict__ q, KvSource src, float *__restrict__ out, int n_tok, int q0,
    int n_q, int n_kv, int window, float scale, int qtiles, const uint32_t *__restrict__ step) {
    if (step) q0 = (int)step[3];
    // Vᵀ first: its reads (32 per compute tile) then address with immediate
    // offsets below 64 KiB
    __shared__ __align__(16) _Float16 vt_s[kHD][kVRow];
    __shared__ __align__(16) _Float16 k_s[kLT][kKRow];
    // IPV views of the Vᵀ tile: int8 Vᵀ, then the tile's V scales [block][dim]
    int8_t(*vt8)[kVRowB] = reinterpret_cast<int8_t(*)[kVRowB]>(&vt_s[0][0]);
    float(*vsc)[kHD] = reinterpret_cast<float(*)[kHD]>(reinterpret_cast<int8_t *>(&vt_s[0][0]) +
                                                       kHD * kVRowB);

    // XCD-aware order: workgroups go to the 8 XCDs round-robin by linear id,
    // and each XCD has its own L2.  With the head groups a multiple of 8,
    // linear id L runs head group (L mod 8)·per + (L/8) mod per, query tile
    // (L/8)/per, so an XCD serves only `per` head groups and its L2 holds
    // their K/V pages (causal config 4: 434 -> 617 TFLOP/s).
    int bx = (int)blockIdx.x, by = (int)blockIdx.y;
    if (gridDim.y % 8 == 0) {
        const int L = bx + by * qtiles, per = (int)gridDim.y / 8, idx = L >> 3;
        by = (L & 7) * per + idx % per;
        bx = idx / per;
    }
    const int tile = qtiles - 1 - bx;  // heaviest (latest) query tile first
    // HPW query heads (of one kv head) share the workgroup and each K/V
    // tile: waves 4h .. 4h+3 take query head HPW·by + h
    const int tid = threadIdx.x, lane = tid & 63, wave = (tid >> 6) & 3;
    const int qh = HPW * by + (tid >> 8), kvh = qh / (n_q / n_kv);
    const int l32 = lane & 31, hh = lane >> 5;

    // this lane's query (column l32 of the wave's 32) and its Qᵀ operand:
    // dims 16c + 8hh .. +7 for c = 0..7, as f16
    const int my_q = tile * kQT + wave * 32 + l32;
    const bool q_valid = my_q < n_tok;
    const int qp = q0 + my_q;  // its position
    // scores come out of the MFMA in log2 units: q carries scale·log2(e),
    // so the softmax exponentials are plain exp2 (v_exp_f32)
    const float qscale = scale * 1.44269504088896341f;
    h8 qb[8];
    {
        const float *qr = q + ((size_t)(q_valid ? my_q : 0) * n_q + qh) * kHD + 8 * hh;
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const float4 a = *reinterpret_cast<const float4 *>(qr + 16 * c);
            const float4 b = *reinterpret_cast<const float4 *>(qr + 16 * c + 4);
            const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int e = 0; e < 8; e++) qb[c][e] = (_Float16)(q_valid ? v[e] * qscale : 0.f);
        }
    }
    f32x16 o[4];
#pragma unroll
    for (int d = 0; d < 4; d++)
#pragma unroll
        for (int i = 0; i < 16; i++) o[d][i] = 0.f;
    float m_run = kNegBig, l_run = 0.f;

    const int qpos_lo = q0 + tile * kQT;
    const int qpos_hi = q0 + min((tile + 1) * kQT, n_tok) - 1;
    const int k_lo = window > 0 ? max(0, qpos_lo + 1 - window) : 0;
    const int k_hi = qpos_hi;

    for (int kl = k_lo; kl <= k_hi; kl += kLT) {
        __syncthreads();  // the previous tile's LDS reads are done
        // dequantize K and V of the tile's keys: thread -> (key pair t/4,
        // 32-block t%4): four lanes read a key's whole 128-byte row, and a
        // Vᵀ row write packs both keys of the pair into one dword (16
        // consecutive dwords per block, the blocks 8 dwords apart)
        for (int t = tid; t < kLT * 2; t += 256 * HPW) {
            const int blk = t & 3, pair = t >> 2;
            uint32_t vpk[32];
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int kk = 2 * pair + e;
                const int key = kl + kk;
                _Float16 kv[32], vv[32];
                if (key <= k_hi) {
                    const bool fresh = src.ckq != nullptr && key >= q0;
                    const int slot = fresh ? key - q0 : src.ring ? key % src.ring : key;
                    const size_t row = (size_t)slot * n_kv + kvh;
                    const int8_t *kqb = fresh ? src.ckq : src.kq;
                    const int8_t *vqb = fresh ? src.cvq : src.vq;
                    const uint16_t *ksb = fresh ? src.cks : src.ks;
                    const uint16_t *vsb = fresh ? src.cvs : src.vs;
                    const i32x4 *kp = reinterpret_cast<const i32x4 *>(kqb + row * kHD + 32 * blk);
                    const i32x4 *vp = reinterpret_cast<const i32x4 *>(vqb + row * kHD + 32 * blk);
                    const i32x4 k0 = kp[0], k1 = kp[1], v0 = vp[0], v1 = vp[1];
                    // q·d in f16 with one rounding, as (f16)(d·q) in f32 (the
                    // product of an int8 and an f16 is exact in both): four
                    // quants at a time become the f16 pairs 1024 + (q + 128)
                    // by a byte permute against 0x64, -1152 gives q exactly,
                    // and a packed f16 multiply applies d
                    const _Float16 sk = __builtin_bit_cast(_Float16, ksb[row * (kHD / 32) + blk]);
                    const _Float16 sv = IPV ? (_Float16)1.f
                                            : __builtin_bit_cast(_Float16, vsb[row * (kHD / 32) + blk]);
                    const h2 dk = {sk, sk}, dv = {sv, sv};
                    const int kw[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
                    const int vw[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
                    for (int w = 0; w < 8; w++) {
                        const h2 k01 = i8_pair_f16((uint32_t)kw[w], 0x04010400u) * dk;
                        const h2 k23 = i8_pair_f16((uint32_t)kw[w], 0x04030402u) * dk;
                        const h2 v01 = i8_pair_f16((uint32_t)vw[w], 0x04010400u) * dv;
                        const h2 v23 = i8_pair_f16((uint32_t)vw[w], 0x04030402u) * dv;
                        kv[4 * w] = k01[0], kv[4 * w + 1] = k01[1], kv[4 * w + 2] = k23[0], kv[4 * w + 3] = k23[1];
                        vv[4 * w] = v01[0], vv[4 * w + 1] = v01[1], vv[4 * w + 2] = v23[0], vv[4 * w + 3] = v23[1];
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < 32; j++) kv[j] = vv[j] = (_Float16)0.f;
                }
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    h8 kt;
#pragma unroll
                    for (int q8 = 0; q8 < 8; q8++) kt[q8] = kv[8 * j + q8];
                    *reinterpret_cast<h8 *>(&k_s[kk][32 * blk + 8 * j]) = kt;
                }
#pragma unroll
                for (int j = 0; j < 32; j++) {
                    // IPV: the raw quants (exact as f16 with a unit scale) as bytes
                    const uint32_t bits = IPV ? (uint32_t)((int)(float)vv[j] & 0xff)
                                              : (uint32_t)__builtin_bit_cast(uint16_t, vv[j]);
                    vpk[j] = e == 0 ? bits : vpk[j] | (bits << (IPV ? 8 : 16));
                }
            }
            if (IPV) {
#pragma unroll
                for (int j = 0; j < 32; j++)
                    *reinterpret_cast<uint16_t *>(&vt8[32 * blk + j][2 * pair]) = (uint16_t)vpk[j];
            } else {
#pragma unroll
                for (int j = 0; j < 32; j++)
                    *reinterpret_cast<uint32_t *>(&vt_s[32 * blk + j][vt_col(2 * pair, blk)]) = vpk[j];
            }
        }
        if (IPV) {  // the tile's key-blocked V scales, [block][dim]
            for (int t = tid; t < (kLT / 32) * kHD; t += 256 * HPW) {
                const int b = t / kHD, dim = t % kHD;
                const int key0 = kl + 32 * b;
                vsc[b][dim] = key0 <= k_hi
                                  ? f16_bits_to_f32(src.vs[((size_t)(key0 / 32) * n_kv + kvh) * kHD + dim])
                                  : 0.f;
            }
        }
        __syncthreads();

#pragma unroll 1
      for (int sub = 0; sub < kSub; sub++) {
        const int kb = kl + kKT * sub, ko = kKT * sub;  // compute tile: keys kb.., LDS rows ko..
        if (kb > k_hi) break;
        // Sᵀ = K·Qᵀ for the tile's two 32-key halves
        f32x16 s[2];
#pragma unroll
        for (int t2 = 0; t2 < 2; t2++)
#pragma unroll
            for (int i = 0; i < 16; i++) s[t2][i] = 0.f;
        // the two halves' MFMA chains interleaved: consecutive MFMAs independent
#pragma unroll
        for (int c = 0; c < 8; c++)
#pragma unroll
            for (int t2 = 0; t2 < 2; t2++) {
                const h8 a = *reinterpret_cast<const h8 *>(&k_s[ko + 32 * t2 + l32][16 * c + 8 * hh]);
                s[t2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qb[c], s[t2], 0, 0, 0);
            }
        // mask and the online softmax for this lane's query.  A tile whose
        // keys all precede the wave's first query (and, with a window, all
        // lie inside the last query's window) needs no mask: the test is
        // wave-uniform, and keys past the chunk's end (zero rows of the last
        // LDS tile) never pass it.
        const int wq_lo = q0 + tile * kQT + wave * 32;
        const bool full = kb + kKT - 1 <= wq_lo && (window <= 0 || kb > wq_lo + 31 - window);
        float mx = m_run;
        if (full) {
#pragma unroll
            for (int t2 = 0; t2 < 2; t2++)
#pragma unroll
                for (int i = 0; i < 16; i++) mx = fmaxf(mx, s[t2][i]);
        } else {
#pragma unroll
            for (int t2 = 0; t2 < 2; t2++)
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const int key = kb + 32 * t2 + 8 * (i / 4) + 4 * hh + (i % 4);
                    const bool ok = q_valid && key <= qp && (window <= 0 || key > qp - window);
                    const float v = ok ? s[t2][i] : kNegBig;
                    s[t2][i] = v;
                    mx = fmaxf(mx, v);
                }
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
        // lazy rescale: the reference max moves only when the tile's max
        // exceeds it by more than 2^8 (p <= 256, exact in f16's range), so
        // the accumulator's rescale is usually skipped; the normalisation by
        // l at the end is unchanged (same reference max in numerator and
        // denominator)
        if (!(mx > m_run + 8.0f)) mx = m_run;
        const float corr = __builtin_amdgcn_exp2f(m_run - mx);
        float rs = 0.f;
        h8 pb[2][2];
        v4i_p pq[2];     // IPV: P quants of block t2 (K order: this lane's 16 keys)
        float pd[2];     // IPV: their f16-rounded scale
        // p = 2^(s - max); masked scores give 0 (a lane whose keys so far are
        // all masked has mx = kNegBig, where 2^(s - mx) alone would give 1)
        float pfa[2][16];
        if (full) {
#pragma unroll
            for (int t2 = 0; t2 < 2; t2++)
#pragma unroll
                for (int i = 0; i < 16; i++) pfa[t2][i] = __builtin_amdgcn_exp2f(s[t2][i] - mx);
        } else {
#pragma unroll
            for (int t2 = 0; t2 < 2; t2++)
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const float v = s[t2][i];
                    pfa[t2][i] = v > kNegBig ? __builtin_amdgcn_exp2f(v - mx) : 0.f;
                }
        }
#pragma unroll
        for (int t2 = 0; t2 < 2; t2++) {
            const float(&pf)[16] = pfa[t2];
            if (!IPV) {
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    rs += pf[i];
                    pb[t2][i / 8][i % 8] = (_Float16)pf[i];
                }
            } else {
                // Q8 of P over the block's 32 keys (16 here, 16 in lane ^ 32):
                // d = amax/127, q = round(p/d), the denominator sums f16(d)·q
                // (attn_prefill_global_flash_sp_ipv.wgsl:157-177)
                float amax = 0.f;
#pragma unroll
                for (int i = 0; i < 16; i++) amax = fmaxf(amax, pf[i]);
                amax = fmaxf(amax, __shfl_xor(amax, 32, kWave));
                const float dq = amax * (1.0f / 127.0f);
                const float id = dq > 0.f ? 1.0f / dq : 0.f;
                const float dd = f16_bits_to_f32(f32_to_f16_bits(dq));
                int qs = 0;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    uint32_t w = 0;
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const int qi = min(127, (int)__builtin_rintf(pf[4 * j + e] * id));
                        qs += qi;
                        w |= (uint32_t)(qi & 0xff) << (8 * e);
                    }
                    pq[t2][j] = (int)w;
                }
                pd[t2] = dd;
                rs += dd * (float)qs;
            }
        }
        rs += __shfl_xor(rs, 32, kWave);
        l_run = l_run * corr + rs;
        m_run = mx;
        if (__builtin_amdgcn_ballot_w64(corr != 1.0f)) {
#pragma unroll
            for (int d = 0; d < 4; d++)
#pragma unroll
                for (int i = 0; i < 16; i++) o[d][i] *= corr;
        }
        if (IPV) {
            // Oᵀ += Vᵀ·Pᵀ per 32-key block: A row = dim 32d + l32 with this
            // lane's keys 8j + 4hh .. +3 (j = 0..3, the order of pq), B column =
            // this lane's query; then ×(v_scale[dim]·p_scale)
#pragma unroll
            for (int t2 = 0; t2 < 2; t2++) {
                const int kbase = ko + 32 * t2;
#pragma unroll
                for (int d = 0; d < 4; d++) {
                    const int8_t *vr = &vt8[32 * d + l32][kbase + 4 * hh];
                    const v4i_p a = {*reinterpret_cast<const int *>(vr),
                                     *reinterpret_cast<const int *>(vr + 8),
                                     *reinterpret_cast<const int *>(vr + 16),
                                     *reinterpret_cast<const int *>(vr + 24)};
                    const v16i_p dot =
                        __builtin_amdgcn_mfma_i32_32x32x32_i8(a, pq[t2], v16i_p{}, 0, 0, 0);
                    const float *vs_row = &vsc[kbase / 32][32 * d + 4 * hh];
#pragma unroll
                    for (int g = 0; g < 4; g++) {
                        const float4 sv = *reinterpret_cast<const float4 *>(vs_row + 8 * g);
                        const float svv[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            o[d][4 * g + e] = __builtin_fmaf((float)dot[4 * g + e], svv[e] * pd[t2],
                                                             o[d][4 * g + e]);
                    }
                }
            }
            continue;
        }
        // Oᵀ += Vᵀ·Pᵀ: key chunk (t2, half) = keys 32t2 + 16half + {4hh..+3, 8+4hh..+3}
        // dim tiles innermost: consecutive MFMAs accumulate into different o[d]
#pragma unroll
        for (int t2 = 0; t2 < 2; t2++)
#pragma unroll
            for (int half = 0; half < 2; half++)
#pragma unroll
                for (int d = 0; d < 4; d++) {
                    const int c0 = ko + 32 * t2 + 16 * half + 4 * hh;
                    const h4 lo = *reinterpret_cast<const h4 *>(&vt_s[32 * d + l32][vt_col(c0, d)]);
                    const h4 hi = *reinterpret_cast<const h4 *>(&vt_s[32 * d + l32][vt_col(c0 + 8, d)]);
                    const h8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                    o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb[t2][half], o[d], 0, 0, 0);
                }
      }
    }

    if (!q_valid) return;
    const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;
    float *orow = out + ((size_t)my_q * n_q + qh) * kHD;
#pragma unroll
    for (int d = 0; d < 4; d++)
#pragma unroll
        for (int i = 0; i < 16; i++) orow[32 * d + 8 * (i / 4) + 4 * hh + (i % 4)] = o[d][i] * inv;
}

// Warp-specialized form of the f16 path (the one the launchers use;
// attn_prefill_kernel serves the int8-PV form): the 8 waves of
// attn_prefill_kernel compute, and 4 more waves (producers)
// dequantize the next 128-key tile into the other of two LDS buffers
// meanwhile, so that the dequant VALU and LDS writes run beside the matrix
// cores instead of between two barriers (3 waves per SIMD: two computing, one
// staging).  One barrier per tile.  The per-tile math and the Vᵀ swizzle
// are those of attn_prefill_kernel.
constexpr int kWLT = 128;           // keys per LDS tile
constexpr int kWSub = kWLT / kKT;   // compute tiles per LDS tile
constexpr int kWVRow = kWLT + 4;    // Vᵀ row: 66 dwords, rows 2 banks apart

template <int HPW>
__global__ __launch_bounds__(256 * HPW + 256) void attn_prefill_ws_kernel(
    const float *__restrict__ q, KvSource src, float *__restrict__ out, int n_tok, int q0,
    int n_q, int n_kv, int window, float scale, int qtiles, const uint32_t *__restrict__ step) {
    if (step) q0 = (int)step[3];
    __shared__ __align__(16) _Float16 vt_s[2][kHD][kWVRow];
    __shared__ __align__(16) _Float16 k_s[2][kWLT][kKRow];

    int bx = (int)blockIdx.x, by = (int)blockIdx.y;
    if (gridDim.y % 8 == 0) {  // XCD-aware order, as in attn_prefill_kernel
        const int L = bx + by * qtiles, per = (int)gridDim.y / 8, idx = L >> 3;
        by = (L & 7) * per + idx % per;
        bx = idx / per;
    }
    const int tile = qtiles - 1 - bx;  // heaviest (latest) query tile first
    const int tid = threadIdx.x;
    const bool producer = tid >= 256 * HPW;
    const int lane = tid & 63, wave = (tid >> 6) & 3;
    const int qh = HPW * by + (producer ? 0 : tid >> 8), kvh = (HPW * by) / (n_q / n_kv);
    const int l32 = lane & 31, hh = lane >> 5;

    const int qpos_lo = q0 + tile * kQT;
    const int qpos_hi = q0 + min((tile + 1) * kQT, n_tok) - 1;
    const int k_lo = window > 0 ? max(0, qpos_lo + 1 - window) : 0;
    const int k_hi = qpos_hi;
    const int n_t = (k_hi - k_lo) / kWLT + 1;

    // ---- producers: key pair t/4, 32-block t%4 of a 128-key tile per thread;
    // tile i+2's quants are loaded into registers before tile i+1 is
    // dequantized, so their latency overlaps the dequant and the barrier
    if (producer) {
        struct Raw {
            i32x4 k[2][2], v[2][2];  // [key of the pair][16-byte half of the block]
            uint16_t sk[2], sv[2];
        };
        const int t = tid - 256 * HPW;
        const int blk = t & 3, pair = t >> 2;
        // kernel-argument pointers pinned in scalar registers (a per-lane
        // choice between them then costs no dependent pointer load)
        const int8_t *const kq_c = sgpr_ptr(src.kq), *const vq_c = sgpr_ptr(src.vq);
        const uint16_t *const ks_c = sgpr_ptr(src.ks), *const vs_c = sgpr_ptr(src.vs);
        const bool has_chunk = src.ckq != nullptr;
        const int8_t *const kq_f = has_chunk ? sgpr_ptr(src.ckq) : kq_c;
        const int8_t *const vq_f = has_chunk ? sgpr_ptr(src.cvq) : vq_c;
        const uint16_t *const ks_f = has_chunk ? sgpr_ptr(src.cks) : ks_c;
        const uint16_t *const vs_f = has_chunk ? sgpr_ptr(src.cvs) : vs_c;
        const int ring = src.ring;
        auto fetch = [&](int kl, Raw &r) {
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int key = min(kl + 2 * pair + e, k_hi);  // past k_hi: zeroed below
                const bool fresh = has_chunk && key >= q0;
                const int slot = fresh ? key - q0 : ring ? key % ring : key;
                const size_t row = (size_t)slot * n_kv + kvh;
                const i32x4 *kp = reinterpret_cast<const i32x4 *>((fresh ? kq_f : kq_c) + row * kHD + 32 * blk);
                const i32x4 *vp = reinterpret_cast<const i32x4 *>((fresh ? vq_f : vq_c) + row * kHD + 32 * blk);
                r.k[e][0] = gload(kp);
                r.k[e][1] = gload(kp + 1);
                r.v[e][0] = gload(vp);
                r.v[e][1] = gload(vp + 1);
                r.sk[e] = gload((fresh ? ks_f : ks_c) + row * (kHD / 32) + blk);
                r.sv[e] = gload((fresh ? vs_f : vs_c) + row * (kHD / 32) + blk);
            }
        };
        auto stage = [&](int kl, const Raw &r, int buf) {
            uint32_t vpk[32];
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int kk = 2 * pair + e;
                const bool live = kl + kk <= k_hi;
                const _Float16 sk = live ? __builtin_bit_cast(_Float16, r.sk[e]) : (_Float16)0.f;
                const _Float16 sv = live ? __builtin_bit_cast(_Float16, r.sv[e]) : (_Float16)0.f;
                const h2 dk = {sk, sk}, dv = {sv, sv};
                const int kw[8] = {r.k[e][0].x, r.k[e][0].y, r.k[e][0].z, r.k[e][0].w,
                                   r.k[e][1].x, r.k[e][1].y, r.k[e][1].z, r.k[e][1].w};
                const int vw[8] = {r.v[e][0].x, r.v[e][0].y, r.v[e][0].z, r.v[e][0].w,
                                   r.v[e][1].x, r.v[e][1].y, r.v[e][1].z, r.v[e][1].w};
                _Float16 kv[32], vv[32];
#pragma unroll
                for (int w = 0; w < 8; w++) {
                    const h2 k01 = i8_pair_f16((uint32_t)kw[w], 0x04010400u) * dk;
                    const h2 k23 = i8_pair_f16((uint32_t)kw[w], 0x04030402u) * dk;
                    const h2 v01 = i8_pair_f16((uint32_t)vw[w], 0x04010400u) * dv;
                    const h2 v23 = i8_pair_f16((uint32_t)vw[w], 0x04030402u) * dv;
                    kv[4 * w] = k01[0], kv[4 * w + 1] = k01[1], kv[4 * w + 2] = k23[0], kv[4 * w + 3] = k23[1];
                    vv[4 * w] = v01[0], vv[4 * w + 1] = v01[1], vv[4 * w + 2] = v23[0], vv[4 * w + 3] = v23[1];
                }
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    h8 kt;
#pragma unroll
                    for (int q8 = 0; q8 < 8; q8++) kt[q8] = kv[8 * j + q8];
                    *reinterpret_cast<h8 *>(&k_s[buf][kk][32 * blk + 8 * j]) = kt;
                }
#pragma unroll
                for (int j = 0; j < 32; j++) {
                    const uint32_t bits = (uint32_t)__builtin_bit_cast(uint16_t, vv[j]);
                    vpk[j] = e == 0 ? bits : vpk[j] | (bits << 16);
                }
            }
#pragma unroll
            for (int j = 0; j < 32; j++)
                *reinterpret_cast<uint32_t *>(&vt_s[buf][32 * blk + j][vt_col(2 * pair, blk)]) = vpk[j];
        };
        Raw ra, rb;
        fetch(k_lo, ra);
        if (n_t > 1) fetch(k_lo + kWLT, rb);
        stage(k_lo, ra, 0);
        __syncthreads();
        // iteration it stages tile it+1 (in rb or ra by parity) and first
        // fetches tile it+2 into the other set
#pragma unroll 1
        for (int it = 0; it < n_t; it += 2) {
            if (it + 1 < n_t) {
                if (it + 2 < n_t) fetch(k_lo + (it + 2) * kWLT, ra);
                stage(k_lo + (it + 1) * kWLT, rb, 1);
            }
            __syncthreads();
            if (it + 1 >= n_t) break;
            if (it + 2 < n_t) {
                if (it + 3 < n_t) fetch(k_lo + (it + 3) * kWLT, rb);
                stage(k_lo + (it + 2) * kWLT, ra, 0);
            }
            __syncthreads();
        }
        return;
    }

    // ---- consumers (the 8 waves of attn_prefill_kernel)
    const int my_q = tile * kQT + wave * 32 + l32;
    const bool q_valid = my_q < n_tok;
    const int qp = q0 + my_q;
    const float qscale = scale * 1.44269504088896341f;
    h8 qb[8];
    {
        const float *qr = q + ((size_t)(q_valid ? my_q : 0) * n_q + qh) * kHD + 8 * hh;
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const float4 a = *reinterpret_cast<const float4 *>(qr + 16 * c);
            const float4 b = *reinterpret_cast<const float4 *>(qr + 16 * c + 4);
            const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int e = 0; e < 8; e++) qb[c][e] = (_Float16)(q_valid ? v[e] * qscale : 0.f);
        }
    }
    f32x16 o[4];
#pragma unroll
    for (int d = 0; d < 4; d++)
#pragma unroll
        for (int i = 0; i < 16; i++) o[d][i] = 0.f;
    float m_run = kNegBig, l_run = 0.f;
    const int wq_lo = q0 + tile * kQT + wave * 32;

    __syncthreads();  // tile 0 staged
#pragma unroll 1
    for (int it = 0; it < n_t; it++) {
        const int kl = k_lo + it * kWLT, buf = it & 1;
#pragma unroll 1
        for (int sub = 0; sub < kWSub; sub++) {
            const int kb = kl + kKT * sub, ko = kKT * sub;
            if (kb > k_hi) break;
            f32x16 s[2];
#pragma unroll
            for (int t2 = 0; t2 < 2; t2++)
#pragma unroll
                for (int i = 0; i < 16; i++) s[t2][i] = 0.f;
#pragma unroll
            for (int c = 0; c < 8; c++)
#pragma unroll
                for (int t2 = 0; t2 < 2; t2++) {
                    const h8 a = *reinterpret_cast<const h8 *>(&k_s[buf][ko + 32 * t2 + l32][16 * c + 8 * hh]);
                    s[t2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qb[c], s[t2], 0, 0, 0);
                }
            const bool full = kb + kKT - 1 <= wq_lo && (window <= 0 || kb > wq_lo + 31 - window);
            float mx = m_run;
            if (full) {
#pragma unroll
                for (int t2 = 0; t2 < 2; t2++)
#pragma unroll
                    for (int i = 0; i < 16; i++) mx = fmaxf(mx, s[t2][i]);
            } else {
#pragma unroll
                for (int t2 = 0; t2 < 2; t2++)
#pragma unroll
                    for (int i = 0; i < 16; i++) {
                        const int key = kb + 32 * t2 + 8 * (i / 4) + 4 * hh + (i % 4);
                        const bool ok = q_valid && key <= qp && (window <= 0 || key > qp - window);
                        const float v = ok ? s[t2][i] : kNegBig;
                        s[t2][i] = v;
                        mx = fmaxf(mx, v);
                    }
            }
            mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
            if (!(mx > m_run + 8.0f)) mx = m_run;
            const float corr = __builtin_amdgcn_exp2f(m_run - mx);
            float rs = 0.f;
            h8 pb[2][2];
#pragma unroll
            for (int t2 = 0; t2 < 2; t2++)
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const float v = s[t2][i];
                    const float p = full || v > kNegBig ? __builtin_amdgcn_exp2f(v - mx) : 0.f;
                    rs += p;
                    pb[t2][i / 8][i % 8] = (_Float16)p;
                }
            rs += __shfl_xor(rs, 32, kWave);
            l_run = l_run * corr + rs;
            m_run = mx;
            if (__builtin_amdgcn_ballot_w64(corr != 1.0f)) {
#pragma unroll
                for (int d = 0; d < 4; d++)
#pragma unroll
                    for (int i = 0; i < 16; i++) o[d][i] *= corr;
            }
#pragma unroll
            for (int t2 = 0; t2 < 2; t2++)
#pragma unroll
                for (int half = 0; half < 2; half++)
#pragma unroll
                    for (int d = 0; d < 4; d++) {
                        const int c0 = ko + 32 * t2 + 16 * half + 4 * hh;
                        const h4 lo = *reinterpret_cast<const h4 *>(&vt_s[buf][32 * d + l32][vt_col(c0, d)]);
                        const h4 hi = *reinterpret_cast<const h4 *>(&vt_s[buf][32 * d + l32][vt_col(c0 + 8, d)]);
                        const h8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                        o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb[t2][half], o[d], 0, 0, 0);
                    }
        }
        __syncthreads();  // this tile read; the producers have staged the next
    }

    if (!q_valid) return;
    const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;
    float *orow = out + ((size_t)my_q * n_q + qh) * kHD;
#pragma unroll
    for (int d = 0; d < 4; d++)
#pragma unroll
        for (int i = 0; i < 16; i++) orow[32 * d + 8 * (i / 4) + 4 * hh + (i % 4)] = o[d][i] * inv;
}

// Prefill attention at head_dim 256 / 512 (the released checkpoint's
// sliding and global layers; crates/sg-gguf/src/desc.rs:66-93), same
// semantics as above.  One query head per workgroup of 8 waves; a query
// tile of 32 is served by D = HD/128 waves, wave ds owning dims [128·ds,
// 128·ds + 128): its slice of the queries sits in registers (as in the
// head_dim-128 kernel), it computes the partial scores Sᵀ = K·Qᵀ of a
// 32-key tile over its dims, and the D partials meet
// through LDS, summed in slice order, so that the D waves hold
// bit-identical scores, run the same online softmax and accumulate Oᵀ for
// their own dims.  Per tile, two barriers:
//   QK(t) → partials out → barrier → K(t+1) and V(t+1) staged (V double-
//   buffered), quants of t+2 issued → partials summed, softmax, PV(t) →
//   barrier.
// Every thread stages one item per tile: two keys × head_dim/32 dims.
// The Vᵀ rows carry a pad of 16 dwords per 16 rows, so the item writes
// (rows 8 or 16 apart within a wave) and the PV reads are free of bank
// conflicts.
//
// Page formats (FMT), one kernel body:
//   kPfQ8   fp32 q, Q8_0 K and V dequantized to f16 in LDS, fp32 out, q0
//           from the host (the model driver's prefill)
//   kPfQ8H  f16 q, Q8_0 K and V as above, f16 out, q0 = step[3]
//           (attn_prefill_global_flash_sp_q8.wgsl)
//   kPfF16  f16 q, K and V f16 pages, f16 out, q0 = step[3]
//           (attn_prefill_sliding[_ring].wgsl, attn_prefill_global[_flash
//           [_sp]].wgsl)
//   kPfIQ   int8 q with f16 scales per 32 dims, K as Q8_0 quants with its
//           scales, V f16, f16 out, q0 = step[3]: the score is the sum over
//           32-dim blocks of q_scale·k_scale·(exact integer dot)
//           (attn_prefill_global_flash_sp_iq.wgsl:94-125).  The integer
//           dot runs on the f16 MFMA over the quants' exact f16 values
//           (|products| < 2^14, block sums < 2^24: exact in fp32).
//   kPfIPV  as kPfIQ for q and K; V int8 with key-blocked f16 scales (one per
//           32 keys and column, kv_append_global_v_q8.wgsl:32-75), causal
//           only, so every 32-key tile is one V scale block; P is quantized
//           per (query, tile): d = amax/127, q = min(127, rint(p/d)), the
//           denominator sums f16(d)·q; Oᵀ += (Vᵀ_q·Pᵀ_q)·v_scale[dim]·f16(d),
//           the integer dot exact on the f16 MFMA
//           (attn_prefill_global_flash_sp_ipv.wgsl:134-210)
// Except for kPfQ8, q enters the MFMA as its exact f16 values and the
// scores are scaled afterwards.
enum PfFmt { kPfQ8 = 0, kPfQ8H = 1, kPfF16 = 2, kPfIQ = 3, kPfIPV = 4 };

template <int HD, int FMT>
__global__ __launch_bounds__(512) void attn_prefill_wide_kernel(
    const void *__restrict__ qv, const uint16_t *__restrict__ q_scales, KvSource src,
    void *__restrict__ outv, int n_tok, int q0_host, const uint32_t *__restrict__ step, int n_q,
    int n_kv, int window, float scale, int qtiles) {
    constexpr bool VKB = FMT == kPfIPV;  // int8 V, key-blocked scales, int8 P
    constexpr bool QF32 = FMT == kPfQ8, QI8 = FMT == kPfIQ || VKB;
    constexpr bool KQ8 = FMT == kPfQ8 || FMT == kPfQ8H;  // dequantized into LDS
    constexpr bool KF16 = FMT == kPfF16, KRAW = FMT == kPfIQ || VKB;
    constexpr bool VF16 = FMT == kPfF16 || FMT == kPfIQ;
    constexpr bool O16 = FMT != kPfQ8;
    constexpr int D = HD / 128;        // waves per query tile
    constexpr int QTW = 8 / D;         // query tiles per workgroup
    constexpr int QW = 32 * QTW;       // queries per workgroup
    constexpr int KT = 32;             // keys per tile
    constexpr int NB = HD / 32;        // 32-dim blocks per row
    constexpr int NP = KT / 2;         // key pairs per tile
    constexpr int CW = HD / 32;        // dims per staging item (8 or 16)
    constexpr int KRow = HD + 8;       // halves
    constexpr int VS = NP + 4;         // Vᵀ row stride, dwords
    constexpr int VBuf = HD * VS + (HD / 16) * NP;  // dwords per Vᵀ buffer
    static_assert(NP * (HD / CW) == 512, "one staging item per thread");
    __shared__ __align__(16) _Float16 k_s[KT][KRow];
    __shared__ __align__(16) uint32_t vt_s[2][VBuf];
    __shared__ __align__(16) float4 ex_s[8][4][64];  // partial scores [wave][i/4][lane]
    __shared__ __align__(16) float ksc_s[KRAW ? NB : 1][KT];  // int8 QK: k scales [block][key]
    __shared__ __align__(16) float vsk_s[VKB ? 2 : 1][VKB ? HD : 1];  // the tile's V scales
    auto vt_at = [](int row, int col) { return row * VS + (row >> 4) * NP + col; };

    int bx = (int)blockIdx.x, by = (int)blockIdx.y;
    if (gridDim.y % 8 == 0) {  // XCD-aware order, as in attn_prefill_kernel
        const int L = bx + by * qtiles, per = (int)gridDim.y / 8, idx = L >> 3;
        by = (L & 7) * per + idx % per;
        bx = idx / per;
    }
    const int q0 = QF32 ? q0_host : (int)step[3];
    const int tile = qtiles - 1 - bx;  // heaviest (latest) query tile first
    const int qh = by, kvh = qh / (n_q / n_kv);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int qt = wave / D, ds = wave % D;
    const int l32 = lane & 31, hh = lane >> 5;
    const int my_q = tile * QW + qt * 32 + l32;
    const bool q_valid = my_q < n_tok;
    const int qp = q0 + my_q;

    // this lane's query (column l32) on the wave's dims as the f16 B
    // operand: dims 128·ds + 16c + 8hh .. +7.  kPfQ8: pre-scaled (scores in
    // log2 units); otherwise exact, with the scale applied to the scores.
    const float qscale = scale * 1.44269504088896341f;
    h8 qb[8];
    float qsb[KRAW ? 4 : 1];  // kPfIQ: q scale · qscale of the wave's 4 blocks
    {
        const size_t qoff = ((size_t)(q_valid ? my_q : 0) * n_q + qh) * HD + 128 * ds + 8 * hh;
        if constexpr (QF32) {
            const float *qr = static_cast<const float *>(qv) + qoff;
#pragma unroll
            for (int c = 0; c < 8; c++) {
                const float4 a = *reinterpret_cast<const float4 *>(qr + 16 * c);
                const float4 b = *reinterpret_cast<const float4 *>(qr + 16 * c + 4);
                const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
                for (int e = 0; e < 8; e++) qb[c][e] = (_Float16)(q_valid ? v[e] * qscale : 0.f);
            }
        } else if constexpr (QI8) {
            const int8_t *qr = static_cast<const int8_t *>(qv) + qoff;
#pragma unroll
            for (int c = 0; c < 8; c++) {
                const uint2 w = *reinterpret_cast<const uint2 *>(qr + 16 * c);
                const h2 a = i8_pair_f16(w.x, 0x04010400u), b = i8_pair_f16(w.x, 0x04030402u);
                const h2 e2 = i8_pair_f16(w.y, 0x04010400u), f = i8_pair_f16(w.y, 0x04030402u);
                const h8 t = {a[0], a[1], b[0], b[1], e2[0], e2[1], f[0], f[1]};
                qb[c] = q_valid ? t : h8{};
            }
            const uint16_t *qs = q_scales + ((size_t)(q_valid ? my_q : 0) * n_q + qh) * NB + 4 * ds;
#pragma unroll
            for (int b = 0; b < 4; b++)
                qsb[b] = q_valid ? (float)__builtin_bit_cast(_Float16, qs[b]) * qscale : 0.f;
        } else {
            const uint16_t *qr = static_cast<const uint16_t *>(qv) + qoff;
#pragma unroll
            for (int c = 0; c < 8; c++) {
                const h8 t = __builtin_bit_cast(h8, *reinterpret_cast<const uint4 *>(qr + 16 * c));
                qb[c] = q_valid ? t : h8{};
            }
        }
    }

    f32x16 o[4];
#pragma unroll
    for (int d = 0; d < 4; d++)
#pragma unroll
        for (int i = 0; i < 16; i++) o[d][i] = 0.f;
    float m_run = kNegBig, l_run = 0.f;

    const int qpos_lo = q0 + tile * QW;
    const int qpos_hi = q0 + min((tile + 1) * QW, n_tok) - 1;
    const int k_lo = window > 0 ? max(0, qpos_lo + 1 - window) : 0;
    const int k_hi = qpos_hi;
    const int wq_lo = q0 + tile * QW + qt * 32;

    // staging item of this thread: keys 2·pair, 2·pair + 1 of the tile,
    // dims CW·chunk .. +CW-1
    const int pair = tid % NP, chunk = tid / NP;
    const int dim0 = CW * chunk, blk = dim0 >> 5;
    constexpr int EK = KF16 ? 2 : 1, EV = VF16 ? 2 : 1;  // bytes per K / V element
    const char *const kq_c = sgpr_ptr(reinterpret_cast<const char *>(src.kq));
    const char *const vq_c = sgpr_ptr(reinterpret_cast<const char *>(src.vq));
    const uint16_t *const ks_c = sgpr_ptr(src.ks), *const vs_c = sgpr_ptr(src.vs);
    const bool has_chunk = src.ckq != nullptr;
    const char *const kq_f = has_chunk ? sgpr_ptr(reinterpret_cast<const char *>(src.ckq)) : kq_c;
    const char *const vq_f = has_chunk ? sgpr_ptr(reinterpret_cast<const char *>(src.cvq)) : vq_c;
    const uint16_t *const ks_f = has_chunk ? sgpr_ptr(src.cks) : ks_c;
    const uint16_t *const vs_f = has_chunk ? sgpr_ptr(src.cvs) : vs_c;
    const int ring = src.ring;
    typedef int kraw_t __attribute__((ext_vector_type(CW * EK / 4)));
    typedef int vraw_t __attribute__((ext_vector_type(CW * EV / 4)));
    kraw_t rk[2];
    vraw_t rv[2];
    uint16_t rsk[2], rsv[2];
    float rvk = 0.f;  // kPfIPV: the V scale of column tid for the tile's key block
    auto fetch = [&](int kl) {
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const int key = min(kl + 2 * pair + e, k_hi);  // past k_hi: zeroed when staged
            const bool fresh = has_chunk && key >= q0;
            const int slot = fresh ? key - q0 : ring ? key % ring : key;
            const size_t row = (size_t)slot * n_kv + kvh;
            rk[e] = gload(reinterpret_cast<const kraw_t *>((fresh ? kq_f : kq_c) + (row * HD + dim0) * EK));
            rv[e] = gload(reinterpret_cast<const vraw_t *>((fresh ? vq_f : vq_c) + (row * HD + dim0) * EV));
            if constexpr (!KF16) rsk[e] = gload((fresh ? ks_f : ks_c) + row * NB + blk);
            if constexpr (!VF16 && !VKB) rsv[e] = gload((fresh ? vs_f : vs_c) + row * NB + blk);
        }
        if constexpr (VKB)
            if (tid < HD)
                rvk = (float)__builtin_bit_cast(
                    _Float16, gload(vs_c + ((size_t)(kl / 32) * n_kv + kvh) * HD + tid));
    };
    auto stage = [&](int kl, int vb) {
        uint32_t *vt = vt_s[vb];
        if constexpr (VKB)
            if (tid < HD) vsk_s[vb][tid] = rvk;
        uint32_t vpk[CW];
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const int kk = 2 * pair + e;
            const bool live = kl + kk <= k_hi;
            h8 kt[CW / 8];
            _Float16 vv[CW];
            if constexpr (KF16) {
#pragma unroll
                for (int h = 0; h < CW / 8; h++) {
                    const int4 w = {rk[e][4 * h], rk[e][4 * h + 1], rk[e][4 * h + 2], rk[e][4 * h + 3]};
                    kt[h] = live ? __builtin_bit_cast(h8, w) : h8{};
                }
            } else {
                const _Float16 sk = KQ8 && live ? __builtin_bit_cast(_Float16, rsk[e]) : (_Float16)1.f;
                const h2 dk = {sk, sk};
#pragma unroll
                for (int w = 0; w < CW / 4; w++) {
                    h2 k01 = i8_pair_f16((uint32_t)rk[e][w], 0x04010400u);
                    h2 k23 = i8_pair_f16((uint32_t)rk[e][w], 0x04030402u);
                    if constexpr (KQ8) k01 *= dk, k23 *= dk;
                    kt[w / 2][4 * (w & 1)] = k01[0], kt[w / 2][4 * (w & 1) + 1] = k01[1];
                    kt[w / 2][4 * (w & 1) + 2] = k23[0], kt[w / 2][4 * (w & 1) + 3] = k23[1];
                }
                if (!live)
#pragma unroll
                    for (int h = 0; h < CW / 8; h++) kt[h] = h8{};
                if constexpr (KRAW)
                    if (dim0 % 32 == 0)
                        ksc_s[blk][kk] = live ? (float)__builtin_bit_cast(_Float16, rsk[e]) : 0.f;
            }
            if constexpr (VF16) {
#pragma unroll
                for (int w = 0; w < CW / 2; w++) {
                    const int word = rv[e][w];  // a plain value: bit_cast of a vector
                                                // element reads element 0
                    const h2 p = __builtin_bit_cast(h2, word);
                    vv[2 * w] = live ? p[0] : (_Float16)0.f;
                    vv[2 * w + 1] = live ? p[1] : (_Float16)0.f;
                }
            } else {
                // kPfIPV: the quants themselves (exact f16), scaled after the dot
                const _Float16 sv = !live ? (_Float16)0.f
                                    : VKB ? (_Float16)1.f
                                          : __builtin_bit_cast(_Float16, rsv[e]);
                const h2 dv = {sv, sv};
#pragma unroll
                for (int w = 0; w < CW / 4; w++) {
                    const h2 v01 = i8_pair_f16((uint32_t)rv[e][w], 0x04010400u) * dv;
                    const h2 v23 = i8_pair_f16((uint32_t)rv[e][w], 0x04030402u) * dv;
                    vv[4 * w] = v01[0], vv[4 * w + 1] = v01[1], vv[4 * w + 2] = v23[0], vv[4 * w + 3] = v23[1];
                }
            }
#pragma unroll
            for (int h = 0; h < CW / 8; h++) *reinterpret_cast<h8 *>(&k_s[kk][dim0 + 8 * h]) = kt[h];
#pragma unroll
            for (int j = 0; j < CW; j++) {
                const uint32_t bits = (uint32_t)__builtin_bit_cast(uint16_t, vv[j]);
                vpk[j] = e == 0 ? bits : vpk[j] | (bits << 16);
            }
        }
#pragma unroll
        for (int j = 0; j < CW; j++) vt[vt_at(dim0 + j, pair)] = vpk[j];
    };

    fetch(k_lo);
    stage(k_lo, 0);
    if (k_lo + KT <= k_hi) fetch(k_lo + KT);
    __syncthreads();
    int buf = 0;
    for (int kl = k_lo; kl <= k_hi; kl += KT) {
        // partial Sᵀ of the tile over this wave's 128 dims
        f32x16 s0, s1;
#pragma unroll
        for (int i = 0; i < 16; i++) s0[i] = s1[i] = 0.f;
        if constexpr (KRAW) {
            // per 32-dim block: the exact integer dot, then q_scale·k_scale
#pragma unroll
            for (int b = 0; b < 4; b++) {
                f32x16 t;
#pragma unroll
                for (int i = 0; i < 16; i++) t[i] = 0.f;
#pragma unroll
                for (int c = 2 * b; c < 2 * b + 2; c++) {
                    const h8 a = *reinterpret_cast<const h8 *>(&k_s[l32][128 * ds + 16 * c + 8 * hh]);
                    t = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qb[c], t, 0, 0, 0);
                }
                const float *kb = ksc_s[4 * ds + b];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float4 k4 = *reinterpret_cast<const float4 *>(kb + 8 * j + 4 * hh);
                    const float kv4[4] = {k4.x, k4.y, k4.z, k4.w};
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int i = 4 * j + r;
                        if (b & 1) s1[i] = __builtin_fmaf(qsb[b] * kv4[r], t[i], s1[i]);
                        else s0[i] = __builtin_fmaf(qsb[b] * kv4[r], t[i], s0[i]);
                    }
                }
            }
        } else {
#pragma unroll
            for (int c = 0; c < 8; c += 2) {
                const h8 a0 = *reinterpret_cast<const h8 *>(&k_s[l32][128 * ds + 16 * c + 8 * hh]);
                const h8 a1 = *reinterpret_cast<const h8 *>(&k_s[l32][128 * ds + 16 * c + 16 + 8 * hh]);
                s0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, qb[c], s0, 0, 0, 0);
                s1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, qb[c + 1], s1, 0, 0, 0);
            }
        }
#pragma unroll
        for (int j = 0; j < 4; j++)
            ex_s[wave][j][lane] = make_float4(s0[4 * j] + s1[4 * j], s0[4 * j + 1] + s1[4 * j + 1],
                                              s0[4 * j + 2] + s1[4 * j + 2], s0[4 * j + 3] + s1[4 * j + 3]);
        __syncthreads();  // the partials visible; K(t) fully read
        if (kl + KT <= k_hi) {  // stage t+1 (V into the other buffer), fetch t+2
            stage(kl + KT, buf ^ 1);
            if (kl + 2 * KT <= k_hi) fetch(kl + 2 * KT);
        }
        // the D partials in slice order: the same bits in every wave of the tile
        f32x16 s;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float4 t = ex_s[qt * D][j][lane];
#pragma unroll
            for (int d2 = 1; d2 < D; d2++) {
                const float4 u = ex_s[qt * D + d2][j][lane];
                t.x += u.x, t.y += u.y, t.z += u.z, t.w += u.w;
            }
            s[4 * j] = t.x, s[4 * j + 1] = t.y, s[4 * j + 2] = t.z, s[4 * j + 3] = t.w;
        }
        if constexpr (!QF32 && !KRAW)
#pragma unroll
            for (int i = 0; i < 16; i++) s[i] *= qscale;
        const uint32_t *vt = vt_s[buf];
        {
            const int kb = kl;
            const bool full = kb + 31 <= wq_lo && (window <= 0 || kb > wq_lo + 31 - window);
            // the mask as one uniform branch (inside the max loop it became a
            // taken branch per element on every unmasked tile)
            if (!full) {
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const int key = kb + 8 * (i / 4) + 4 * hh + (i % 4);
                    const bool ok = q_valid && key <= qp && (window <= 0 || key > qp - window);
                    s[i] = ok ? s[i] : kNegBig;
                }
            }
            float mx = m_run;
#pragma unroll
            for (int i = 0; i < 16; i++) mx = fmaxf(mx, s[i]);
            mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
            if (!(mx > m_run + 8.0f)) mx = m_run;
            const float corr = __builtin_amdgcn_exp2f(m_run - mx);
            float rs = 0.f;
            h8 pb[2];
            float pdd = 0.f;  // kPfIPV: f16(d) of the tile's P quants
            if constexpr (VKB) {
                float pf[16], amax = 0.f;
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    pf[i] = full || s[i] > kNegBig ? __builtin_amdgcn_exp2f(s[i] - mx) : 0.f;
                    amax = fmaxf(amax, pf[i]);
                }
                amax = fmaxf(amax, __shfl_xor(amax, 32, kWave));  // the other 16 keys
                const float dq = amax * (1.0f / 127.0f);
                const float id = dq > 0.f ? 1.0f / dq : 0.f;
                pdd = (float)(_Float16)dq;
                int qsum = 0;
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const int qi = min(127, (int)__builtin_rintf(pf[i] * id));
                    qsum += qi;
                    pb[i / 8][i % 8] = (_Float16)(float)qi;
                }
                rs = pdd * (float)qsum;
            } else {
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const float p = full || s[i] > kNegBig ? __builtin_amdgcn_exp2f(s[i] - mx) : 0.f;
                    rs += p;
                    pb[i / 8][i % 8] = (_Float16)p;
                }
            }
            rs += __shfl_xor(rs, 32, kWave);
            l_run = l_run * corr + rs;
            m_run = mx;
            if (__builtin_amdgcn_ballot_w64(corr != 1.0f)) {
#pragma unroll
                for (int d = 0; d < 4; d++)
#pragma unroll
                    for (int i = 0; i < 16; i++) o[d][i] *= corr;
            }
            // Oᵀ (this wave's 128 dims) += Vᵀ·Pᵀ over the group's two 16-key halves
            auto v_operand = [&](int hf, int d) __attribute__((always_inline)) {
                const int row = 128 * ds + 32 * d + l32;
                const int c0 = (16 * hf + 4 * hh) / 2;  // dword column (key pair)
                const uint2 lo = *reinterpret_cast<const uint2 *>(&vt[vt_at(row, c0)]);
                const uint2 hi = *reinterpret_cast<const uint2 *>(&vt[vt_at(row, c0 + 4)]);
                const h4 l4 = __builtin_bit_cast(h4, lo), h4v = __builtin_bit_cast(h4, hi);
                return h8{l4[0], l4[1], l4[2], l4[3], h4v[0], h4v[1], h4v[2], h4v[3]};
            };
            if constexpr (VKB) {
                // per dim chunk: the tile's exact integer dot, then ×v_scale[dim]·f16(d)
#pragma unroll
                for (int d = 0; d < 4; d++) {
                    f32x16 t;
#pragma unroll
                    for (int i = 0; i < 16; i++) t[i] = 0.f;
                    t = __builtin_amdgcn_mfma_f32_32x32x16_f16(v_operand(0, d), pb[0], t, 0, 0, 0);
                    t = __builtin_amdgcn_mfma_f32_32x32x16_f16(v_operand(1, d), pb[1], t, 0, 0, 0);
                    const float *vsr = &vsk_s[buf][128 * ds + 32 * d + 4 * hh];
#pragma unroll
                    for (int g = 0; g < 4; g++) {
                        const float4 sv = *reinterpret_cast<const float4 *>(vsr + 8 * g);
                        const float svv[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            o[d][4 * g + e] = __builtin_fmaf(t[4 * g + e], svv[e] * pdd, o[d][4 * g + e]);
                    }
                }
            } else {
#pragma unroll
                for (int hf = 0; hf < 2; hf++)
#pragma unroll
                    for (int d = 0; d < 4; d++)
                        o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(v_operand(hf, d), pb[hf], o[d], 0, 0, 0);
            }
        }
        buf ^= 1;
        __syncthreads();  // V(t) and the slots read; K(t+1), V(t+1) visible
    }

    if (!q_valid) return;
    const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;
    const size_t obase = ((size_t)my_q * n_q + qh) * HD + 128 * ds;
#pragma unroll
    for (int d = 0; d < 4; d++)
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const size_t at = obase + 32 * d + 8 * (i / 4) + 4 * hh + (i % 4);
            if constexpr (O16)
                static_cast<uint16_t *>(outv)[at] = __builtin_bit_cast(uint16_t, (_Float16)(o[d][i] * inv));
            else
                static_cast<float *>(outv)[at] = o[d][i] * inv;
        }
}

}  // namespace

int launch_attn_prefill_ipv(hipStream_t st, const float *q, const int8_t *kq, const uint16_t *ks,
                            const int8_t *vq, const uint16_t *vs_kb, float *out, int n_tok, int q0,
                            int n_q, int n_kv, int head_dim, float scale, const uint32_t *step) {
    SGQ_CHECK(head_dim == kHD, "attn_prefill_ipv: head_dim %d unsupported (128)", head_dim);
    SGQ_CHECK(n_tok > 0 && q0 >= 0, "attn_prefill_ipv: n_tok %d, q0 %d", n_tok, q0);
    SGQ_CHECK(n_kv > 0 && n_q > 0 && n_q % n_kv == 0, "attn_prefill_ipv: n_q %% n_kv != 0");
    SGQ_CHECK(((uintptr_t)q & 15) == 0 && ((uintptr_t)kq & 15) == 0 && ((uintptr_t)vq & 15) == 0 &&
                  ((uintptr_t)ks & 1) == 0 && ((uintptr_t)vs_kb & 1) == 0,
              "attn_prefill_ipv: misaligned operand");
    const int qtiles = (n_tok + kQT - 1) / kQT;
    const KvSource src{kq, vq, ks, vs_kb, 0, nullptr, nullptr, nullptr, nullptr};
    const int qpk = n_q / n_kv;
    if (kPrefillPairHeads && qpk % 2 == 0)
        hipLaunchKernelGGL((attn_prefill_kernel<2, true>), dim3(qtiles, n_q / 2), dim3(512), 0, st,
                           q, src, out, n_tok, q0, n_q, n_kv, 0, scale, qtiles, step);
    else
        hipLaunchKernelGGL((attn_prefill_kernel<1, true>), dim3(qtiles, n_q), dim3(256), 0, st, q,
                           src, out, n_tok, q0, n_q, n_kv, 0, scale, qtiles, step);
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}

int launch_attn_prefill_q8(hipStream_t st, const float *q, const int8_t *kq, const uint16_t *ks,
                           const int8_t *vq, const uint16_t *vs, float *out, int n_tok, int q0,
                           int n_q, int n_kv, int head_dim, int window, float scale, int ring,
                           const int8_t *ckq, const uint16_t *cks, const int8_t *cvq,
                           const uint16_t *cvs, const uint32_t *step) {
    SGQ_CHECK(head_dim == kHD || head_dim == 256 || head_dim == 512,
              "attn_prefill_q8: head_dim %d unsupported (128, 256, 512)", head_dim);
    SGQ_CHECK(n_tok > 0 && q0 >= 0, "attn_prefill_q8: n_tok %d, q0 %d", n_tok, q0);
    SGQ_CHECK(n_kv > 0 && n_q > 0 && n_q % n_kv == 0, "attn_prefill_q8: n_q %% n_kv != 0");
    SGQ_CHECK(window >= 0 && ring >= 0, "attn_prefill_q8: negative window or ring");
    SGQ_CHECK(ckq == nullptr || (cks && cvq && cvs && ((uintptr_t)ckq & 15) == 0 &&
                                 ((uintptr_t)cvq & 15) == 0),
              "attn_prefill_q8: incomplete or misaligned chunk pages");
    SGQ_CHECK(ring == 0 || ckq != nullptr, "attn_prefill_q8: a ring cache needs the chunk's pages");
    SGQ_CHECK(ring == 0 || window <= ring, "attn_prefill_q8: window %d exceeds the ring (%d)",
              window, ring);
    SGQ_CHECK(((uintptr_t)q & 15) == 0 && ((uintptr_t)kq & 15) == 0 && ((uintptr_t)vq & 15) == 0 &&
                  ((uintptr_t)ks & 1) == 0 && ((uintptr_t)vs & 1) == 0,
              "attn_prefill_q8: misaligned operand");
    const KvSource src{kq, vq, ks, vs, ring, ckq, cvq, cks, cvs};
    if (head_dim != kHD) {
        SGQ_CHECK(step == nullptr, "attn_prefill_q8: head_dim %d needs q0 from the host", head_dim);
        SGQ_CHECK(((uintptr_t)kq & 15) == 0 && ((uintptr_t)vq & 15) == 0,
                  "attn_prefill_q8: misaligned cache");
        const int qw = head_dim == 256 ? 128 : 64;  // queries per workgroup
        const int qt = (n_tok + qw - 1) / qw;
        const uint32_t *no_step = nullptr;
        const uint16_t *no_qs = nullptr;
        if (head_dim == 256)
            hipLaunchKernelGGL((attn_prefill_wide_kernel<256, kPfQ8>), dim3(qt, n_q), dim3(512), 0,
                               st, q, no_qs, src, out, n_tok, q0, no_step, n_q, n_kv, window, scale,
                               qt);
        else
            hipLaunchKernelGGL((attn_prefill_wide_kernel<512, kPfQ8>), dim3(qt, n_q), dim3(512), 0,
                               st, q, no_qs, src, out, n_tok, q0, no_step, n_q, n_kv, window, scale,
                               qt);
        SGQ_HIP(hipGetLastError());
        return SGQ_OK;
    }
    const int qtiles = (n_tok + kQT - 1) / kQT;
    const int qpk = n_q / n_kv;
    if (kPrefillPairHeads && qpk % 2 == 0)
        hipLaunchKernelGGL(attn_prefill_ws_kernel<2>, dim3(qtiles, n_q / 2), dim3(768), 0, st, q,
                           src, out, n_tok, q0, n_q, n_kv, window, scale, qtiles, step);
    else
        hipLaunchKernelGGL(attn_prefill_ws_kernel<1>, dim3(qtiles, n_q), dim3(512), 0, st, q, src,
                           out, n_tok, q0, n_q, n_kv, window, scale, qtiles, step);
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}

int launch_attn_prefill_pages(hipStream_t st, int fmt, const void *q, const uint16_t *q_scales,
                              const void *k, const uint16_t *k_scales, const void *v,
                              const uint16_t *v_scales, int ring, const void *ck, const void *cv,
                              const uint16_t *cks, const uint16_t *cvs, void *out, int n_tok,
                              const uint32_t *step, int n_q, int n_kv, int head_dim, int window,
                              float scale) {
    SGQ_CHECK(fmt == kPfQ8H || fmt == kPfF16 || fmt == kPfIQ || fmt == kPfIPV,
              "attn_prefill_pages: format %d", fmt);
    SGQ_CHECK(fmt != kPfIPV || (window == 0 && ring == 0 && v_scales),
              "attn_prefill_pages: int8 PV is causal over a linear cache with key-blocked V scales");
    SGQ_CHECK(head_dim == 256 || head_dim == 512, "attn_prefill_pages: head_dim %d (256, 512)",
              head_dim);
    SGQ_CHECK(q && k && v && out && step, "attn_prefill_pages: NULL operand");
    SGQ_CHECK(n_tok > 0 && n_kv > 0 && n_q > 0 && n_q % n_kv == 0,
              "attn_prefill_pages: n_tok %d, n_q %d, n_kv %d", n_tok, n_q, n_kv);
    SGQ_CHECK((fmt != kPfIQ && fmt != kPfIPV) || (q_scales && k_scales),
              "attn_prefill_pages: int8 q needs the scales");
    SGQ_CHECK(fmt != kPfQ8H || (k_scales && v_scales), "attn_prefill_pages: Q8_0 pages need scales");
    SGQ_CHECK(window >= 0 && ring >= 0 && (ring == 0 || (ck && cv && window <= ring)),
              "attn_prefill_pages: a ring needs the chunk's pages and a window within it");
    SGQ_CHECK(((uintptr_t)q & 15) == 0 && ((uintptr_t)k & 15) == 0 && ((uintptr_t)v & 15) == 0 &&
                  ((uintptr_t)ck & 15) == 0 && ((uintptr_t)cv & 15) == 0,
              "attn_prefill_pages: misaligned operand");
    const KvSource src{static_cast<const int8_t *>(k), static_cast<const int8_t *>(v), k_scales,
                       v_scales, ring, static_cast<const int8_t *>(ck),
                       static_cast<const int8_t *>(cv), cks, cvs};
    const int qw = head_dim == 256 ? 128 : 64;  // queries per workgroup
    const int qt = (n_tok + qw - 1) / qw;
    const dim3 grid(qt, n_q);
#define SGQ_PF_PAGES(HD, F)                                                                     \
    hipLaunchKernelGGL((attn_prefill_wide_kernel<HD, F>), grid, dim3(512), 0, st, q, q_scales, src, \
                       out, n_tok, 0, step, n_q, n_kv, window, scale, qt)
    if (head_dim == 256) {
        if (fmt == kPfQ8H) SGQ_PF_PAGES(256, kPfQ8H);
        else if (fmt == kPfF16) SGQ_PF_PAGES(256, kPfF16);
        else if (fmt == kPfIQ) SGQ_PF_PAGES(256, kPfIQ);
        else SGQ_PF_PAGES(256, kPfIPV);
    } else {
        if (fmt == kPfQ8H) SGQ_PF_PAGES(512, kPfQ8H);
        else if (fmt == kPfF16) SGQ_PF_PAGES(512, kPfF16);
        else if (fmt == kPfIQ) SGQ_PF_PAGES(512, kPfIQ);
        else SGQ_PF_PAGES(512, kPfIPV);
    }
#undef SGQ_PF_PAGES
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}

}  // namespace sgq
