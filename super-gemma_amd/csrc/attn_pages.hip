// Decode attention over the reference's own page formats for the released
// checkpoint's names (crates/sg-gpu/build.rs:255-394), so that its
// record_layer (crates/sg-model/src/graph.rs:572-650) dispatches unchanged:
//   attn_decode_sliding     f16 q, f16 K and V ring pages, head_dim 256,
//                           16 kv heads, 2 query heads per kv head, kv_len
//                           = step[1]   (attn_decode_sliding.wgsl:51-121)
//   attn_decode_global      the same at head_dim 512, 4 kv heads, 8 query
//                           heads per kv head, kv_len = step[2]
//   attn_decode_global_q8k  K from Q8_0 pages (i8 quants, f16 scale per
//                           32 dims), V f16  (attn_decode_global_q8k.wgsl)
//   attn_reduce_d256 / _d512   the split merge, f16 rows out (attn_reduce.wgsl)
//   kv_append_sliding / _global   f16 rows into the ring (slot = (pos + t)
//                           mod 1024) or the linear cache (kv_append.wgsl)
// Semantics: split s of kv head g covers slots [s·c, min(s·c + c, kv_len)),
// c = ceil(kv_len / n_splits), in physical slot order; score = (q·k)·scale;
// the partial (acc, m, l) of query head h at [(h·n_splits + s)·(head_dim +
// 2)] is the unnormalised softmax-weighted V sum, its max and its sum (an
// empty split: acc 0, m -3e38, l 0).  The model driver keeps Q8_0 K and V
// (csrc/attn_generic.hip); these serve callers that hold f16 pages.
//
// Design (MFMA; the reference's grid gives 128-256 workgroups, so each
// must use its CU well): one workgroup of head_dim/32 waves per (kv head,
// split) walks its chunk in tiles of 64 slots, with v_mfma_f32_32x32x16_f16
// for both products (query heads padded to the 32 MFMA columns):
//  * Sᵀ = K·Qᵀ: wave w takes slot block w & 1 (32 slots) and 64 dims; K
//    goes from HBM straight into the A operand (16 bytes a lane), q sits in
//    registers as the B operand.  f16 products are exact and Q8_0 quants
//    enter as their exact f16 values, each 32-dim block accumulated on its
//    own; the partials meet in LDS and are summed in dim order (times the
//    block's k scale for Q8_0) by one wave per query head, which runs the
//    tile's online-softmax step;
//  * Oᵀ = Vᵀ·Pᵀ: the V tile is staged in LDS (rows padded so the transposed
//    reads of rows 8 apart fall on other banks), wave w owns dims
//    [32w, 32w + 32) of every query head, and P enters as two f16 parts
//    (p = hi + lo, 22 bits) so the PV keeps fp32 accuracy;
//  * the next tile's V is requested as soon as this tile's V is in LDS
//    (before the scores), its K after the score MFMAs have consumed this
//    tile's K registers.
#include "sgq_internal.h"

namespace sgq {
namespace {

constexpr int kPTile = 64;  // slots per tile
constexpr float kPNegBig = -3.0e38f;

__device__ __forceinline__ float h2f(uint16_t b) {
    return (float)__builtin_bit_cast(_Float16, b);
}

typedef _Float16 ph8 __attribute__((ext_vector_type(8)));
typedef float pf16x __attribute__((ext_vector_type(16)));

// 8 int8 quants (two words) -> their exact f16 values.
__device__ __forceinline__ ph8 i8x8_f16(uint32_t w0, uint32_t w1) {
    ph8 r;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        r[e] = (_Float16)(float)(int8_t)(w0 >> (8 * e));
        r[4 + e] = (_Float16)(float)(int8_t)(w1 >> (8 * e));
    }
    return r;
}

template <int HD, int QPK, bool KQ8>
__global__ __launch_bounds__(HD * 2) void attn_decode_pages_kernel(
    const uint16_t *__restrict__ q16, const void *__restrict__ kp,
    const uint16_t *__restrict__ k_scales, const uint16_t *__restrict__ v16,
    float *__restrict__ part, const uint32_t *__restrict__ step, int step_word, int n_kv,
    int n_splits, float scale) {
    constexpr int NW = HD / 32;            // waves = PV dim blocks
    constexpr int NT = NW * 64;            // threads
    constexpr int NDG = NW / 2;            // score dim groups of 64 per slot block
    constexpr int NG = KQ8 ? 2 * NDG : NDG;  // score partials per slot
    constexpr int VP = HD + 8;             // V tile row pitch, halves
    constexpr int NU = kPTile * HD / 8 / NT;  // uint4 of V per thread per tile (4)
    static_assert(QPK <= 32 && NU == 4, "layout");
    __shared__ __align__(16) _Float16 vs_s[kPTile][VP];
    __shared__ float sp_s[NG][QPK][kPTile];
    __shared__ __align__(16) _Float16 ph_s[QPK][kPTile], pl_s[QPK][kPTile];
    __shared__ float m_s[QPK], l_s[QPK], corr_s[QPK];
    __shared__ __align__(16) uint32_t ks_s[KQ8 ? kPTile : 1][8];  // Q8_0 block scales per slot
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, hh = lane >> 5;
    const int kvh = blockIdx.x, split = blockIdx.y;
    const uint32_t kv_len = step[step_word];
    const uint32_t chunk = (kv_len + (uint32_t)n_splits - 1) / (uint32_t)n_splits;
    const uint32_t t_begin = min((uint32_t)split * chunk, kv_len);
    const uint32_t t_end = min(t_begin + chunk, kv_len);
    const size_t kv_row = (size_t)n_kv * HD;  // elements per slot
    const int sb = wave & 1, dg = wave >> 1;  // score role
    const bool hcol = l32 < QPK;              // this lane's MFMA column is a real head

    // q of head l32 on the wave's 64 score dims, as four B operands
    ph8 qb[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const uint4 w = hcol ? *reinterpret_cast<const uint4 *>(
                                   q16 + ((size_t)kvh * QPK + l32) * HD + 64 * dg + 16 * c + 8 * hh)
                             : make_uint4(0, 0, 0, 0);
        qb[c] = __builtin_bit_cast(ph8, w);
    }
    if (tid < QPK) m_s[tid] = kPNegBig, l_s[tid] = 0.f;
    pf16x acc;
#pragma unroll
    for (int i = 0; i < 16; i++) acc[i] = 0.f;

    // K (A operands) and V (staging words) of a tile, loaded ahead
    // (vector values, not arrays: arrays assigned on two paths stay in scratch)
    constexpr int KW = KQ8 ? 2 : 4;  // K words per A operand
    typedef uint32_t kv_t __attribute__((ext_vector_type(4 * KW)));
    typedef uint32_t vv_t __attribute__((ext_vector_type(4 * NU)));
    typedef uint32_t sv_t __attribute__((ext_vector_type(8)));
    kv_t kr;
    vv_t vr;
    sv_t ksr;  // Q8_0: the 16 block scales of slot `lane` (wave 0)
    auto load_k = [&](uint32_t t0) __attribute__((always_inline)) {
        const int n = (int)min((uint32_t)kPTile, t_end - t0);
        const size_t krow = (size_t)(t0 + min(32 * sb + l32, n - 1)) * n_kv + kvh;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const size_t off = krow * HD + 64 * dg + 16 * c + 8 * hh;
            if constexpr (KQ8) {
                const uint2 w = *reinterpret_cast<const uint2 *>(static_cast<const int8_t *>(kp) + off);
                kr[2 * c] = w.x, kr[2 * c + 1] = w.y;
            } else {
                const uint4 w = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(kp) + off);
                kr[4 * c] = w.x, kr[4 * c + 1] = w.y, kr[4 * c + 2] = w.z, kr[4 * c + 3] = w.w;
            }
        }
        if constexpr (KQ8)
            if (wave == 0) {
                const uint4 *kss = reinterpret_cast<const uint4 *>(
                    k_scales + ((size_t)(t0 + min(lane, n - 1)) * n_kv + kvh) * (HD / 32));
                const uint4 a = kss[0], b = kss[1];
                ksr[0] = a.x, ksr[1] = a.y, ksr[2] = a.z, ksr[3] = a.w;
                ksr[4] = b.x, ksr[5] = b.y, ksr[6] = b.z, ksr[7] = b.w;
            }
    };
    auto load_v = [&](uint32_t t0) __attribute__((always_inline)) {
        const int n = (int)min((uint32_t)kPTile, t_end - t0);
#pragma unroll
        for (int j = 0; j < NU; j++) {
            const int u = tid + j * NT, sl = u / (HD / 8), c8 = u % (HD / 8);
            const uint4 w = *reinterpret_cast<const uint4 *>(
                v16 + (size_t)(t0 + min(sl, n - 1)) * kv_row + (size_t)kvh * HD + 8 * c8);
            vr[4 * j] = w.x, vr[4 * j + 1] = w.y, vr[4 * j + 2] = w.z, vr[4 * j + 3] = w.w;
        }
    };
    if (t_begin < t_end) {
        load_k(t_begin);
        load_v(t_begin);
    }
    __syncthreads();

    for (uint32_t t0 = t_begin; t0 < t_end; t0 += kPTile) {
        const int n = (int)min((uint32_t)kPTile, t_end - t0);
        // ---- V into LDS; partial Sᵀ of the wave's slot block and dims
#pragma unroll
        for (int j = 0; j < NU; j++) {
            const int u = tid + j * NT, sl = u / (HD / 8), c8 = u % (HD / 8);
            *reinterpret_cast<uint4 *>(&vs_s[sl][8 * c8]) =
                make_uint4(vr[4 * j], vr[4 * j + 1], vr[4 * j + 2], vr[4 * j + 3]);
        }
        // the next tile's V as soon as this one's registers are free
        if (t0 + kPTile < t_end) load_v(t0 + kPTile);
        if constexpr (KQ8)
            if (wave == 0) {
                *reinterpret_cast<uint4 *>(&ks_s[lane][0]) = make_uint4(ksr[0], ksr[1], ksr[2], ksr[3]);
                *reinterpret_cast<uint4 *>(&ks_s[lane][4]) = make_uint4(ksr[4], ksr[5], ksr[6], ksr[7]);
            }
        pf16x d0, d1;
#pragma unroll
        for (int i = 0; i < 16; i++) d0[i] = d1[i] = 0.f;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            ph8 a;
            if constexpr (KQ8) a = i8x8_f16(kr[2 * c], kr[2 * c + 1]);
            else a = __builtin_bit_cast(ph8, make_uint4(kr[4 * c], kr[4 * c + 1], kr[4 * c + 2], kr[4 * c + 3]));
            if (KQ8 && c >= 2) d1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qb[c], d1, 0, 0, 0);
            else d0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qb[c], d0, 0, 0, 0);
        }
        if (hcol)
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int slot = 32 * sb + 8 * (i / 4) + 4 * hh + (i % 4);
                if constexpr (KQ8) {
                    sp_s[2 * dg][l32][slot] = d0[i];
                    sp_s[2 * dg + 1][l32][slot] = d1[i];
                } else {
                    sp_s[dg][l32][slot] = d0[i];
                }
            }
        if (t0 + kPTile < t_end) load_k(t0 + kPTile);  // the next tile's K, in flight
        __syncthreads();
        // ---- the tile's softmax step, one wave per query head (lane = slot)
        if (wave < QPK) {
            const int h = wave;
            float sum = 0.f;
            if constexpr (KQ8) {
                const uint4 ka = *reinterpret_cast<const uint4 *>(&ks_s[lane][0]);
                const uint4 kb = *reinterpret_cast<const uint4 *>(&ks_s[lane][4]);
                const uint32_t kw[8] = {ka.x, ka.y, ka.z, ka.w, kb.x, kb.y, kb.z, kb.w};
#pragma unroll
                for (int g = 0; g < NG; g++)
                    sum = __builtin_fmaf(h2f((uint16_t)(kw[g / 2] >> (16 * (g & 1)))), sp_s[g][h][lane], sum);
            } else {
#pragma unroll
                for (int g = 0; g < NG; g++) sum += sp_s[g][h][lane];
            }
            const float s = lane < n ? sum * scale : kPNegBig;
            float mt = s;
            for (int o = 32; o > 0; o >>= 1) mt = fmaxf(mt, __shfl_xor(mt, o, kWave));
            const float m_old = m_s[h];
            const float m_new = fmaxf(m_old, mt);
            const float p = lane < n ? expf(s - m_new) : 0.f;
            float ps = p;
            for (int o = 32; o > 0; o >>= 1) ps += __shfl_xor(ps, o, kWave);
            const _Float16 phi = (_Float16)p;
            ph_s[h][lane] = phi;
            pl_s[h][lane] = (_Float16)(p - (float)phi);
            if (lane == 0) {
                const float corr = expf(m_old - m_new);  // the first tile: exp(-3e38 - m) = 0
                corr_s[h] = corr;
                l_s[h] = l_s[h] * corr + ps;
                m_s[h] = m_new;
            }
        }
        __syncthreads();
        // ---- Oᵀ(dims 32·wave.., heads) += Vᵀ·Pᵀ over the tile's 64 slots
        {
            const float c = corr_s[hcol ? l32 : 0];
#pragma unroll
            for (int i = 0; i < 16; i++) acc[i] *= c;
#pragma unroll
            for (int c4 = 0; c4 < 4; c4++) {
                const int s0 = 16 * c4 + 8 * hh;
                ph8 a;
#pragma unroll
                for (int e = 0; e < 8; e++) a[e] = vs_s[s0 + e][32 * wave + l32];
                const ph8 bh = hcol ? *reinterpret_cast<const ph8 *>(&ph_s[l32][s0]) : ph8{};
                const ph8 bl = hcol ? *reinterpret_cast<const ph8 *>(&pl_s[l32][s0]) : ph8{};
                acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bh, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bl, acc, 0, 0, 0);
            }
        }
        __syncthreads();  // vs_s, sp_s and the P tiles are rewritten by the next tile
    }

    constexpr int stride = HD + 2;
    if (hcol) {
        float *pp = part + ((size_t)(kvh * QPK + l32) * n_splits + split) * stride + 32 * wave;
#pragma unroll
        for (int i = 0; i < 16; i++) pp[8 * (i / 4) + 4 * hh + (i % 4)] = acc[i];
    }
    if (tid < QPK) {
        float *pp = part + ((size_t)(kvh * QPK + tid) * n_splits + split) * stride;
        pp[HD] = m_s[tid];
        pp[HD + 1] = l_s[tid];
    }
}

// The split merge (attn_reduce.wgsl:33-56 folds the splits in order with a
// running max; the same sum, weighted by exp(m_s - max over all splits)):
// out = f16(sum_s e^(m_s - M)·acc_s / sum_s e^(m_s - M)·l_s).  One 256-thread
// workgroup per query head: wave 0 loads every split's (m, l) at once (a
// lane per split, up to 64 at a time), takes the max over the wave and
// leaves the weights in LDS; then every thread folds its dims over the
// splits in order, all loads of a batch of 16 issued together.
template <int HD>
__global__ __launch_bounds__(256) void attn_reduce_pages_kernel(const float *__restrict__ part,
                                                                 int n_splits,
                                                                 uint16_t *__restrict__ out) {
    constexpr int ND = HD / 256, stride = HD + 2;
    __shared__ float w_s[64];
    __shared__ float l_s[1];
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
    const float *ph = part + (size_t)h * n_splits * stride;
    float acc[ND];
#pragma unroll
    for (int e = 0; e < ND; e++) acc[e] = 0.f;
    float M = kPNegBig;  // wave 0: the max over all splits so far (chunks of 64)
    float lsum = 0.f;
    for (int s0 = 0; s0 < n_splits; s0 += 64) {
        const int cnt = min(64, n_splits - s0);
        if (tid < 64) {
            const float m = lane < cnt ? ph[(size_t)(s0 + lane) * stride + HD] : kPNegBig;
            const float l = lane < cnt ? ph[(size_t)(s0 + lane) * stride + HD + 1] : 0.f;
            float mx = m;
            for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
            const float Mn = fmaxf(M, mx);
            const float r = expf(M - Mn);  // rescale of the chunks before
            const float w = lane < cnt ? expf(m - Mn) : 0.f;
            float lw = w * l;
            for (int o = 32; o > 0; o >>= 1) lw += __shfl_xor(lw, o, kWave);
            lsum = lsum * r + lw;
            M = Mn;
            w_s[lane] = w;
            if (lane == 0) l_s[0] = r;
        }
        __syncthreads();
        const float r = l_s[0];
#pragma unroll
        for (int e = 0; e < ND; e++) acc[e] *= r;
        for (int b = 0; b < cnt; b += 16) {
            float v[16][ND];
#pragma unroll
            for (int u = 0; u < 16; u++)
#pragma unroll
                for (int e = 0; e < ND; e++)
                    v[u][e] = b + u < cnt ? ph[(size_t)(s0 + b + u) * stride + tid * ND + e] : 0.f;
#pragma unroll
            for (int u = 0; u < 16; u++) {
                const float w = b + u < cnt ? w_s[b + u] : 0.f;
#pragma unroll
                for (int e = 0; e < ND; e++) acc[e] = __builtin_fmaf(w, v[u][e], acc[e]);
            }
        }
        __syncthreads();  // w_s rewritten by the next chunk
    }
    if (tid == 0) l_s[0] = lsum;
    __syncthreads();
    const float l = l_s[0];
    // every split empty (kv_len 0): l = 0 and acc = 0; the output is 0, not
    // the 0/0 that attn_reduce.wgsl's acc/l would give
#pragma unroll
    for (int e = 0; e < ND; e++)
        out[(size_t)h * HD + tid * ND + e] =
            __builtin_bit_cast(uint16_t, (_Float16)(l > 0.f ? acc[e] / l : 0.f));
}

// f16 rows [n_tok × row] to slot step[0] + t (mod ring when ring > 0); eight
// halves per thread.
__global__ __launch_bounds__(256) void kv_append_f16_kernel(const uint4 *__restrict__ src,
                                                            uint4 *__restrict__ dst,
                                                            const uint32_t *__restrict__ step,
                                                            uint64_t n8, uint32_t row8,
                                                            uint32_t ring) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n8) return;
    const uint32_t t = (uint32_t)(i / row8), j = (uint32_t)(i % row8);
    const uint32_t slot = ring ? (step[0] + t) % ring : step[0] + t;
    dst[(size_t)slot * row8 + j] = src[i];
}

}  // namespace

int launch_attn_decode_pages(hipStream_t st, const uint16_t *q, const void *k,
                             const uint16_t *k_scales, const uint16_t *v, float *part,
                             const uint32_t *step, int step_word, int head_dim, int n_q, int n_kv,
                             int n_splits, float scale) {
    SGQ_CHECK(q && k && v && part && step, "attn_decode_pages: NULL operand");
    SGQ_CHECK(n_kv > 0 && n_q % n_kv == 0, "attn_decode_pages: n_q %% n_kv != 0");
    SGQ_CHECK(n_splits >= 1 && n_splits <= 65535, "attn_decode_pages: n_splits %d", n_splits);
    SGQ_CHECK(((uintptr_t)q & 15) == 0 && ((uintptr_t)k & 15) == 0 && ((uintptr_t)v & 15) == 0 &&
                  ((uintptr_t)k_scales & 15) == 0,
              "attn_decode_pages: q, the pages and the K scales must be 16-byte aligned");
    const int qpk = n_q / n_kv;
    const dim3 grid(n_kv, n_splits);
    if (head_dim == 256 && qpk == 2 && !k_scales)
        hipLaunchKernelGGL((attn_decode_pages_kernel<256, 2, false>), grid, dim3(512), 0, st, q, k,
                           k_scales, v, part, step, step_word, n_kv, n_splits, scale);
    else if (head_dim == 512 && qpk == 8 && !k_scales)
        hipLaunchKernelGGL((attn_decode_pages_kernel<512, 8, false>), grid, dim3(1024), 0, st, q, k,
                           k_scales, v, part, step, step_word, n_kv, n_splits, scale);
    else if (head_dim == 512 && qpk == 8 && k_scales)
        hipLaunchKernelGGL((attn_decode_pages_kernel<512, 8, true>), grid, dim3(1024), 0, st, q, k,
                           k_scales, v, part, step, step_word, n_kv, n_splits, scale);
    else
        return fail(SGQ_ERR_VALIDATION,
                    "attn_decode_pages: head_dim %d with %d query heads per kv head (%s K) is "
                    "not a built variant", head_dim, qpk, k_scales ? "Q8_0" : "f16");
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}

int launch_attn_reduce_pages(hipStream_t st, const float *part, int n_q, int head_dim,
                             int n_splits, uint16_t *out) {
    SGQ_CHECK(part && out && n_q > 0 && n_splits >= 1, "attn_reduce_pages: bad operands");
    if (head_dim == 256)
        hipLaunchKernelGGL(attn_reduce_pages_kernel<256>, dim3(n_q), dim3(256), 0, st, part,
                           n_splits, out);
    else if (head_dim == 512)
        hipLaunchKernelGGL(attn_reduce_pages_kernel<512>, dim3(n_q), dim3(256), 0, st, part,
                           n_splits, out);
    else
        return fail(SGQ_ERR_VALIDATION, "attn_reduce_pages: head_dim %d (256 / 512)", head_dim);
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}

int launch_kv_append_f16(hipStream_t st, const uint16_t *src, uint16_t *dst,
                         const uint32_t *step, uint32_t n_tok, uint32_t row, uint32_t ring) {
    SGQ_CHECK(src && dst && step, "kv_append_f16: NULL operand");
    SGQ_CHECK(row % 8 == 0 && ((uintptr_t)src & 15) == 0 && ((uintptr_t)dst & 15) == 0,
              "kv_append_f16: rows must be 16-byte aligned multiples of 8 halves");
    const uint64_t n8 = (uint64_t)n_tok * (row / 8);
    if (n8 == 0) return SGQ_OK;
    hipLaunchKernelGGL(kv_append_f16_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, st,
                       reinterpret_cast<const uint4 *>(src), reinterpret_cast<uint4 *>(dst), step,
                       n8, row / 8, ring);
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}

}  // namespace sgq
