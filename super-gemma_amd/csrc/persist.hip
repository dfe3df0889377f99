// Persistent decode step: the whole forward pass of one token in one
// cooperative launch of one 512-thread workgroup per CU.
//
// Same semantics as the multi-kernel decode step (crates/sg-model/src/
// reference.rs:157-316; graph.rs:478-756 record_layer / record_logits),
// restaged so that the weight stream never stops at a stage boundary:
//
//   per layer   QKV GEMV | attention (+ merge) | O GEMV | post-attn reduce |
//               gate/up GEMV + GeGLU | h limbs | down GEMV | post-FFN reduce |
//
// where "|" is a grid barrier (software, two-level agent-scope counters).
// Before a workgroup waits at a barrier it has already issued the first
// ring slots of its next GEMV (global_load_lds into LDS; the data never
// needs registers), so weights stream during barriers, reductions and
// attention: the O projection is prefetched whole while attention runs in
// the other half of LDS, QKV while the post-FFN reduction runs.
//
// Norms move to small reduce stages that own 32-element blocks: each
// computes the global sum of squares it needs itself (every workgroup in
// the same fixed order, so all agree bit for bit), updates its block of the
// residual, writes the block's x limbs for the next GEMV and its block's
// partial sum of squares; the consumer GEMV turns the partials into the
// RMS factor and applies it to its outputs (a GEMV is linear in x).
//
// Memory protocol (multi-XCD: per-XCD L2s are not coherent with each
// other): everything a stage hands to another workgroup is written with
// agent-scope stores (write-through), into buffers written once per launch
// (one arena region per layer), and only read after the barrier that
// follows the write: such addresses were never cached by any L2 in this
// launch, and kernel boundaries invalidate stale lines from earlier
// launches, so plain (cacheable) loads see the new data.  Counters are
// agent-scope atomics.  Every spin is bounded and watches an error flag, so
// a workgroup that cannot proceed makes every other one exit.
#include <algorithm>

#include "attn_body.h"
#include "persist.h"
#include "ring.h"

namespace sgq {
namespace {

constexpr int kPWG = 512;                    // threads per workgroup
constexpr int kPWaves = kPWG / kWave;        // 8 waves
constexpr int kPRing = kRStages * kPWaves * kRSlot;  // 144 KB: ring, slot-major
constexpr int kPAttnOff = 3 * kPWaves * kRSlot;      // attention: ring slots 3..5
constexpr int kSpin = 1 << 22;               // barrier poll bound (~seconds)

__device__ __forceinline__ unsigned ld_agent_u32(const unsigned *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int ld_agent_i32(const int *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent_f4(float *p, float4 v) {
    st_agent(p, v.x);
    st_agent(p + 1, v.y);
    st_agent(p + 2, v.z);
    st_agent(p + 3, v.w);
}
__device__ __forceinline__ float gelu_tanh_p(float x) {
    const float k = 0.7978845608028654f;
    return 0.5f * x * (1.f + tanhf(k * (x + 0.044715f * x * x * x)));
}

// Grid barrier.  The caller has waited for its own stores (vmcnt) in every
// wave.  Group counters (8 of them, one per XCD under round-robin dispatch)
// take the arrivals; the last arrival of a group bumps the global counter,
// which everyone polls.  Returns false (after flagging) when the barrier
// does not complete or another workgroup flagged an error.
__device__ __forceinline__ bool grid_sync(unsigned *sync, int *err, unsigned &epoch) {
    __shared__ int ok_s;
    epoch++;
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned G = gridDim.x;
        const unsigned groups = G % 8 == 0 ? 8u : 1u, per = G / groups;
        const unsigned grp = blockIdx.x % groups;
        const unsigned old = __hip_atomic_fetch_add(sync + 16 * (1 + grp), 1u, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT);
        if (old + 1 == epoch * per)
            __hip_atomic_fetch_add(sync, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        int ok = 1;
        for (int i = 0; ld_agent_u32(sync) < epoch * groups; i++) {
            if (i >= kSpin || ld_agent_i32(err)) {
                ok = 0;
                __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        ok_s = ok;
    }
    __syncthreads();
    return ok_s != 0;
}

// Sum over the 512-thread workgroup in a fixed order.
__device__ __forceinline__ float wg_sum(float v) {
    __shared__ float red_s[kPWaves];
    v = wave_sum_dpp(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red_s[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = 0.f;
#pragma unroll
    for (int w = 0; w < kPWaves; w++) r += red_s[w];
    return r;
}

// ---- streamed GEMV over the persistent ring ------------------------------

// A GEMV stage: up to 3 matrices sharing x, their rows concatenated
// (rows [end[j-1], end[j]) are matrix j), or, in GeGLU mode, gate and up
// interleaved per unit (unit i = gate row i then up row i on one wave).
struct Stage {
    const void *w0, *w1, *w2;  // scalar fields, not arrays: a runtime index
    float *y0, *y1, *y2;       // into an array member puts the struct in scratch
    int end0, end1, end2;
    int count;
    int n;         // units: rows, or GeGLU pairs
    int nb;        // 32-blocks per row
    int S, slice;  // K-slices and blocks per slice
    int geglu;
    float softcap;
    const BlockLimbs *xl;  // x limb table
};

struct WaveGeo {
    int s, P, U, u0, rounds, slice_off, slice_blocks, b0;
    int doff[kRLoads];
};

__device__ __forceinline__ WaveGeo wave_geo(const Stage &st, int wave, int lane) {
    WaveGeo g;
    g.s = wave % st.S;
    const int rw = wave / st.S;
    g.P = kPWaves / st.S;
    g.U = gridDim.x * g.P;
    g.u0 = blockIdx.x * g.P + rw;
    int units;
    if (st.S == 1) {
        units = g.u0 < st.n ? (st.n - g.u0 + g.U - 1) / g.U : 0;
    } else {  // the waves of a row meet at a barrier: workgroup-uniform count
        const int first = blockIdx.x * g.P;
        units = first < st.n ? (st.n - first + g.U - 1) / g.U : 0;
    }
    g.rounds = units * (st.geglu ? 2 : 1);
    g.b0 = g.s * st.slice;
    g.slice_blocks = min(st.slice, st.nb - g.b0);
    g.slice_off = g.b0 * 18;
    const int slice_bytes = g.slice_blocks * 18;
#pragma unroll
    for (int i = 0; i < kRLoads; i++) {
        const int off = (i * kWave + lane) * 16;
        g.doff[i] = off + 16 > slice_bytes ? 0 : off;
    }
    return g;
}

__device__ __forceinline__ uint8_t *ring_slot(uint8_t *ring, int slot, int wave) {
    return ring + (slot * kPWaves + wave) * kRSlot;
}

// Unit of ring iteration `it` (may be >= n: such rounds load row 0 and
// store nothing).
__device__ __forceinline__ int unit_of(const Stage &st, const WaveGeo &g, int it) {
    return g.u0 + (st.geglu ? (it >> 1) : it) * g.U;
}

// Wave-uniform copies of a stage's matrix and output pointers (selected
// among as values: selecting among struct members turns into an indexed
// load from a stack copy of the struct).
struct Ptrs {
    const uint8_t *w0, *w1, *w2;
    float *y0, *y1, *y2;
};
__device__ __forceinline__ const uint8_t *uni(const void *p) {
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<const uint8_t *>(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ Ptrs ptrs_of(const Stage &st) {
    return Ptrs{uni(st.w0), uni(st.w1), uni(st.w2), (float *)uni(st.y0), (float *)uni(st.y1),
                (float *)uni(st.y2)};
}

__device__ __forceinline__ void issue(const Stage &st, const Ptrs &pt, const WaveGeo &g,
                                      uint8_t *ring, int wave, int it) {
    int unit = unit_of(st, g, it);
    if (unit >= st.n) unit = 0;
    int j, local;
    if (st.geglu) {
        j = it & 1;
        local = unit;
    } else {
        j = st.count > 1 && unit >= st.end0 ? (st.count > 2 && unit >= st.end1 ? 2 : 1) : 0;
        local = unit - (j == 0 ? 0 : j == 1 ? st.end0 : st.end1);
    }
    const uint8_t *wj = j == 0 ? pt.w0 : j == 1 ? pt.w1 : pt.w2;
    const uint8_t *src = wj + (size_t)local * st.nb * 18 + g.slice_off;
    uint8_t *slot = ring_slot(ring, it % kRStages, wave);
#pragma unroll
    for (int i = 0; i < kRLoads; i++)
        __builtin_amdgcn_global_load_lds((gvoid_t *)(src + g.doff[i]),
                                         (lvoid_t *)(slot + i * kWave * 16), 16, 0,
                                         kStreamPolicy);
}

// Issue the first min(npf, rounds) ring slices of a stage (the prefetch
// done before a barrier).  Returns the number of DMA loads issued.
__device__ __forceinline__ int gemv_prefetch(const Stage &st, uint8_t *ring, int npf) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const WaveGeo g = wave_geo(st, wave, lane);
    const Ptrs pt = ptrs_of(st);
    const int n = min(npf, g.rounds);
    for (int it = 0; it < n; it++) issue(st, pt, g, ring, wave, it);
    return n * kRLoads;
}

__device__ __forceinline__ void wait_vm(int n_after) {
    switch (n_after) {
        case 5: __builtin_amdgcn_s_waitcnt(vmcnt_imm(kRLoads * 5)); break;
        case 4: __builtin_amdgcn_s_waitcnt(vmcnt_imm(kRLoads * 4)); break;
        case 3: __builtin_amdgcn_s_waitcnt(vmcnt_imm(kRLoads * 3)); break;
        case 2: __builtin_amdgcn_s_waitcnt(vmcnt_imm(kRLoads * 2)); break;
        case 1: __builtin_amdgcn_s_waitcnt(vmcnt_imm(kRLoads * 1)); break;
        default: __builtin_amdgcn_s_waitcnt(vmcnt_imm(0)); break;
    }
}

// Run a stage whose first `npf` slices were issued by gemv_prefetch with the
// same Stage.  Outputs are scaled by `r` (wave-uniform), capped by softcap,
// and stored with agent-scope stores.
template <int NBL>
__device__ __forceinline__ void gemv_run(const Stage &st, uint8_t *ring, int npf, float r) {
    __shared__ float part_s[2][kPWaves];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const WaveGeo g = wave_geo(st, wave, lane);
    const Ptrs pt = ptrs_of(st);
    XLimbs<NBL> L;
    int boff[NBL];
#pragma unroll
    for (int i = 0; i < NBL; i++) {
        const int lb = lane + kWave * i;
        const bool valid = lb < g.slice_blocks;
        boff[i] = valid ? lb * 18 - (lane & 1) * 2 : (lane & 1) * 16;
        BlockLimbs t = valid ? st.xl[g.b0 + lb] : BlockLimbs{};
#pragma unroll
        for (int l = 0; l < kLimbs; l++)
#pragma unroll
            for (int w = 0; w < 4; w++) L.q[i][l][w] = t.q[l][w];
        L.d[i] = t.d;
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    const uint32_t sel = (lane & 1) ? 0x07060504u : 0x05040302u;
    const uint32_t dshift = (lane & 1) ? 16u : 0u;
    int issued = min(npf, g.rounds);
    float gate = 0.f;
    for (int it = 0; it < g.rounds; it++) {
        while (issued < g.rounds && issued <= it + kRStages - 1) issue(st, pt, g, ring, wave, issued++);
        wait_vm(issued - it - 1);
        uint32_t wv[NBL][5];
        lds_read_blocks<NBL>(ring_slot(ring, it % kRStages, wave), boff, wv);
        float a = 0.f;
#pragma unroll
        for (int i = 0; i < NBL; i++) a += block_dot(wv[i], sel, dshift, L, i);
        a = wave_sum_dpp(a);
        const int unit = unit_of(st, g, it);
        bool have = true;
        if (st.S > 1) {  // slices of one row meet in LDS, summed in slice order
            uint8_t *rb = reinterpret_cast<uint8_t *>(part_s[it & 1]);
            if (lane == 0) lds_write_f32(rb + wave * 4, a);
            __builtin_amdgcn_s_barrier();
            have = g.s == 0;
            if (have) {
                const int base = wave - g.s;
                float v = 0.f;
                for (int q = 0; q < st.S; q++) v += lds_read_f32(rb + (base + q) * 4);
                a = v;
            }
        }
        if (!have || unit >= st.n) continue;
        a *= r;
        if (st.geglu) {
            if ((it & 1) == 0) {
                gate = a;
            } else if (lane == 0) {
                st_agent(pt.y0 + unit, gelu_tanh_p(gate) * a);
            }
            continue;
        }
        if (lane == 0) {
            const int j =
                st.count > 1 && unit >= st.end0 ? (st.count > 2 && unit >= st.end1 ? 2 : 1) : 0;
            const int local = unit - (j == 0 ? 0 : j == 1 ? st.end0 : st.end1);
            if (st.softcap > 0.f) a = st.softcap * tanhf(a / st.softcap);
            float *yj = j == 0 ? pt.y0 : j == 1 ? pt.y1 : pt.y2;
            st_agent(yj + local, a);
        }
    }
}

__device__ __forceinline__ void gemv_run_any(const Stage &st, uint8_t *ring, int npf, float r) {
    const int nbl = (st.slice + kWave - 1) / kWave;
    if (nbl == 1) gemv_run<1>(st, ring, npf, r);
    else if (nbl == 2) gemv_run<2>(st, ring, npf, r);
    else gemv_run<3>(st, ring, npf, r);
}

// RMS factor 1/sqrt(Σ ss / n + eps) from per-block partial sums (every wave
// adds them in the same fixed order).
__device__ __forceinline__ float rms_from_partials(const float *ss, int nblk, int n, float eps) {
    const int lane = threadIdx.x & 63;
    float v = 0.f;
    for (int b = lane; b < nblk; b += kWave) v += ss[b];
    v = wave_sum_dpp(v);
    return 1.0f / sqrtf(v / (float)n + eps);
}

// ---- reduce stages: one 8-lane group per 32-block -----------------------

// 1/sqrt(mean(v²)+eps) over a whole vector, fixed order (all workgroups
// compute the same value).
__device__ __forceinline__ float rms_of(const float *v, int n, float eps) {
    float s = 0.f;
    for (int i = threadIdx.x; i < n / 4; i += kPWG) {
        const float4 a = reinterpret_cast<const float4 *>(v)[i];
        s += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
    }
    return 1.0f / sqrtf(wg_sum(s) / (float)n + eps);
}

__device__ __forceinline__ float group8_sum(float v) {
    v += __shfl_xor(v, 1, kWave);
    v += __shfl_xor(v, 2, kWave);
    v += __shfl_xor(v, 4, kWave);
    return v;
}

// Blocks of this workgroup: [b_begin, b_end) with one 8-lane group each.
struct BlockRange {
    int b, e;  // this thread's block and float4 lane (0..7); b < 0: idle
};
__device__ __forceinline__ BlockRange block_of(int nblk) {
    const int per = (nblk + gridDim.x - 1) / gridDim.x;
    const int j = threadIdx.x >> 3;
    BlockRange br{-1, (int)threadIdx.x & 7};
    const int b = blockIdx.x * per + j;
    if (j < per && b < nblk) br.b = b;
    return br;
}

__device__ __forceinline__ float4 ld4(const float *p, int i) {
    return reinterpret_cast<const float4 *>(p)[i];
}
__device__ __forceinline__ float4 mul4(float4 a, float4 b) {
    return make_float4(a.x * b.x, a.y * b.y, a.z * b.z, a.w * b.w);
}

// Residual update + next norm's limbs:
//   post == nullptr:  xn = x_in                          (embedding handled by caller)
//   else:             xn = (x_in + r·o∘w_post)·scale     with r = rms(o)
// then  x_out = xn,  limbs(xn∘w_next) -> xl,  Σ_block xn² -> ss.
__device__ __forceinline__ void residual_stage(const float *o, const float *w_post, const float *x_in,
                               const float *scale_p, const float *w_next, float *x_out,
                               BlockLimbs *xl, float *ss, int H, float eps) {
    const int nblk = H / 32;
    const BlockRange br = block_of(nblk);
    if (__syncthreads_or(br.b >= 0) == 0) return;
    const float r = rms_of(o, H, eps);
    if (br.b < 0) return;
    const int i = br.b * 8 + br.e;
    const float s = scale_p ? *scale_p : 1.f;
    const float4 ov = ld4(o, i), wp = ld4(w_post, i), xv = ld4(x_in, i);
    float4 xn;
    xn.x = (xv.x + ov.x * r * wp.x) * s;
    xn.y = (xv.y + ov.y * r * wp.y) * s;
    xn.z = (xv.z + ov.z * r * wp.z) * s;
    xn.w = (xv.w + ov.w * r * wp.w) * s;
    st_agent_f4(x_out + 4 * i, xn);
    limbs_block8<true>(mul4(xn, ld4(w_next, i)), br.e, &xl[br.b]);
    const float b2 = group8_sum(xn.x * xn.x + xn.y * xn.y + xn.z * xn.z + xn.w * xn.w);
    if (br.e == 0) st_agent(ss + br.b, b2);
}

// x0 = dequant(E[token])·scale; limbs(x0∘w) -> xl; Σ_block x0² -> ss.
__device__ __forceinline__ void embed_stage(const uint8_t *E, uint32_t token, float scale, const float *w,
                            float *x_out, BlockLimbs *xl, float *ss, int H) {
    const BlockRange br = block_of(H / 32);
    if (br.b < 0) return;
    const uint8_t *blk = E + ((size_t)token * (H / 32) + br.b) * 18;
    const float d = f16_bits_to_f32(blk[0] | (blk[1] << 8));
    const int j0 = 4 * br.e;
    const int sh = j0 < 16 ? 0 : 4;
    const uint8_t *qs = blk + 2 + (j0 & 15);
    float e[4];
#pragma unroll
    for (int u = 0; u < 4; u++) e[u] = d * (float)(((qs[u] >> sh) & 15) - 8) * scale;
    const float4 x0 = make_float4(e[0], e[1], e[2], e[3]);
    const int i = br.b * 8 + br.e;
    st_agent_f4(x_out + 4 * i, x0);
    limbs_block8<true>(mul4(x0, ld4(w, i)), br.e, &xl[br.b]);
    const float b2 = group8_sum(x0.x * x0.x + x0.y * x0.y + x0.z * x0.z + x0.w * x0.w);
    if (br.e == 0) st_agent(ss + br.b, b2);
}

// limbs of h (F values) -> hl.
__device__ __forceinline__ void limbs_stage(const float *h, BlockLimbs *hl, int F) {
    const BlockRange br = block_of(F / 32);
    if (br.b < 0) return;
    limbs_block8<true>(ld4(h, br.b * 8 + br.e), br.e, &hl[br.b]);
}

// ---- the kernel ------------------------------------------------------------

__device__ __forceinline__ uint8_t *region(const PParams &p, int layer) {
    return p.arena + (size_t)layer * p.ar.stride;
}
template <typename T>
__device__ __forceinline__ T *at(uint8_t *base, size_t off) {
    return reinterpret_cast<T *>(base + off);
}

// Stores issued before `loads_after` later DMA loads are complete once
// vmcnt <= loads_after (gfx9 counts and retires vector memory ops in order).
__device__ __forceinline__ void wait_stores_before(int loads_after) {
    switch (loads_after) {
        case 0: __builtin_amdgcn_s_waitcnt(vmcnt_imm(0)); break;
        case kRLoads * 1: __builtin_amdgcn_s_waitcnt(vmcnt_imm(kRLoads * 1)); break;
        case kRLoads * 2: __builtin_amdgcn_s_waitcnt(vmcnt_imm(kRLoads * 2)); break;
        case kRLoads * 3: __builtin_amdgcn_s_waitcnt(vmcnt_imm(kRLoads * 3)); break;
        case kRLoads * 4: __builtin_amdgcn_s_waitcnt(vmcnt_imm(kRLoads * 4)); break;
        default: __builtin_amdgcn_s_waitcnt(vmcnt_imm(kRLoads * 5)); break;
    }
}

template <int QPK>
__global__ __launch_bounds__(kPWG) void decode_persistent_kernel(PParams p) {
    extern __shared__ __align__(16) uint8_t ring[];
    __shared__ __align__(16) float o_s[QPK * kHD];
    __shared__ int last_s;
    unsigned epoch = 0;
    const PArena &A = p.ar;
    const int H = p.H, F = p.F, QD = p.QD, KD = p.KD;
    const uint32_t pos = p.step[0], token = p.step[4];

    auto qkv_stage = [&](int l) {
        const PLayer &L = p.layers[l];
        uint8_t *R = region(p, l);
        Stage s{};
        s.w0 = L.wq, s.w1 = L.wk, s.w2 = L.wv;
        float *qkv = at<float>(R, A.qkv);
        s.y0 = qkv, s.y1 = qkv + QD, s.y2 = qkv + QD + KD;
        s.end0 = QD, s.end1 = QD + KD, s.end2 = QD + 2 * KD;
        s.count = L.wv ? 3 : 2;
        s.n = L.wv ? s.end2 : s.end1;
        s.nb = H / 32, s.S = p.s_h, s.slice = p.slice_h;
        s.xl = at<BlockLimbs>(R, A.xl_attn);
        return s;
    };
    auto o_stage = [&](int l) {
        uint8_t *R = region(p, l);
        Stage s{};
        s.w0 = p.layers[l].wo, s.y0 = at<float>(R, A.y), s.end0 = H, s.count = 1, s.n = H;
        s.nb = QD / 32, s.S = p.s_q, s.slice = p.slice_q;
        s.xl = at<BlockLimbs>(R, A.xl_o);
        return s;
    };
    auto gu_stage = [&](int l) {
        uint8_t *R = region(p, l);
        Stage s{};
        s.w0 = p.layers[l].wg, s.w1 = p.layers[l].wu, s.y0 = at<float>(R, A.h);
        s.count = 2, s.n = F, s.geglu = 1;
        s.nb = H / 32, s.S = p.s_h, s.slice = p.slice_h;
        s.xl = at<BlockLimbs>(R, A.xl_ffn);
        return s;
    };
    auto down_stage = [&](int l) {
        uint8_t *R = region(p, l);
        Stage s{};
        s.w0 = p.layers[l].wd, s.y0 = at<float>(R, A.d), s.end0 = H, s.count = 1, s.n = H;
        s.nb = F / 32, s.S = p.s_f, s.slice = p.slice_f;
        s.xl = at<BlockLimbs>(R, A.xl_h);
        return s;
    };
    auto head_stage = [&]() {
        uint8_t *R = region(p, p.n_layers);
        Stage s{};
        s.w0 = p.embd, s.y0 = p.logits, s.end0 = p.vocab, s.count = 1, s.n = p.vocab;
        s.nb = H / 32, s.S = p.s_h, s.slice = p.slice_h;
        s.softcap = p.softcap;
        s.xl = at<BlockLimbs>(R, A.xl_attn);
        return s;
    };
    // every wave: prefetch, then wait for the stores issued before it
#define SGQ_SYNC_AFTER_PREFETCH(STAGE, NPF)                       \
    {                                                             \
        const int _n = gemv_prefetch((STAGE), ring, (NPF));       \
        wait_stores_before(_n);                                   \
        if (!grid_sync(p.sync, p.err, epoch)) return;             \
    }
#define SGQ_SYNC()                                                \
    {                                                             \
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));                 \
        if (!grid_sync(p.sync, p.err, epoch)) return;             \
    }

    // embedding -> x_0, limbs of its attention norm input
    {
        const Stage q0 = qkv_stage(0);
        (void)gemv_prefetch(q0, ring, kRStages - 1);
        uint8_t *R = region(p, 0);
        embed_stage(p.embd, token, p.embed_scale, p.layers[0].attn_norm, at<float>(R, A.x),
                    at<BlockLimbs>(R, A.xl_attn), at<float>(R, A.ss_attn), H);
        SGQ_SYNC()
    }
    for (int l = 0; l < p.n_layers; l++) {
        const PLayer &L = p.layers[l];
        uint8_t *R = region(p, l);
        // QKV
        {
            const float r = rms_from_partials(at<float>(R, A.ss_attn), H / 32, H, p.eps);
            gemv_run_any(qkv_stage(l), ring, kRStages - 1, r);
            SGQ_SYNC()
        }
        // attention (+ merge by the last split of each kv head); the O
        // projection streams into ring slots 0..2 meanwhile
        {
            const Stage os = o_stage(l);
            (void)gemv_prefetch(os, ring, 3);
            const float *qkv = at<float>(R, A.qkv);
            float *part = at<float>(R, A.part);
            const int ns = p.n_splits;
            const int item = blockIdx.x;
            if (item < p.n_kv * ns) {
                const int kvh = item / ns, split = item % ns;
                AttnPost post{qkv, qkv + QD, L.wv ? qkv + QD + KD : qkv + QD, L.q_norm, L.k_norm,
                              p.rope_cs + (L.global ? kHD : 0), p.eps,
                              L.global ? 0 : (int)L.slots, L.kq, L.vq, L.ks, L.vs};
                const uint32_t kv_len = p.step[L.global ? 2 : 1];
                attn_split<QPK, true, kPWG>(nullptr, L.kq, L.ks, L.vq, L.vs, kv_len, p.n_kv, ns,
                                            p.attn_scale, part, post, kvh, split, kPAttnOff, pos);
                __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
                __syncthreads();
                if (threadIdx.x == 0) {
                    const unsigned old = __hip_atomic_fetch_add(
                        p.sync + kSyncMergeOff + l * p.n_kv + kvh, 1u, __ATOMIC_RELAXED,
                        __HIP_MEMORY_SCOPE_AGENT);
                    last_s = old + 1 == (unsigned)ns;
                }
                __syncthreads();
                if (last_s)
                    attn_merge<QPK, true>(part, ns, kvh, nullptr, at<BlockLimbs>(R, A.xl_o), o_s);
            }
            SGQ_SYNC()
        }
        // O projection; gate/up starts streaming before the barrier
        {
            gemv_run_any(o_stage(l), ring, 3, 1.f);
            SGQ_SYNC_AFTER_PREFETCH(gu_stage(l), kRStages - 1)
        }
        // post-attention residual + FFN norm limbs
        {
            const float *x_in = at<float>(R, A.x);
            residual_stage(at<float>(R, A.y), L.post_attn_norm, x_in, nullptr, L.ffn_norm,
                           at<float>(R, A.xm), at<BlockLimbs>(R, A.xl_ffn), at<float>(R, A.ss_ffn),
                           H, p.eps);
            SGQ_SYNC()
        }
        // gate/up + GeGLU; down starts streaming before the barrier
        {
            const float r = rms_from_partials(at<float>(R, A.ss_ffn), H / 32, H, p.eps);
            gemv_run_any(gu_stage(l), ring, kRStages - 1, r);
            SGQ_SYNC_AFTER_PREFETCH(down_stage(l), kRStages - 1)
        }
        // limbs of h
        {
            limbs_stage(at<float>(R, A.h), at<BlockLimbs>(R, A.xl_h), F);
            SGQ_SYNC()
        }
        // down; the next QKV (or the head) starts streaming before the barrier
        {
            gemv_run_any(down_stage(l), ring, kRStages - 1, 1.f);
            if (l + 1 < p.n_layers) {
                SGQ_SYNC_AFTER_PREFETCH(qkv_stage(l + 1), kRStages - 1)
            } else {
                SGQ_SYNC_AFTER_PREFETCH(head_stage(), kRStages - 1)
            }
        }
        // post-FFN residual + layer scale + next norm's limbs
        {
            uint8_t *Rn = region(p, l + 1);
            const float *w_next = l + 1 < p.n_layers ? p.layers[l + 1].attn_norm : p.out_norm;
            residual_stage(at<float>(R, A.d), L.post_ffw_norm, at<float>(R, A.xm), L.out_scale,
                           w_next, at<float>(Rn, A.x), at<BlockLimbs>(Rn, A.xl_attn),
                           at<float>(Rn, A.ss_attn), H, p.eps);
            SGQ_SYNC()
        }
    }
    // tied LM head with softcap
    {
        uint8_t *R = region(p, p.n_layers);
        const float r = rms_from_partials(at<float>(R, A.ss_attn), H / 32, H, p.eps);
        gemv_run_any(head_stage(), ring, kRStages - 1, r);
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    }
#undef SGQ_SYNC
#undef SGQ_SYNC_AFTER_PREFETCH
}

}  // namespace

int persist_lds_bytes() { return kPRing; }

int persist_prepare(int qpk) {
    static bool done[3] = {false, false, false};
    if (qpk < 1 || qpk > 2) return fail(SGQ_ERR_VALIDATION, "persistent decode: qpk %d", qpk);
    if (done[qpk]) return SGQ_OK;
    const void *k = qpk == 1 ? (const void *)decode_persistent_kernel<1>
                             : (const void *)decode_persistent_kernel<2>;
    SGQ_HIP(hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, kPRing));
    int per_cu = 0;
    SGQ_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, kPWG, kPRing));
    SGQ_CHECK(per_cu >= 1, "persistent decode: kernel does not fit a CU");
    done[qpk] = true;
    return SGQ_OK;
}

int launch_decode_persistent(hipStream_t st, const PParams &p, int qpk, int grid) {
    if (int rc = persist_prepare(qpk)) return rc;
    PParams args = p;
    void *kargs[] = {&args};
    const void *k = qpk == 1 ? (const void *)decode_persistent_kernel<1>
                             : (const void *)decode_persistent_kernel<2>;
    SGQ_HIP(hipLaunchCooperativeKernel(k, dim3(grid), dim3(kPWG), kargs, kPRing, st));
    return SGQ_OK;
}

}  // namespace sgq
