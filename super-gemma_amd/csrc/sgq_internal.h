// Internal declarations shared by the libsgq translation units.
// gfx950 (CDNA4) only: wave64, MFMA, v_dot4_i32_i8.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "../../include/sgq.h"

namespace sgq {

constexpr int kWave = 64;
struct BlockLimbs;

// Status plumbing: every entry point returns an sgq_status and leaves a
// human-readable message in a thread-local buffer (sgq_last_error()).
int fail(int status, const char *fmt, ...);
int check_hip(hipError_t e, const char *what);
#define SGQ_HIP(expr)                                            \
    do {                                                         \
        hipError_t _e = (expr);                                  \
        if (_e != hipSuccess) return ::sgq::check_hip(_e, #expr); \
    } while (0)
#define SGQ_CHECK(cond, ...)                                          \
    do {                                                              \
        if (!(cond)) return ::sgq::fail(SGQ_ERR_VALIDATION, __VA_ARGS__); \
    } while (0)

// Launch-time device facts, cached per device ordinal.
struct DeviceInfo {
    int cus = 256;
    int xcds = 8;
};
const DeviceInfo &device_info();

hipStream_t ctx_stream(const sgq_ctx *ctx);
void *ctx_workspace(const sgq_ctx *ctx);

// ---- kernel launchers (one per hot-path kernel family) ------------------
// workspace: >= kGemvWorkspace bytes of device memory (x limb table), or
// nullptr to force the register path.
constexpr size_t kGemvWorkspace = 2048 * 96;
// Context workspace layout (device memory, per context):
//   [0, kGemvWorkspace)                GEMV x limb table
//   [kAttnPartOff, kWorkspaceBytes)    attention split partials
constexpr int kAttnMaxKv = 1024;
constexpr size_t kAttnPartOff = 256 * 1024 + 4096;
constexpr size_t kWorkspaceBytes = 16u << 20;
int launch_gemv_q4_0(hipStream_t st, const void *w, const float *x, float *y, uint32_t n,
                     uint32_t k, void *workspace);
// f16 x and y (the reference's gemv_q4_0 binding types): sums in f32 as
// for fp32 x, each output rounded to f16.
int launch_gemv_q4_0(hipStream_t st, const void *w, const uint16_t *x, uint16_t *y, uint32_t n,
                     uint32_t k, void *workspace);
// Up to kGemvMaxTargets Q4_0 matrices with the same K whose rows form one
// concatenated row space (rows [end[j-1], end[j]) belong to matrix j), read
// against one x limb table.  softcap > 0 applies cap*tanh(v/cap) on output.
constexpr int kGemvMaxTargets = 4;
struct GemvTargets {
    const void *w[kGemvMaxTargets];
    float *y[kGemvMaxTargets];
    int end[kGemvMaxTargets];
    int count;
    float softcap;
    // split_out != 0 (single target, K above one slice): each K-slice s
    // writes its partial row sums to y[0] + s*n instead of meeting at a
    // workgroup barrier; the consumer adds the slices in order s = 0..S-1.
    int split_out;
    // half_out != 0: the targets y[j] hold f16 rows (uint16_t bits; rows
    // are rounded to nearest even); not with split_out
    int half_out;
};
// Number of K-slices the streamed GEMV uses for K (1, 2 or 4); 0 if K is
// outside the streamed geometry.
int gemv_slices(uint32_t k);
// Sets the streamed kernels' launch attributes (call before graph capture).
int gemv_prepare();
int launch_quant_limbs(hipStream_t st, const float *x, void *xl, uint32_t k);
int launch_quant_limbs(hipStream_t st, const uint16_t *x, void *xl, uint32_t k);
// Q6_K logits GEMV (gemv_q6_k.hip): rows at a 16-byte-multiple stride.
int launch_gemv_q6_k(hipStream_t st, const void *w, size_t row_stride, const float *x, float *y,
                     uint32_t n, uint32_t k, float softcap);
// f16 x (gemv_q6_k_logits.wgsl:19); the fp32 form rounds x to f16 itself.
int launch_gemv_q6_k(hipStream_t st, const void *w, size_t row_stride, const uint16_t *x,
                     float *y, uint32_t n, uint32_t k, float softcap);
// Fused forms of the streamed GEMV (single K-slice for the prologues).
// Prologue (what the GEMV's x limbs are computed from, inside the launch):
//   kProTable  the limb table xl (written by an earlier kernel), each wave
//              loading its lanes' entries into registers;
//   kProTableLds  the same table copied into LDS once per workgroup by
//              DMA (one K-slice, or up to four with the residual epilogue
//              while the table fits two workgroups' LDS);
//   kProSliceLds  K-sliced rows with split output: workgroup b takes K-slice
//              b % S of its rows and copies only that slice of the table
//              into LDS; each K-slice partial goes to y[slice·n + row];
//   kProNorm   f = rb·s·(A + ra·B) with ra = 1/sqrt(P1/K + eps),
//              rb = 1/sqrt(s²(P4 + 2·ra·P2 + ra²·P3)/K + eps) from the np
//              partial sums (P1..P4) an kEpiResid launch left in part, and
//              x_out = s·(x_in + ra·u) (each workgroup writes a slice);
//              s = *scale (1 when null).  That is the residual update
//              x_out = (x_in + rmsnorm(o)∘w_post)·s followed by
//              rmsnorm(x_out)∘w_next, with A = x_in∘w_next, u = o∘w_post,
//              B = u∘w_next;
//   kProEmbed  x0 = dequant(embd[step[4]])·embed_scale, f = rmsnorm(x0)∘w,
//              x_out = x0 (sliced);
//   kProX      f = x_raw (fp32, or f16 when x_half), split into limbs by
//              every workgroup.
// Epilogue (what is done with the output rows o):
//   kEpiRows   stored to the targets (softcap, split_out as GemvTargets);
//   kEpiResid  single target: per row u = o·w_post, A = x_res·w_next,
//              B = u·w_next into u_out/A_out/B_out, and the workgroup's
//              (Σo², Σx_res·u, Σu², Σx_res²) into part_out[workgroup];
//   kEpiGeglu  targets gate (w[0]) and up (w[1]), n = units: workgroup b
//              computes units [32b, 32b+32) and writes block b of the limbs
//              of gelu_tanh(gate)·up into hl.
enum { kProTable = 0, kProNorm = 1, kProEmbed = 2, kProX = 3, kProTableLds = 4, kProSliceLds = 5 };
enum { kEpiRows = 0, kEpiResid = 1, kEpiGeglu = 2 };
constexpr int kGemvMaxPartials = 512;
struct GemvFuse {
    const float4 *part;
    int np;
    const float *A, *B, *u, *x_in, *scale;
    float *x_out;
    const uint8_t *embd;
    const uint32_t *step;
    float embed_scale;
    const float *w;
    float eps;
    const float *x_res, *w_post, *w_next;
    float *u_out, *A_out, *B_out;
    float4 *part_out;
    struct BlockLimbs *hl;
    const void *x_raw;  // kProX
    int x_half;
};
// Workgroups a fused launch uses (= the np its kEpiResid partials need).
int gemv_fused_grid(uint32_t n, uint32_t k, int epi, int pro = kProTable);
int launch_gemv_fused(hipStream_t st, const GemvTargets &tg, const void *xl, uint32_t k, int pro,
                      int epi, const GemvFuse &fz);

int launch_gemv_limbs(hipStream_t st, const GemvTargets &tg, const void *xl, uint32_t k);
int launch_quant_q8_0(hipStream_t st, const float *x, uint16_t *scales, int8_t *quants,
                      uint64_t n_elems);
int launch_dequant_q8_0(hipStream_t st, const uint16_t *scales, const int8_t *quants, float *out,
                        uint64_t n_elems);
int launch_kv_append_q8(hipStream_t st, const float *src, uint16_t *scales, int8_t *quants,
                        const uint32_t *step, uint32_t n_tokens, uint32_t row_len,
                        uint32_t ring);
// V quantized in 32-KEY blocks per column (kv_append_global_v_q8.wgsl):
// rows [n_tokens × row_len] appended at pos (step[0] when step is given;
// a multiple of 32), scales [block × row_len] f16.
int launch_kv_append_v_q8(hipStream_t st, const float *src, uint16_t *scales, int8_t *quants,
                          const uint32_t *step, uint32_t pos, uint32_t n_tokens, uint32_t row_len);
// The Q8_0 operators over f16 activations (uint16_t bits): an f16 source
// widens exactly, so quants and scales are those of its fp32 value; the
// dequantized output rounds to f16.
int launch_quant_q8_0(hipStream_t st, const uint16_t *x, uint16_t *scales, int8_t *quants,
                      uint64_t n_elems);
int launch_dequant_q8_0(hipStream_t st, const uint16_t *scales, const int8_t *quants,
                        uint16_t *out, uint64_t n_elems);
int launch_kv_append_q8(hipStream_t st, const uint16_t *src, uint16_t *scales, int8_t *quants,
                        const uint32_t *step, uint32_t n_tokens, uint32_t row_len, uint32_t ring);
int launch_kv_append_v_q8(hipStream_t st, const uint16_t *src, uint16_t *scales, int8_t *quants,
                          const uint32_t *step, uint32_t pos, uint32_t n_tokens, uint32_t row_len);
// Prefill attention with int8 PV (attn_prefill_global_flash_sp_ipv.wgsl):
// causal over a linear Q8_0 cache with key-blocked V scales vs_kb
// [ceil(keys/32) × n_kv × 128]; q0 from step[3] when step is given.
int launch_attn_prefill_ipv(hipStream_t st, const float *q, const int8_t *kq, const uint16_t *ks,
                            const int8_t *vq, const uint16_t *vs_kb, float *out, int n_tok, int q0,
                            int n_q, int n_kv, int head_dim, float scale, const uint32_t *step);
int launch_gemm_q4_0_q8(hipStream_t st, const void *w, const int8_t *xq, const uint16_t *xs,
                        float *y, uint32_t m, uint32_t n, uint32_t k, uint32_t split_k,
                        float *partials);
// f16 output (the reference's y binding), no split-K.
int launch_gemm_q4_0_q8(hipStream_t st, const void *w, const int8_t *xq, const uint16_t *xs,
                        uint16_t *y, uint32_t m, uint32_t n, uint32_t k);
int launch_attn_decode_q8(hipStream_t st, const float *q, const int8_t *kq, const uint16_t *ks,
                          const int8_t *vq, const uint16_t *vs, const uint32_t *step,
                          int step_word, uint32_t kv_len, int n_q, int n_kv, int head_dim,
                          int n_splits, float scale, float *out, void *workspace,
                          size_t workspace_bytes, void *limbs_out = nullptr);
// The split kernel alone, reading kv_len from step[step_word] and writing
// every split's partial (acc[128], m, l) per query head to part
// [n_q × n_splits × 130] (attn_decode_global_q8k.wgsl's part layout); then
// the merge of those partials in split order into out [n_q × 128]
// (attn_reduce.wgsl:24-57).  head_dim 128, 1 or 2 query heads per kv head.
int launch_attn_decode_parts(hipStream_t st, const float *q, const int8_t *kq,
                             const uint16_t *ks, const int8_t *vq, const uint16_t *vs,
                             const uint32_t *step, int step_word, int n_q, int n_kv, int n_splits,
                             float scale, float *part);
// Prefill attention at head_dim 256/512 over the reference's page formats
// (prefill_attn.hip, PfFmt): fmt 1 f16 q with Q8_0 K/V (k_scales/v_scales),
// 2 f16 q/K/V, 3 int8 q (q_scales) with Q8_0 K and f16 V, 4 the same with int8 V
// under key-blocked v_scales (causal, linear cache) and int8 P; f16 out
// [n_tok × n_q × head_dim]; q0 = step[3]; window 0 = causal; ring > 0:
// keys before q0 from the ring (slot = pos mod ring), from q0 on from the
// chunk's pages ck/cv (rows = pos - q0; Q8_0 formats: cks/cvs scales).
int launch_attn_prefill_pages(hipStream_t st, int fmt, const void *q, const uint16_t *q_scales,
                              const void *k, const uint16_t *k_scales, const void *v,
                              const uint16_t *v_scales, int ring, const void *ck, const void *cv,
                              const uint16_t *cks, const uint16_t *cvs, void *out, int n_tok,
                              const uint32_t *step, int n_q, int n_kv, int head_dim, int window,
                              float scale);
// Decode attention over f16 pages (or Q8_0 K with f16 V) for the released
// checkpoint's names (attn_pages.hip): q f16 [n_q × head_dim], pages
// [slot × n_kv × head_dim], k_scales non-null selects Q8_0 K (f16 scale per
// 32 dims); kv_len = step[step_word]; split s covers the s-th chunk of
// ceil(kv_len / n_splits) slots; partials [n_q × n_splits × (head_dim + 2)].
// Built: head_dim 256 with 2 q heads per kv head (f16 K), 512 with 8 (f16
// or Q8_0 K).
int launch_attn_decode_pages(hipStream_t st, const uint16_t *q, const void *k,
                             const uint16_t *k_scales, const uint16_t *v, float *part,
                             const uint32_t *step, int step_word, int head_dim, int n_q, int n_kv,
                             int n_splits, float scale);
// Their merge in split order into f16 rows [n_q × head_dim] (256 / 512).
int launch_attn_reduce_pages(hipStream_t st, const float *part, int n_q, int head_dim,
                             int n_splits, uint16_t *out);
// f16 rows [n_tok × row] into pages at slot step[0] + t (mod ring if ring > 0).
int launch_kv_append_f16(hipStream_t st, const uint16_t *src, uint16_t *dst,
                         const uint32_t *step, uint32_t n_tok, uint32_t row, uint32_t ring);
int launch_attn_reduce(hipStream_t st, const float *part, int n_q, int n_kv, int n_splits,
                       float *out);
// Decode attention at head_dim 128/256/512 and 1/2/4/8 query heads per kv
// head (attn_generic.hip).  q [n_q × head_dim] ready, or with post the
// post-projection fused in (GenericPost).  Attention: splits of 64 slots
// (attn_generic_splits(slots) of them cover a cache of `slots`), kv_len =
// step[step_word], partials in part [n_q × n_splits × (head_dim+2)], merged
// in split order into out [n_q × head_dim] and/or the x limbs xl.
int attn_generic_splits(uint32_t slots);
// The q/k/v post-projection fused into the attention (q/k norms with
// weights q_norm / k_norm, weightless v norm, NEOX RoPE of q and k with cs
// [head_dim/2 pairs], the new K/V rows quantized (Q8_0) into slot step[0],
// mod ring when ring > 0): q_raw [n_q × head_dim], k_raw / v_src
// [n_kv × head_dim], and writable views of the cache pages.
struct GenericPost {
    const float *q_raw, *k_raw, *v_src, *q_norm, *k_norm;
    const float2 *cs;
    float eps;
    uint32_t ring;
    int8_t *kq_w, *vq_w;
    uint16_t *ks_w, *vs_w;
};
int launch_attn_decode_generic(hipStream_t st, const float *q, const int8_t *kq,
                               const uint16_t *ks, const int8_t *vq, const uint16_t *vs,
                               const uint32_t *step, int step_word, int n_q, int n_kv,
                               int head_dim, int n_splits, float scale, float *part, float *out,
                               void *xl, const GenericPost *post = nullptr);
// Sets the attention kernels' launch attributes (call before graph capture).
int attn_prepare();
// Decode attention with the step's q/k/v post-projection fused in, then the
// split merge as a second launch: q, k and v_src are the raw projections (v_src may alias k_raw), rope_cs the
// (cos, sin) table of the current position; appends the new K/V rows at the
// current slot (pos % ring, or pos when ring == 0).  head_dim 128.
int launch_attn_decode_fused(hipStream_t st, const float *q_raw, const float *k_raw,
                             const float *v_src, const float *wq_norm, const float *wk_norm,
                             const float *rope_cs, float eps, const uint32_t *step, int step_word,
                             uint32_t ring, int8_t *kq, uint16_t *ks, int8_t *vq, uint16_t *vs,
                             int n_q, int n_kv, int n_splits, float scale, float *out,
                             void *workspace, size_t workspace_bytes, void *limbs_out);
// Keys before q0 come from the cache (ring: slot = pos % ring), keys from q0
// on from the chunk's pages ckq.. (row = pos - q0) when given, else the cache.
// With step non-null, q0 is read on the device from step[3] (the host value
// is ignored), so a recorded graph replays with a new chunk position.
int launch_attn_prefill_q8(hipStream_t st, const float *q, const int8_t *kq, const uint16_t *ks,
                           const int8_t *vq, const uint16_t *vs, float *out, int n_tok, int q0,
                           int n_q, int n_kv, int head_dim, int window, float scale, int ring = 0,
                           const int8_t *ckq = nullptr, const uint16_t *cks = nullptr,
                           const int8_t *cvq = nullptr, const uint16_t *cvs = nullptr,
                           const uint32_t *step = nullptr);
int launch_rmsnorm(hipStream_t st, const float *x, const float *w, float *y, uint32_t rows,
                   uint32_t row_len, int plus_one, float eps);
int launch_rope(hipStream_t st, float *xs, const float *cos_sin, uint64_t rows, uint32_t head_dim,
                uint32_t rot_dims, uint32_t n_heads);
int launch_geglu(hipStream_t st, const float *g, const float *u, float *y, uint64_t n);
int launch_add_scaled(hipStream_t st, const float *a, const float *b, float *y, uint64_t n,
                      float s);
// The same operators over f16 activations (uint16_t bits), the reference's
// storage type: rmsnorm/geglu/add_scaled read f16, compute in f32, round
// the result to f16; rope rotates f16 rows in place.
int launch_rmsnorm(hipStream_t st, const uint16_t *x, const float *w, uint16_t *y, uint32_t rows,
                   uint32_t row_len, int plus_one, float eps);
int launch_rope(hipStream_t st, uint16_t *xs, const float *cos_sin, uint64_t rows,
                uint32_t head_dim, uint32_t rot_dims, uint32_t n_heads);
int launch_geglu(hipStream_t st, const uint16_t *g, const uint16_t *u, uint16_t *y, uint64_t n);
int launch_add_scaled(hipStream_t st, const uint16_t *a, const uint16_t *b, uint16_t *y,
                      uint64_t n, float s);
int launch_fill_q4_0(hipStream_t st, void *w, uint64_t n_blocks, uint64_t seed, float sigma);
int launch_fill_normal(hipStream_t st, float *x, uint64_t n, uint64_t seed, float mean,
                       float sigma);
// Random Q6_K rows (k/256 blocks of 210 B) at a byte stride, padding zeroed.
int launch_fill_q6k(hipStream_t st, void *w, uint64_t n_rows, uint32_t k, uint64_t row_stride,
                    uint64_t seed);

}  // namespace sgq

// ---- small device helpers -------------------------------------------------
namespace sgq {

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float v) {
    // v_cvt_f16_f32 rounds to nearest even in the default FP mode.
    return __builtin_bit_cast(uint16_t, (_Float16)v);
}

// Activation element access for kernels built for both activation types:
// fp32, or f16 held as its bits (the reference's activation storage).  A
// load widens exactly; an f16 store rounds to nearest even.
__device__ __forceinline__ float act_ld(const float *p, size_t i) { return p[i]; }
__device__ __forceinline__ float act_ld(const uint16_t *p, size_t i) { return f16_bits_to_f32(p[i]); }
__device__ __forceinline__ void act_st(float *p, size_t i, float v) { p[i] = v; }
__device__ __forceinline__ void act_st(uint16_t *p, size_t i, float v) { p[i] = f32_to_f16_bits(v); }
// Four consecutive activations starting at element 4j.
__device__ __forceinline__ float4 act_ld4(const float *p, size_t j) {
    return reinterpret_cast<const float4 *>(p)[j];
}
__device__ __forceinline__ float4 act_ld4(const uint16_t *p, size_t j) {
    const uint2 w = reinterpret_cast<const uint2 *>(p)[j];
    return make_float4(f16_bits_to_f32(w.x & 0xffffu), f16_bits_to_f32(w.x >> 16),
                       f16_bits_to_f32(w.y & 0xffffu), f16_bits_to_f32(w.y >> 16));
}

}  // namespace sgq
