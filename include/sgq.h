/*
 * sgq.h — C ABI of libsgq, the MI355X (gfx950) quantized compute core that
 * replaces super-gemma's sg-gpu kernel-dispatch surface.
 *
 * Two layers, both plain C (no torch or HIP types in any signature):
 *
 *  1. The dispatch surface, mirroring sg-gpu's public API
 *     (crates/sg-gpu/src/lib.rs:20-44): a context, device buffers, kernel
 *     lookup by variant NAME, a dispatch of (kernel, bindings, push constants,
 *     groups), re-submittable recorded graphs and a per-step state buffer.
 *     Variant names, binding order, push-constant layout and group counts are
 *     the reference's (crates/sg-gpu/build.rs VARIANTS), so a forward graph
 *     that records `load_kernel(name)` + `dispatch(...)` drives this library
 *     unchanged.  Under the reference's names, activation buffers hold f16
 *     as the reference's shaders bind them (gemv_q4_0.wgsl:18-19,
 *     rmsnorm.wgsl:14-16, rope.wgsl:26, geglu.wgsl:7-9, add_scaled.wgsl:12-14,
 *     gemm_q4_0_i8.wgsl:63, kv_quant_q8.wgsl:24, kv_dequant_q8.wgsl:11,
 *     kv_append_global_q8.wgsl:19, kv_append_global_v_q8.wgsl:20,
 *     gemv_q6_k_logits.wgsl:19); the same kernel over fp32 activations is
 *     NAME_f32 (e.g. gemv_q4_0_k5376_f32, rmsnorm_5376_f32, geglu_f32,
 *     gemm_q4_0_i8_bb_pfd4_f32).  Families with no reference counterpart
 *     (the head_dim-128 attention and RoPE forms, kv_append_sliding_q8, the
 *     split-K MMQ) take fp32 and no suffix.  Q4_0 weights and Q8_0 pages are
 *     byte-identical formats.
 *
 *  2. Typed entry points (sgq_gemv_q4_0, sgq_gemm_q4_0_q8, ...) that compute
 *     their own launch geometry; the name dispatch routes to the same code.
 *
 * Pointers passed as buffers are device pointers (from sgq_buf_alloc or any
 * HIP allocation on the context's device).  All work is enqueued on the
 * context's stream (sgq_ctx_set_stream) in call order, which gives the
 * compute→compute ordering the reference gets from its per-dispatch barrier.
 * A context is used by one host thread at a time.
 */
#ifndef SGQ_H
#define SGQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes mirror sg_gpu::GpuError (crates/sg-gpu/src/lib.rs:31-44);
 * SGQ_ERR_HIP takes the place of the Vulkan error. */
typedef enum {
    SGQ_OK = 0,
    SGQ_ERR_LIBRARY = 1,        /* GpuError::Library */
    SGQ_ERR_HIP = 2,            /* GpuError::Vk */
    SGQ_ERR_NO_DEVICE = 3,      /* GpuError::NoDevice: callers skip, not fail */
    SGQ_ERR_UNKNOWN_KERNEL = 4, /* GpuError::UnknownKernel */
    SGQ_ERR_PIPELINE = 5,       /* GpuError::Pipeline */
    SGQ_ERR_VALIDATION = 6      /* GpuError::Validation: bad shapes/bindings */
} sgq_status;

typedef struct sgq_ctx sgq_ctx;
typedef struct sgq_kernel sgq_kernel;
typedef struct sgq_graph sgq_graph;

/* Message for the last failing call on this thread ("" if none). */
const char *sgq_last_error(void);
/* Library version string. */
const char *sgq_version(void);

/* ---- context: GpuContext::new (crates/sg-gpu/src/context.rs:103-236) ---- */
int sgq_ctx_create(int device, sgq_ctx **out);
int sgq_ctx_destroy(sgq_ctx *ctx);
/* Use an existing hipStream_t (passed as void*); NULL = the null stream. */
int sgq_ctx_set_stream(sgq_ctx *ctx, void *hip_stream);
/* submit_blocking's wait half (crates/sg-gpu/src/graph.rs:640). */
int sgq_sync(sgq_ctx *ctx);

/* ---- buffers: crates/sg-gpu/src/buffer.rs:233-300 ------------------------ */
int sgq_buf_alloc(sgq_ctx *ctx, uint64_t bytes, void **dev_ptr);
int sgq_buf_free(sgq_ctx *ctx, void *dev_ptr);
int sgq_buf_upload(sgq_ctx *ctx, void *dst_dev, const void *src_host, uint64_t bytes);
int sgq_buf_download(sgq_ctx *ctx, void *dst_host, const void *src_dev, uint64_t bytes);
/* Zero-fill on the context stream.  Returns SGQ_ERR_VALIDATION while a graph
   capture (sgq_graph_begin) is open: no memset is ever recorded into a graph. */
int sgq_buf_fill_zero(sgq_ctx *ctx, void *dev_ptr, uint64_t bytes);

/* ---- kernel registry: KernelBlob (crates/sg-gpu/src/kernel.rs:18-34) and
 *      GpuContext::load_kernel (kernel.rs:79-163) ------------------------- */
typedef struct {
    uint32_t workgroup[3]; /* the reference's workgroup size (for its group math) */
    uint32_t bindings;     /* storage-buffer bindings 0..bindings-1 */
    uint32_t push_bytes;   /* push-constant bytes (0 = none) */
    uint32_t subgroup_size;
} sgq_kernel_info;

/* Attention and KV-append variants (the reference's record_layer dispatches,
 * crates/sg-model/src/graph.rs:560-656, at this build's geometry: Q8_0 K and
 * V pages, head_dim 128, 32 query / 16 kv heads, window and ring 1024):
 *   kv_append_global_q8 / kv_append_sliding_q8
 *       0 src [n_tok × ROW] (f16 for kv_append_global_q8, fp32 for its
 *       _f32 form and for kv_append_sliding_q8; whole rows), 1 scales,
 *       2 quants, 3 step; slot = step[0] + t (global) or (step[0] + t) % 1024
 *       (sliding); ROW = groups.y·32 when groups.y > 1, else 2048
 *   attn_decode_global_q8_hd128 / attn_decode_sliding_q8_hd128
 *       0 q, 1 k_quants, 2 k_scales, 3 v_quants, 4 v_scales, 5 part, 6 step;
 *       push {n_splits: u32, scale: f32}; groups [16, n_splits, 1];
 *       kv_len = step[2] / step[1]  (attn_decode_global_q8k.wgsl:18-25)
 *   attn_reduce_d128
 *       0 part [32 × n_splits × 130], 1 out [32 × 128]; push n_splits;
 *       groups [32, 1, 1]  (attn_reduce.wgsl:11-14)
 *   attn_prefill_global_flash_q8_hd128
 *       0 q fp32, 1..4 cache K/V pages, 5 out, 6 step; push f32 scale;
 *       groups [32, ceil(M/16), 1]; q0 = step[3]
 *       (attn_prefill_global_flash_sp_iq.wgsl:24-35)
 *   attn_prefill_sliding_ring_q8_hd128
 *       0 q, 1..4 ring K/V pages, 5..8 chunk K/V pages, 9 out, 10 step;
 *       push f32 scale; groups [16, M, 1]  (attn_prefill_sliding_ring.wgsl:28-40)
 *   kv_append_global_v_q8  (kv_append_global_v_q8.wgsl:19-25)
 *       0 src f16 (fp32 for _f32) [n_tok × ROW], whole rows, 1 key-blocked
 *       scales [ceil(n_tok/32) × ROW], 2 quants [n_tok × ROW], 3 step
 *       (pos = step[0], a multiple of 32); ROW = groups.y·32 when
 *       groups.y > 1, else 2048
 *   attn_prefill_global_flash_ipv_hd128  (attn_prefill_global_flash_sp_ipv.wgsl:24-35)
 *       0 q fp32, 1 k_quants, 2 k_scales, 3 v_quants, 4 key-blocked v_scales,
 *       5 out, 6 step; push f32 scale; groups [32, ceil(M/16), 1]
 * M (prefill) is the out binding's range / (32·128·4).
 * The real checkpoint's decode side over f16 pages (crates/sg-gpu/build.rs:
 * 255-394; record_layer, crates/sg-model/src/graph.rs:572-650), 32 q heads:
 *   attn_decode_sliding   head_dim 256, 16 kv heads; 0 q f16 [32 × 256],
 *       1 K ring f16 [slot × 16 × 256], 2 V ring f16, 3 part fp32
 *       [32 × n_splits × 258], 4 step; kv_len = step[1]
 *   attn_decode_global    head_dim 512, 4 kv heads, the same bindings;
 *       kv_len = step[2]
 *   attn_decode_global_q8k  0 q, 1 k_quants i8 [slot × 4 × 512], 2 k_scales
 *       f16 [slot × 4 × 16], 3 V f16, 4 part, 5 step
 *       (all three: push {n_splits: u32, scale: f32}; groups [n_kv, n_splits,
 *       1]; split s covers the s-th ceil(kv_len/n_splits) slots;
 *       attn_decode_sliding.wgsl:16-50)
 *   attn_reduce_d256 / attn_reduce_d512  0 part, 1 out f16 [32 × HD]; push
 *       n_splits; groups [32, 1, 1]  (attn_reduce.wgsl:14-30)
 *   kv_append_sliding / kv_append_global  0 src f16 [n_tok × ROW], 1 dst f16
 *       [slot × ROW], 2 step; ROW 4096 into the 1024-slot ring (slot =
 *       (step[0] + t) mod 1024) / 2048 linear; groups cover n_tok·ROW
 *       elements at 256 a group  (kv_append.wgsl:15-35)
 * Its prefill (crates/sg-gpu/build.rs:395-438, :2206-2292; record_prefill_
 * layer, graph.rs:1176-1225); push {scale: f32}; q0 = step[3]; out f16
 * [M × 32 × HD]; M = groups.y (grid [n_kv, M, 1]) or 16·groups.y (grid
 * [32, M/16, 1]):
 *   attn_prefill_sliding       hd 256, window 1024, [16, M]; 0 q f16, 1 K f16
 *       [pos × 16 × 256], 2 V f16, 3 out, 4 step
 *   attn_prefill_sliding_ring  hd 256, window 1024, [16, M]; 0 q, 1 K ring,
 *       2 V ring (1024 slots, before this chunk's append), 3 chunk K, 4 chunk
 *       V [M × 16 × 256], 5 out, 6 step
 *   attn_prefill_global        hd 512 causal, [4, M]; bindings as _sliding
 *   attn_prefill_global_flash / _flash_sp   hd 512 causal, [32, M/16]; the same
 *   attn_prefill_global_flash_sp_q8  [32, M/16]; 0 q f16, 1 k_quants, 2 k_scales,
 *       3 v_quants, 4 v_scales, 5 out, 6 step (K/V dequantized to f16)
 *   attn_prefill_global_flash_sp_iq  [32, M/16]; 0 q_i8, 1 q_scales f16
 *       [M × 32 × 16], 2 k_quants, 3 k_scales, 4 V f16, 5 out, 6 step (score
 *       = sum over 32-dim blocks of q_scale·k_scale·integer dot)
 *   attn_prefill_global_flash_sp_ipv / _ipv_bcast  [32, M/16]; 0 q_i8,
 *       1 q_scales, 2 k_quants, 3 k_scales, 4 v_quants, 5 key-blocked v_scales
 *       f16 [pos/32 × 4 × 512], 6 out, 7 step (P quantized per query and
 *       32-key block; attn_prefill_global_flash_sp_ipv.wgsl:134-210)
 * Any other name returns SGQ_ERR_UNKNOWN_KERNEL. */
int sgq_kernel_lookup(sgq_ctx *ctx, const char *name, const sgq_kernel **out,
                      sgq_kernel_info *info);
/* Number of registered variant names / the i-th one (for enumeration). */
uint32_t sgq_kernel_count(void);
const char *sgq_kernel_name(uint32_t i);

/* BufferBinding{binding, buffer, offset, range} (graph.rs:199-225).
 * range == 0 means "to the end of the allocation is unknown": callers pass the
 * byte length actually bound, as Vulkan's arrayLength() semantics need it. */
typedef struct {
    uint32_t binding;
    uint32_t _pad;
    void *ptr;
    uint64_t offset;
    uint64_t range;
} sgq_binding;

/* GraphRecorder::dispatch (crates/sg-gpu/src/graph.rs:225-324): groups are the
 * reference's group counts for this variant. */
int sgq_dispatch(sgq_ctx *ctx, const sgq_kernel *kernel, const sgq_binding *bindings,
                 uint32_t n_bindings, const void *push, uint32_t push_bytes,
                 const uint32_t groups[3]);

/* ---- recorded graphs: CommandGraph / GraphRecorder / submit (graph.rs:
 *      523-660), backed by hipGraph capture of the context's stream ------- */
int sgq_graph_begin(sgq_ctx *ctx);
int sgq_graph_end(sgq_ctx *ctx, sgq_graph **out);
int sgq_graph_submit(sgq_ctx *ctx, sgq_graph *graph);
int sgq_graph_destroy(sgq_graph *graph);

/* StepState::write_to (crates/sg-gpu/src/graph.rs:33-61): the 4-word step
 * buffer [pos, kv_len_sliding, kv_len_global, q0], written on the stream. */
int sgq_step_write(sgq_ctx *ctx, void *step_dev, uint32_t pos, uint32_t kv_len_sliding,
                   uint32_t kv_len_global, uint32_t q0);

/* ---- timers: GpuTimer (graph.rs:404-460) over hipEvents ----------------- */
int sgq_timer_start(sgq_ctx *ctx);
/* Milliseconds since sgq_timer_start, after waiting for the stream. */
int sgq_timer_stop(sgq_ctx *ctx, float *ms);

/* ---- typed entry points -------------------------------------------------- */

/* Decode GEMV y[n] = W[n×k]·x[k]; W is Q4_0 row-major (k/32 blocks of 18 B
 * per row), x and y fp32.  Replaces gemv_q4_0_k{K} / gemv_q4_0_generic
 * (crates/sg-gpu/shaders/gemv_q4_0.wgsl:52-112).  k % 64 == 0, k <= 65536.
 * x enters the integer dot as four signed 4-bit limbs per value (error
 * <= 1.7e-5 of its 32-block's max |x|, below an f16 rounding of x). */
int sgq_gemv_q4_0(sgq_ctx *ctx, const void *w, const float *x, float *y, uint32_t n,
                  uint32_t k);

/* The decode GEMV in its two halves, as the decode graph runs them: x is
 * split once into its limb table (sgq_x_limbs: k/32 entries of
 * SGQ_X_LIMBS_BYTES_PER_BLOCK bytes, 16-byte aligned), then one launch
 * streams up to 4 Q4_0 matrices that share x (the reference's per-matrix
 * gemv_q4_0 dispatches of one x, e.g. Q/K/V or gate/up, graph.rs:478-560),
 * writing rows[j] outputs to y[j]; softcap > 0 applies cap·tanh(v/cap) to
 * every output (the LM head, graph.rs:740-756).  k % 256 == 0,
 * 256 <= k <= 65536 (up to 4 K-slices of <= 170 blocks); weights 16-byte
 * aligned.  No counterpart for the limb table in the reference: it is this
 * GEMV's activation format (four signed 4-bit limbs per value, see
 * sgq_gemv_q4_0 for the error bound). */
#define SGQ_X_LIMBS_BYTES_PER_BLOCK 80
int sgq_x_limbs(sgq_ctx *ctx, const float *x, void *x_limbs, uint32_t k);
int sgq_gemv_q4_0_limbs(sgq_ctx *ctx, uint32_t n_targets, const void *const *w, float *const *y,
                        const uint32_t *rows, const void *x_limbs, uint32_t k, float softcap);

/* Allocation-free form of sgq_gemv_q4_0: no counterpart in the reference.
 * For callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  No context:
 * work goes on `hip_stream` (NULL = the null stream), which must belong to the
 * current device.  The x limb table lives in a library-owned device array of
 * 192 KiB per device (kept until the process ends), so k <= 65536; larger k
 * returns SGQ_ERR_VALIDATION.  Every call on one device shares that array.
 * Calls on one stream are ordered; a call on a different stream while the
 * previous eager call (on another stream) has not finished returns
 * SGQ_ERR_VALIDATION instead of racing (a library-owned event, created with
 * the array's address on the device's first call, marks the end of each
 * eager call).  Calls recorded under graph capture are not tracked: graph
 * replays that overlap other calls on the device race, as do calls from two
 * host threads that enqueue on two streams at the same moment. */
int sgq_gemv_q4_0_noalloc(void *hip_stream, const void *w, const float *x, float *y, uint32_t n,
                          uint32_t k);

/* Q6_K LM head: y[n] = softcap·tanh((E[n×k]·x[k]) / softcap) (softcap <= 0:
 * the raw dot).  Replaces gemv_q6_k_logits
 * (crates/sg-gpu/shaders/gemv_q6_k_logits.wgsl:41-104; registry entry
 * crates/sg-gpu/build.rs:322-327).  E holds rows of k/256 GGUF Q6_K
 * super-blocks (210 B each, crates/sg-gguf/src/q6_k.rs:25-62) at a byte
 * stride of row_stride (a multiple of 16; the reference pads 4410 -> 4416
 * at k = 5376); x is fp32 and is rounded to f16, the reference's activation
 * type; y fp32.  k % 256 == 0, k <= 6144; E 16-byte aligned. */
int sgq_gemv_q6_k(sgq_ctx *ctx, const void *w, size_t row_stride, const float *x, float *y,
                  uint32_t n, uint32_t k, float softcap);

/* Q8_0 quantization of n fp32 values (n % 32 == 0) into f16 scales [n/32] and
 * int8 quants [n]: kv_quant_q8 (crates/sg-gpu/shaders/kv_quant_q8.wgsl:30-57),
 * d = amax*(1/127), q = round_ties_even(x/d) with an IEEE reciprocal. */
int sgq_quant_q8_0(sgq_ctx *ctx, const float *x, uint16_t *scales, int8_t *quants,
                   uint64_t n);

/* Q8_0 → fp32 (x = f32(d)*q): kv_dequant_q8 with fp32 output. */
int sgq_dequant_q8_0(sgq_ctx *ctx, const uint16_t *scales, const int8_t *quants, float *out,
                     uint64_t n);

/* Prefill int8 MMQ Y[m×n] = Xq[m×k]·W[n×k]^T with per-32-block rescale
 * (d_a[m,b]*d_w[n,b]) in fp32: gemm_q4_0_i8_* (crates/sg-gpu/shaders/
 * gemm_q4_0_i8.wgsl:153-393, gemm_q4_0_i8_bb_pfd.wgsl).  split_k in
 * {1,2,4,8}: for split_k > 1, `partials` must hold split_k*m*n floats and the
 * slices are summed in fixed order s = 0..split_k-1.  With split_k == 1,
 * `partials` is optional (NULL or at least m*n floats): when given, tiles
 * past the last whole round of resident workgroups are split over K into
 * 2-4 parts summed in part order (fp32 output, m and n multiples of 128).
 * k % 32 == 0. */
int sgq_gemm_q4_0_q8(sgq_ctx *ctx, const void *w, const int8_t *xq, const uint16_t *xs,
                     float *y, uint32_t m, uint32_t n, uint32_t k, uint32_t split_k,
                     float *partials);

/* Split-K decode attention over a Q8_0 KV cache: attn_decode_global_q8k /
 * attn_decode_sliding + attn_reduce (crates/sg-gpu/shaders/
 * attn_decode_global_q8k.wgsl:41-112, attn_reduce.wgsl:24-57), with V in
 * Q8_0 as well.  q [n_q_heads × head_dim] fp32; cache quants
 * [slot × n_kv_heads × head_dim] int8 and scales [slot × n_kv_heads ×
 * head_dim/32] f16 for K and V; slots 0..kv_len-1 are attended in physical
 * order (a linear cache or a full/partial ring); out [n_q_heads × head_dim].
 * Query head h reads kv head h / (n_q_heads / n_kv_heads).  The n_splits
 * chunks are merged in split order inside the same launch.  head_dim 128. */
int sgq_attn_decode_q8(sgq_ctx *ctx, const float *q, const int8_t *k_quants,
                       const uint16_t *k_scales, const int8_t *v_quants, const uint16_t *v_scales,
                       uint32_t kv_len, uint32_t n_q_heads, uint32_t n_kv_heads,
                       uint32_t head_dim, uint32_t n_splits, float scale, float *out);

/* Prefill flash attention over a Q8_0 KV cache (attn_prefill_global_flash_*
 * and attn_prefill_sliding_ring, crates/sg-gpu/shaders/
 * attn_prefill_global_flash_sp_q8.wgsl:65-183): q [n_tokens × n_q_heads ×
 * head_dim] fp32 for positions q0..q0+n_tokens-1; the cache is linear
 * (slot = position) and must hold positions 0..q0+n_tokens-1 (the chunk's
 * own K/V included).  Query at position p attends keys k <= p, and with
 * window > 0 only k > p - window.  K/V are dequantized to f16 and P is
 * rounded to f16 as in the reference; accumulation fp32.  head_dim 128, or
 * 256 / 512 (the released checkpoint's sliding and global layers);
 * out [n_tokens × n_q_heads × head_dim] fp32. */
int sgq_attn_prefill_q8(sgq_ctx *ctx, const float *q, const int8_t *k_quants,
                        const uint16_t *k_scales, const int8_t *v_quants, const uint16_t *v_scales,
                        uint32_t n_tokens, uint32_t q0, uint32_t n_q_heads, uint32_t n_kv_heads,
                        uint32_t head_dim, uint32_t window, float scale, float *out);

/* Row and elementwise operators (fp32 activations; f32 math as in the
 * reference shaders).  Name dispatch: rmsnorm_{ROW}[_plus1] (bindings x, w,
 * y; groups [rows]), rope_{sliding,global}_{q,k} and the head_dim-128 forms
 * rope_hd128_{sliding,global}_{q,k} (bindings xs, cos_sin), geglu (gate,
 * up, y), add_scaled (a, b, y; push f32 scale). */
/* V quantized in 32-KEY blocks per column and appended at rows pos ..
 * pos+n_tokens-1 (kv_append_global_v_q8, crates/sg-gpu/shaders/
 * kv_append_global_v_q8.wgsl:32-75): src fp32 [n_tokens × row_len]; quants
 * [slot × row_len] int8 (the layout of the K pages); scales f16
 * [slot/32 × row_len], one per (32-key block, column), the kv_quant_q8 rule
 * over the block's live rows.  pos must be a multiple of 32. */
int sgq_kv_append_v_q8(sgq_ctx *ctx, const float *src, uint32_t n_tokens, uint32_t row_len,
                       uint32_t pos, int8_t *v_quants, uint16_t *v_scales);
/* Prefill attention with int8 PV (attn_prefill_global_flash_sp_ipv,
 * crates/sg-gpu/shaders/attn_prefill_global_flash_sp_ipv.wgsl:1-20,
 * :134-210): causal over a linear Q8_0 cache holding positions
 * 0..q0+n_tokens-1, K pages as sgq_attn_prefill_q8, V quants with the
 * key-blocked scales of sgq_kv_append_v_q8.  P is quantized per (query,
 * 32-key block) in the kernel and the softmax denominator sums the
 * dequantized P; head_dim 128. */
int sgq_attn_prefill_ipv(sgq_ctx *ctx, const float *q, const int8_t *k_quants,
                         const uint16_t *k_scales, const int8_t *v_quants,
                         const uint16_t *v_scales_kb, uint32_t n_tokens, uint32_t q0,
                         uint32_t n_q_heads, uint32_t n_kv_heads, uint32_t head_dim, float scale,
                         float *out);

/* rmsnorm.wgsl:24-61: y = x·rsqrt(mean(x²)+eps)·w per row of row_len
 * (w + 1 when plus_one; w NULL = weightless). */
int sgq_rmsnorm(sgq_ctx *ctx, const float *x, const float *w, float *y, uint32_t rows,
                uint32_t row_len, int plus_one, float eps);
/* rope.wgsl:35-52, in place: rows [n_tokens × n_heads × head_dim]; pair i
 * couples dims (i, i+head_dim/2), the first rot_dims/2 pairs rotate by
 * cos_sin[token × rot_dims/2] (cos, sin) (crates/sg-model/src/rope.rs). */
int sgq_rope(sgq_ctx *ctx, float *x, const float *cos_sin, uint64_t n_tokens, uint32_t n_heads,
             uint32_t head_dim, uint32_t rot_dims);
/* geglu.wgsl:14-24: y = gelu_tanh(gate)·up. */
int sgq_geglu(sgq_ctx *ctx, const float *gate, const float *up, float *y, uint64_t n);
/* add_scaled.wgsl:21-27: y = (a + b)·s. */
int sgq_add_scaled(sgq_ctx *ctx, const float *a, const float *b, float *y, uint64_t n, float s);

/* ---- decode-step driver ------------------------------------------------- */
/* A random-init decoder of the reference's model family (the CPU forward pass
 * crates/sg-model/src/reference.rs:157-316 and the GPU graph
 * crates/sg-model/src/graph.rs:478-756): Q4_0 linears, weighted q/k norms,
 * weightless v norm, NEOX RoPE (sliding theta / global theta with the first
 * global_rope_frac of pairs rotating), Q8_0 K and V pages (a ring of
 * sliding_window slots on sliding layers, max_ctx slots on global ones),
 * GeGLU FFN, post-norms, per-layer output scale, tied Q4_0 LM head with
 * softcap.  Layer l is global iff l % global_every == global_every - 1.
 * Weights: Q4_0 d = f16(|N(0, weight_sigma)|) with uniform nibbles, norm
 * weights N(1, 0.1), layer output scales N(0.9, 0.05), all keyed by seed. */
typedef struct sgq_model sgq_model;
typedef struct {
    uint32_t n_layers, hidden, ffn, n_q_heads, n_kv_heads, head_dim, vocab;
    uint32_t sliding_window, global_every, max_ctx;
    float rope_theta_sliding, rope_theta_global, global_rope_frac;
    float eps, attn_scale, final_softcap, weight_sigma;
    uint32_t global_k_eq_v; /* 1: global layers take V from the K projection */
    uint32_t prefill_chunk; /* tokens per prefill chunk (its buffers are sized by it) */
    uint64_t seed;
    /* The real checkpoint's per-kind geometry (crates/sg-gguf/src/desc.rs:
     * 66-93): global layers' head_dim and kv heads (0: as the sliding
     * layers'), and a Q6_K token embedding / tied head (q6_k.rs:25-62)
     * instead of Q4_0.  Any of them, or head_dim != 128, selects the
     * any-geometry attention (decode modes 2 and 3 only; see
     * sgq_model_set_decode_mode). */
    uint32_t head_dim_global;
    uint32_t n_kv_heads_global;
    uint32_t embed_q6k;
    uint32_t reserved;
} sgq_model_config;

/* The benchmark shape: 62 layers, hidden 5376, ffn 21504, 32 q / 16 kv heads
 * of 128, vocab 262144, window 1024, every 6th layer global, 16K context,
 * 4096-token prefill chunks. */
void sgq_model_default_config(sgq_model_config *cfg);
/* Allocates and fills every weight and cache on the context's device. */
int sgq_model_create(sgq_ctx *ctx, const sgq_model_config *cfg, sgq_model **out);
int sgq_model_destroy(sgq_model *model);
/* Forget the cached context (position back to 0). */
int sgq_model_reset(sgq_model *model);
uint32_t sgq_model_position(const sgq_model *model);
/* One decode step at the current position: appends token's K/V, writes the
 * softcapped logits [vocab] fp32 to the device buffer `logits`, advances the
 * position.  Enqueued on the context's stream (no host wait).  The _graph
 * form records the step into a hipGraph on first use (per logits buffer) and
 * replays it; the per-token inputs travel through a device step buffer. */
int sgq_model_decode(sgq_model *model, uint32_t token, float *logits);
int sgq_model_decode_graph(sgq_model *model, uint32_t token, float *logits);
/* Decode implementation (no counterpart in the reference, whose graph is one
 * dispatch per operator, graph.rs:478-756): 0 = one kernel per operator
 * (the _graph form captures them), 2 = five launches per layer (QKV, attention, O, gate/up, down GEMVs) with
 * the norms, residual updates, GeGLU and the split merge fused into them
 * (the _graph form captures them), 3 = one kernel per operator at any
 * supported geometry: head_dim 128/256/512 per layer kind, 1/2/4/8 query
 * heads per kv head, Q4_0 or Q6_K embedding (the real checkpoint's shape;
 * attention on the VALU).  Models of another geometry than the benchmark's
 * (head_dim 128 everywhere, <= 2 q heads per kv head, Q4_0 embedding) run in
 * mode 2 (the default for them: the fused GEMVs around the any-geometry
 * attention) or mode 3; their prefill is the chunked MMQ driver at their
 * per-layer widths (head_dim 256/512 prefill attention).
 * Mode 1 (a persistent one-launch step, measured slower) is not built and
 * fails with SGQ_ERR_VALIDATION. */
int sgq_model_set_decode_mode(sgq_model *model, int mode);
int sgq_model_decode_mode(const sgq_model *model);
/* Waits for the context's stream. */
int sgq_model_status(sgq_model *model);
/* Prefill (GpuModel::prefill, crates/sg-model/src/graph.rs:1451-1482): runs
 * the host tokens[0..n) at positions pos..pos+n-1 in chunks of
 * prefill_chunk, appends their K/V, advances the position, and writes the
 * last token's softcapped logits to the device buffer `logits` (NULL: none).
 * Linear layers are int8 MMQs over Q8_0 activations (the reference's
 * prefill path), attention is the flash kernel of sgq_attn_prefill_q8 with
 * keys before the chunk from the cache (ring or linear).  Returns after the
 * last chunk is enqueued. */
int sgq_model_prefill(sgq_model *model, const uint32_t *tokens, uint32_t n_tokens, float *logits);
/* Synthetic context: fills the K/V pages of positions 0..n_tokens-1 (the
 * last sliding_window of them on ring layers) with Q8_0 of N(0,1) values and
 * sets the position to n_tokens, so a decode step can be measured at a long
 * context without decoding up to it.  Blocks the host until done. */
int sgq_model_fill_cache(sgq_model *model, uint32_t n_tokens, uint64_t seed);
/* Device pointer and byte size of a named tensor: layer -1 for
 * token_embd / output_norm / x (the residual stream); per layer the GGUF
 * names attn_q, attn_k, attn_v, attn_output, ffn_gate, ffn_up, ffn_down,
 * attn_norm, attn_q_norm, attn_k_norm, post_attention_norm, ffn_norm,
 * post_ffw_norm, layer_output_scale and the cache pages k_quants, k_scales,
 * v_quants, v_scales. */
int sgq_model_tensor(const sgq_model *model, int layer, const char *name, void **ptr,
                     uint64_t *bytes);

/* ---- GGUF (crates/sg-gguf/src/parse.rs:112-210): v3 files, read-only
 * mapped; tensors of type F32 (0), F16 (1), Q4_0 (2), Q8_0 (8), Q6_K (14);
 * dims in ggml order (dims[0] contiguous); `data` points into the mapping
 * and lives until sgq_gguf_close.  Malformed files fail with
 * SGQ_ERR_VALIDATION and a message naming what is wrong. */
typedef struct sgq_gguf sgq_gguf;
typedef struct {
    const char *name;
    uint32_t type;
    uint32_t n_dims;
    uint64_t dims[4];
    uint64_t offset; /* within the data section */
    uint64_t bytes;
    const void *data;
} sgq_gguf_tensor;
int sgq_gguf_open(const char *path, sgq_gguf **out);
int sgq_gguf_close(sgq_gguf *gguf);
uint64_t sgq_gguf_tensor_count(const sgq_gguf *gguf);
int sgq_gguf_tensor_at(const sgq_gguf *gguf, uint64_t i, sgq_gguf_tensor *out);
int sgq_gguf_tensor_find(const sgq_gguf *gguf, const char *name, sgq_gguf_tensor *out);
/* Metadata: any integer type (and bool) / f32-f64 / string. */
int sgq_gguf_meta_int(const sgq_gguf *gguf, const char *key, int64_t *out);
int sgq_gguf_meta_float(const sgq_gguf *gguf, const char *key, double *out);
int sgq_gguf_meta_string(const sgq_gguf *gguf, const char *key, const char **out);
/* Upload a GGUF's weights into a model (weights.rs / desc.rs expected_tensors:
 * token_embd, output_norm and per layer blk.N.{attn_q, attn_k, attn_v (not on
 * K=V global layers), attn_output, attn_q_norm, attn_k_norm, attn_norm,
 * post_attention_norm, ffn_norm, post_ffw_norm, ffn_gate, ffn_up, ffn_down,
 * layer_output_scale}.weight).  Every tensor's type and shape is checked
 * against the model's config before anything is written; matrices and the
 * tied embedding must be Q4_0, norms F32.  An optional rope_freqs.weight must
 * match global_rope_frac. */
int sgq_model_load_gguf(sgq_model *model, const sgq_gguf *gguf);

/* ---- synthetic inputs (not on the hot path; for benches and tests) ------ */
/* Q4_0 blocks with d = f16(|N(0, sigma)|) and uniform nibble bytes, from a
 * counter-based generator keyed by (seed, block index). */
int sgq_fill_q4_0_random(sgq_ctx *ctx, void *w, uint64_t n_blocks, uint64_t seed, float sigma);
/* fp32 N(mean, sigma) from a counter-based generator keyed by (seed, index). */
int sgq_fill_normal(sgq_ctx *ctx, float *x, uint64_t n, uint64_t seed, float mean,
                    float sigma);

#ifdef __cplusplus
}
#endif
#endif /* SGQ_H */
