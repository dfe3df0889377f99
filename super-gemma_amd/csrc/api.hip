// libsgq C ABI: context, buffers, the variant registry with name dispatch,
// recorded graphs, step buffer, timers and the typed entry points.
//
// The name registry is the drop-in half of the boundary: it accepts the
// variant names of crates/sg-gpu/build.rs VARIANTS (plus the same families
// at the BASELINE geometry, e.g. head_dim 128), with their binding order,
// push-constant layout and group-count convention, and routes each dispatch
// to the typed launcher that computes its own HIP grid.
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "sgq_internal.h"

struct sgq_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    void *workspace = nullptr;  // per-context scratch (GEMV x limb table)
    bool capturing = false;
    hipEvent_t t0 = nullptr, t1 = nullptr;
};

struct sgq_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

namespace sgq {

static thread_local char g_err[1024] = "";

int fail(int status, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return status;
}

int check_hip(hipError_t e, const char *what) {
    return fail(SGQ_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

const DeviceInfo &device_info() {
    static DeviceInfo info[16];
    static bool done[16] = {};
    static std::mutex mu;
    int dev = 0;
    (void)hipGetDevice(&dev);
    if (dev < 0 || dev >= 16) dev = 0;
    std::lock_guard<std::mutex> lock(mu);
    if (!done[dev]) {
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, dev) == hipSuccess) info[dev].cus = p.multiProcessorCount;
        done[dev] = true;
    }
    return info[dev];
}

hipStream_t ctx_stream(const sgq_ctx *ctx) { return ctx ? ctx->stream : nullptr; }
void *ctx_workspace(const sgq_ctx *ctx) { return ctx ? ctx->workspace : nullptr; }

}  // namespace sgq

using namespace sgq;

// ---------------------------------------------------------------------------
// Kernel registry
// ---------------------------------------------------------------------------

enum class Kind {
    Gemv,          // gemv_q4_0_k{K} / gemv_q4_0_generic
    GemvQ6kLogits, // gemv_q6_k_logits: K 5376, rows padded to 4416 B, softcap 30
    QuantQ8,       // kv_quant_q8
    DequantQ8,     // kv_dequant_q8
    AppendQ8,      // kv_append_global_q8 (linear) / kv_append_sliding_q8 (ring)
    GemmI8,        // gemm_q4_0_i8_*_k{K}_n{N}: groups [M/64, N/16]
    GemmI8Down,    // gemm_q4_0_i8_bb_pfd{1,2,4}: K=21504, N=5376, groups [M/64, 336]
    GemmI8Split,   // gemm_q4_0_i8_splitk{S}_k{K}_n{N} (no reference counterpart)
    RmsNorm,       // rmsnorm_{ROW}[_plus1]: groups [rows]
    Rope,          // rope_{sliding,global}_{q,k} (+ head_dim-128 forms)
    Geglu,         // geglu
    AddScaled,     // add_scaled (push: f32 scale)
    AttnDecode,    // attn_decode_{sliding,global}_q8_hd128: groups [n_kv, n_splits]
    AttnReduce,    // attn_reduce_d128: groups [n_q]
    AttnPrefill,   // attn_prefill_{global_flash,sliding_ring}_q8_hd128
    AttnPrefillIpv,  // attn_prefill_global_flash_ipv_hd128 (int8 PV, key-blocked V)
    AppendVQ8,     // kv_append_global_v_q8 (V in 32-key blocks per column)
    AttnDecodePages,  // attn_decode_{sliding,global,global_q8k}: f16 q / V pages
    AttnReducePages,  // attn_reduce_d{256,512}: f16 rows out
    AppendF16,     // kv_append_{sliding,global}: f16 rows
    AttnPrefillPages,  // attn_prefill_{sliding[_ring],global[_flash[_sp[_q8,_iq]]]}
};

struct sgq_kernel {
    std::string name;
    Kind kind;
    sgq_kernel_info info;
    uint32_t k = 0, n = 0;  // baked dims (0 = from push/bindings)
    uint32_t param = 0;     // split factor, ring length, ...
    // activation type: f16 (the reference's) under the reference's names,
    // fp32 under the same names with the suffix _f32
    bool f16 = false;
};

namespace {

// Every name a caller may look up; the numbers in the pattern names are
// parsed from the actual name at lookup (e.g. gemv_q4_0_k5376).
const char *const kNames[] = {
    "gemv_q4_0_k5376",  "gemv_q4_0_k8192",  "gemv_q4_0_k16384", "gemv_q4_0_k21504",
    "gemv_q4_0_k4096",  "gemv_q4_0_generic", "kv_quant_q8",     "kv_dequant_q8",
    "kv_append_global_q8",
    "gemm_q4_0_i8_swz_m4n1_k5376_n21504",   "gemm_q4_0_i8_swz_m4n1_k21504_n5376",
    "gemm_q4_0_i8_swz_m4n1_k5376_n8192",    "gemm_q4_0_i8_swz_m4n1_k5376_n16384",
    "gemm_q4_0_i8_swz_m4n1_k5376_n4096",    "gemm_q4_0_i8_swz_m4n1_k5376_n2048",
    "gemm_q4_0_i8_swz_m4n1_k8192_n5376",    "gemm_q4_0_i8_swz_m4n1_k16384_n5376",
    "gemm_q4_0_i8_swz_m4n1_k4096_n5376",    "gemm_q4_0_i8_bb_pfd4",
    "gemm_q4_0_i8_splitk4_k21504_n5376",
    "rmsnorm_5376", "rmsnorm_5376_plus1", "rmsnorm_512", "rmsnorm_512_plus1",
    "rmsnorm_256",  "rmsnorm_256_plus1",  "rmsnorm_128", "rmsnorm_128_plus1",
    "rope_sliding_q", "rope_sliding_k", "rope_global_q", "rope_global_k",
    "rope_hd128_sliding_q", "rope_hd128_sliding_k", "rope_hd128_global_q", "rope_hd128_global_k",
    "geglu", "add_scaled", "gemv_q6_k_logits",
    "kv_append_sliding_q8",
    "attn_decode_sliding_q8_hd128", "attn_decode_global_q8_hd128", "attn_reduce_d128",
    "attn_prefill_global_flash_q8_hd128", "attn_prefill_sliding_ring_q8_hd128",
    "kv_append_global_v_q8", "attn_prefill_global_flash_ipv_hd128",
    "attn_decode_sliding", "attn_decode_global", "attn_decode_global_q8k",
    "attn_reduce_d256", "attn_reduce_d512", "kv_append_sliding", "kv_append_global",
    "attn_prefill_sliding", "attn_prefill_sliding_ring", "attn_prefill_global",
    "attn_prefill_global_flash", "attn_prefill_global_flash_sp", "attn_prefill_global_flash_sp_q8",
    "attn_prefill_global_flash_sp_iq", "attn_prefill_global_flash_sp_ipv",
    "attn_prefill_global_flash_sp_ipv_bcast",
    // the same kernels over fp32 activations
    "gemv_q4_0_k5376_f32", "gemv_q4_0_k8192_f32", "gemv_q4_0_k16384_f32", "gemv_q4_0_k21504_f32",
    "gemv_q4_0_k4096_f32", "gemv_q4_0_generic_f32", "kv_quant_q8_f32", "kv_dequant_q8_f32",
    "kv_append_global_q8_f32", "kv_append_global_v_q8_f32",
    "gemm_q4_0_i8_swz_m4n1_k5376_n21504_f32", "gemm_q4_0_i8_bb_pfd4_f32",
    "rmsnorm_5376_f32", "rmsnorm_256_f32", "rmsnorm_512_f32", "rope_sliding_q_f32",
    "rope_global_q_f32", "geglu_f32", "add_scaled_f32", "gemv_q6_k_logits_f32",
};

// The benchmark geometry of the hd128 attention forms (32 query heads over
// 16 kv heads of 128, sliding window and ring 1024), baked into the names as
// the reference bakes HEAD_DIM / N_KV_HEADS / Q_PER_KV / WINDOW into its
// variants (crates/sg-gpu/build.rs:331-430).
constexpr uint32_t kAttnNQ = 32, kAttnNKv = 16, kAttnWindow = 1024;

// The real checkpoint's decode-side variants over f16 pages (crates/sg-gpu/
// build.rs:255-394): head_dim 256 sliding (16 kv heads, 2 q heads each,
// ring 1024) and 512 global (4 kv heads, 8 q heads each, K = V rows).
constexpr uint32_t kRealNQ = 32, kSlNKv = 16, kGlNKv = 4;

// The real checkpoint's prefill attention variants (crates/sg-gpu/build.rs:
// 395-438, :2206-2335): head_dim, kv heads, page format (the kernel's
// PfFmt: 1 Q8_0 K/V with f16 q, 2 f16 pages, 3 int8 q and Q8_0 K with f16
// V, 4 the same with int8 V under key-blocked scales and int8 P), window,
// ring, bindings, and the grid form: per token [n_kv, M] or per 16-query
// tile [32, M/16].
struct PrefillVariant {
    const char *name;
    uint32_t head_dim, n_kv, fmt, window, ring, bindings;
    bool per_token;
};
const PrefillVariant kPrefill[] = {
    {"attn_prefill_sliding", 256, kSlNKv, 2, kAttnWindow, 0, 5, true},
    {"attn_prefill_sliding_ring", 256, kSlNKv, 2, kAttnWindow, kAttnWindow, 7, true},
    {"attn_prefill_global", 512, kGlNKv, 2, 0, 0, 5, true},
    {"attn_prefill_global_flash", 512, kGlNKv, 2, 0, 0, 5, false},
    {"attn_prefill_global_flash_sp", 512, kGlNKv, 2, 0, 0, 5, false},
    {"attn_prefill_global_flash_sp_q8", 512, kGlNKv, 1, 0, 0, 7, false},
    {"attn_prefill_global_flash_sp_iq", 512, kGlNKv, 3, 0, 0, 7, false},
    {"attn_prefill_global_flash_sp_ipv", 512, kGlNKv, 4, 0, 0, 8, false},
    {"attn_prefill_global_flash_sp_ipv_bcast", 512, kGlNKv, 4, 0, 0, 8, false},
};

// RoPE variants: (name, head_dim, rot_dims, n_heads).  The first four are
// the reference's (crates/sg-gpu/build.rs:126-164: the real checkpoint's
// head_dim 256 sliding / 512 global with partial rotation 0.25); the
// hd128 forms, which have no counterpart in the reference, are the
// benchmark decoder's (32 q / 16 kv heads of 128).
struct RopeVariant {
    const char *name;
    uint32_t head_dim, rot_dims, n_heads;
};
const RopeVariant kRope[] = {
    {"rope_sliding_q", 256, 256, 32}, {"rope_sliding_k", 256, 256, 16},
    {"rope_global_q", 512, 128, 32},  {"rope_global_k", 512, 128, 4},
    {"rope_hd128_sliding_q", 128, 128, 32}, {"rope_hd128_sliding_k", 128, 128, 16},
    {"rope_hd128_global_q", 128, 32, 32},   {"rope_hd128_global_k", 128, 32, 16},
};

bool parse_u32_after(const std::string &s, const std::string &key, uint32_t *out) {
    size_t p = s.rfind(key);
    if (p == std::string::npos) return false;
    p += key.size();
    if (p >= s.size() || s[p] < '0' || s[p] > '9') return false;
    uint64_t v = 0;
    while (p < s.size() && s[p] >= '0' && s[p] <= '9') v = v * 10 + (uint64_t)(s[p++] - '0');
    if (v > 0xffffffffu) return false;
    *out = (uint32_t)v;
    return true;
}

bool starts_with(const std::string &s, const char *p) { return s.rfind(p, 0) == 0; }

// Build the registry entry for `name` (without an _f32 suffix), or return
// false if it is unknown.
bool resolve_base(const std::string &name, sgq_kernel *k) {
    k->name = name;
    k->info = {{64, 1, 1}, 0, 0, 0};
    if (starts_with(name, "gemv_q4_0_")) {
        k->kind = Kind::Gemv;
        k->info.bindings = 3;
        if (name == "gemv_q4_0_generic") {
            k->info.push_bytes = 4;
            return true;
        }
        if (!parse_u32_after(name, "_k", &k->k)) return false;
        return name == "gemv_q4_0_k" + std::to_string(k->k) && k->k % 64 == 0 && k->k > 0;
    }
    if (name == "gemv_q6_k_logits") {  // crates/sg-gpu/build.rs:322-327
        k->kind = Kind::GemvQ6kLogits;
        k->info.bindings = 3;
        k->k = 5376;        // BLOCKS_PER_ROW 21
        k->param = 4416;    // ROW_WORDS 1104 × 4 bytes
        return true;
    }
    if (name == "kv_quant_q8") {
        k->kind = Kind::QuantQ8;
        k->info.bindings = 3;
        return true;
    }
    if (name == "kv_dequant_q8") {
        k->kind = Kind::DequantQ8;
        k->info.bindings = 3;
        return true;
    }
    if (name == "kv_append_global_q8" || name == "kv_append_sliding_q8") {
        k->kind = Kind::AppendQ8;
        k->info.bindings = 4;
        k->param = name == "kv_append_sliding_q8" ? kAttnWindow : 0;  // ring slots
        return true;
    }
    if (name == "kv_append_global_v_q8") {
        // bindings: 0 src f16 (fp32: _f32) [n_tok × row], 1 scales f16 [block × row],
        // 2 quants [slot × row], 3 step (pos = step[0], a multiple of 32);
        // row = groups.y·32 when groups.y > 1, else 2048 (16 kv heads × 128,
        // also the real checkpoint's 4 global kv heads × 512)
        k->kind = Kind::AppendVQ8;
        k->info.bindings = 4;
        return true;
    }
    if (name == "attn_prefill_global_flash_ipv_hd128") {
        // 0 q fp32 [M × 32 × 128], 1 k_quants, 2 k_scales (Q8_0 pages), 3 v
        // quants [slot × 16 × 128], 4 v scales key-blocked [slot/32 × 16 ×
        // 128], 5 out, 6 step; push {scale: f32}; groups [32, ceil(M/16)];
        // causal, q0 = step[3], keys 0..q0+M-1 in the linear cache
        // (attn_prefill_global_flash_sp_ipv.wgsl:24-35)
        k->kind = Kind::AttnPrefillIpv;
        k->info = {{256, 1, 1}, 7, 4, 0};
        k->k = kAttnNQ;
        k->n = kAttnNKv;
        return true;
    }
    if (name == "attn_decode_sliding_q8_hd128" || name == "attn_decode_global_q8_hd128") {
        // bindings: 0 q fp32 [n_q × 128], 1 k_quants, 2 k_scales, 3 v_quants,
        // 4 v_scales (Q8_0 pages [slot × n_kv × 128]), 5 part fp32
        // [n_q × n_splits × 130], 6 step; push {n_splits: u32, scale: f32};
        // kv_len = step[1] (sliding ring) or step[2] (global)
        k->kind = Kind::AttnDecode;
        k->info = {{256, 1, 1}, 7, 8, 0};
        k->k = kAttnNQ;
        k->n = kAttnNKv;
        k->param = name == "attn_decode_sliding_q8_hd128" ? 1 : 2;
        return true;
    }
    if (name == "attn_decode_sliding" || name == "attn_decode_global" ||
        name == "attn_decode_global_q8k") {
        // f16: 0 q f16 [32 × HD], 1 k pages, 2 v pages f16 [slot × n_kv × HD],
        //   3 part fp32 [32 × n_splits × (HD + 2)], 4 step
        // q8k: 1 k_quants i8, 2 k_scales f16 [slot × n_kv × HD/32], 3 v f16,
        //   4 part, 5 step
        // push {n_splits: u32, scale: f32}; groups [n_kv, n_splits, 1];
        // kv_len = step[1] (sliding) or step[2] (global)
        // (attn_decode_sliding.wgsl:16-50, attn_decode_global_q8k.wgsl)
        const bool q8k = name == "attn_decode_global_q8k";
        const bool sl = name == "attn_decode_sliding";
        k->kind = Kind::AttnDecodePages;
        k->info = {{256, 1, 1}, q8k ? 6u : 5u, 8, 0};
        k->k = sl ? 256 : 512;          // head_dim
        k->n = sl ? kSlNKv : kGlNKv;    // kv heads
        k->param = (sl ? 1 : 2) | (q8k ? 4 : 0);  // step word, Q8_0 K
        return true;
    }
    if (name == "attn_reduce_d256" || name == "attn_reduce_d512") {
        // 0 part, 1 out f16 [32 × HD]; push n_splits; groups [32, 1, 1]
        // (attn_reduce.wgsl:14-30)
        k->kind = Kind::AttnReducePages;
        k->info = {{256, 1, 1}, 2, 4, 0};
        k->k = name == "attn_reduce_d256" ? 256 : 512;
        return true;
    }
    if (name == "kv_append_sliding" || name == "kv_append_global") {
        // 0 src f16 [n_tok × ROW], 1 dst f16 [slot × ROW], 2 step; groups
        // cover n_tok × ROW elements at 256 per group; ROW 4096 (sliding,
        // ring 1024) or 2048 (global, linear) (kv_append.wgsl:15-35)
        k->kind = Kind::AppendF16;
        k->info = {{256, 1, 1}, 3, 0, 0};
        const bool sl = name == "kv_append_sliding";
        k->k = sl ? kSlNKv * 256 : kGlNKv * 512;  // row halves
        k->param = sl ? kAttnWindow : 0;          // ring slots
        return true;
    }
    for (uint32_t i = 0; i < sizeof kPrefill / sizeof kPrefill[0]; i++)
        if (name == kPrefill[i].name) {
            // per-token grids: [n_kv, M, 1], M = groups.y; flash grids:
            // [32, M/16, 1], M = 16·groups.y; push {scale: f32}; q0 = step[3]
            // f16 (5): 0 q, 1 K, 2 V, 3 out, 4 step
            // ring (7): 0 q, 1 K ring, 2 V ring, 3 chunk K, 4 chunk V, 5 out, 6 step
            // q8 (7): 0 q f16, 1 k_quants, 2 k_scales, 3 v_quants, 4 v_scales, 5 out, 6 step
            // iq (7): 0 q_i8, 1 q_scales, 2 k_quants, 3 k_scales, 4 V f16, 5 out, 6 step
            // ipv (8): 0 q_i8, 1 q_scales, 2 k_quants, 3 k_scales, 4 v_quants, 5 key-blocked
            //   v_scales [slot/32 × n_kv × HD], 6 out, 7 step
            k->kind = Kind::AttnPrefillPages;
            k->info = {{64, 1, 1}, kPrefill[i].bindings, 4, 0};
            k->param = i;
            return true;
        }
    if (name == "attn_reduce_d128") {
        // bindings: 0 part, 1 out fp32 [n_q × 128]; push n_splits; groups [n_q]
        k->kind = Kind::AttnReduce;
        k->info = {{256, 1, 1}, 2, 4, 0};
        k->k = kAttnNQ;
        k->n = kAttnNKv;
        return true;
    }
    if (name == "attn_prefill_global_flash_q8_hd128" ||
        name == "attn_prefill_sliding_ring_q8_hd128") {
        // global: 0 q fp32 [M × n_q × 128], 1 k_quants, 2 k_scales,
        //   3 v_quants, 4 v_scales (linear cache holding the chunk's keys),
        //   5 out fp32, 6 step; groups [n_q, ceil(M/16)]
        // sliding: 0 q, 1..4 the ring's K/V pages, 5..8 the chunk's K/V
        //   pages [M × n_kv × 128], 9 out, 10 step; groups [n_kv, M]
        // push {scale: f32}; q0 = step[3]; M = out range / (n_q·128·4)
        k->kind = Kind::AttnPrefill;
        const bool ring = name == "attn_prefill_sliding_ring_q8_hd128";
        k->info = {{256, 1, 1}, ring ? 11u : 7u, 4, 0};
        k->k = kAttnNQ;
        k->n = kAttnNKv;
        k->param = ring ? kAttnWindow : 0;
        return true;
    }
    if (starts_with(name, "gemm_q4_0_i8_bb_pfd")) {
        k->kind = Kind::GemmI8Down;
        k->info.bindings = 4;
        k->k = 21504;
        k->n = 5376;
        return name == "gemm_q4_0_i8_bb_pfd1" || name == "gemm_q4_0_i8_bb_pfd2" ||
               name == "gemm_q4_0_i8_bb_pfd4";
    }
    if (starts_with(name, "gemm_q4_0_i8_splitk")) {
        k->kind = Kind::GemmI8Split;
        k->info.bindings = 5;
        if (!parse_u32_after(name, "splitk", &k->param)) return false;
        if (!parse_u32_after(name, "_k", &k->k) || !parse_u32_after(name, "_n", &k->n))
            return false;
        return (k->param == 1 || k->param == 2 || k->param == 4 || k->param == 8) &&
               k->k % 64 == 0 && k->n > 0;
    }
    if (starts_with(name, "rmsnorm_")) {
        k->kind = Kind::RmsNorm;
        k->info = {{256, 1, 1}, 3, 0, 0};
        if (!parse_u32_after(name, "rmsnorm_", &k->k) || k->k == 0) return false;
        const std::string base = "rmsnorm_" + std::to_string(k->k);
        k->param = name == base + "_plus1";
        return name == base || k->param;
    }
    for (const RopeVariant &v : kRope)
        if (name == v.name) {
            k->kind = Kind::Rope;
            k->info = {{256, 1, 1}, 2, 0, 0};
            k->k = v.head_dim;
            k->n = v.n_heads;
            k->param = v.rot_dims;
            return true;
        }
    if (name == "geglu") {
        k->kind = Kind::Geglu;
        k->info = {{256, 1, 1}, 3, 0, 0};
        return true;
    }
    if (name == "add_scaled") {
        k->kind = Kind::AddScaled;
        k->info = {{256, 1, 1}, 3, 4, 0};
        return true;
    }
    if (starts_with(name, "gemm_q4_0_i8_")) {
        k->kind = Kind::GemmI8;
        k->info.bindings = 4;
        if (!parse_u32_after(name, "_k", &k->k) || !parse_u32_after(name, "_n", &k->n))
            return false;
        return k->k % 64 == 0 && k->n > 0;
    }
    return false;
}

// Kernels that exist for both activation types: the reference's names
// take f16 activations as its shaders do; NAME_f32 is the same kernel over
// fp32 activations.  The families of our own (head_dim-128 forms, the
// split-K MMQ, the ring Q8 append) are fp32 only and take no suffix.
bool dual_type(const sgq_kernel &k) {
    switch (k.kind) {
        case Kind::Gemv:
        case Kind::GemvQ6kLogits:
        case Kind::RmsNorm:
        case Kind::Geglu:
        case Kind::AddScaled:
        case Kind::QuantQ8:
        case Kind::DequantQ8:
        case Kind::GemmI8:
        case Kind::GemmI8Down:
        case Kind::AppendVQ8: return true;
        case Kind::Rope: return k.k != 128;
        case Kind::AppendQ8: return k.param == 0;  // kv_append_global_q8
        default: return false;
    }
}

bool resolve(const std::string &full, sgq_kernel *k) {
    static const std::string sfx = "_f32";
    const bool f32 = full.size() > sfx.size() &&
                     full.compare(full.size() - sfx.size(), sfx.size(), sfx) == 0;
    if (!resolve_base(f32 ? full.substr(0, full.size() - sfx.size()) : full, k)) return false;
    k->name = full;
    if (!dual_type(*k)) return !f32;
    k->f16 = !f32;
    return true;
}

struct Registry {
    std::mutex mu;
    std::vector<sgq_kernel *> loaded;
    ~Registry() {
        for (auto *k : loaded) delete k;
    }
};
Registry &registry() {
    static Registry r;
    return r;
}

// Binding table lookup with range check.
constexpr uint32_t kMaxBindings = 16;
struct Binds {
    const sgq_binding *b[kMaxBindings] = {};
    int get(uint32_t i, void **p, uint64_t *range) const {
        if (i >= kMaxBindings || !b[i]) return fail(SGQ_ERR_VALIDATION, "binding %u missing", i);
        *p = static_cast<uint8_t *>(b[i]->ptr) + b[i]->offset;
        *range = b[i]->range;
        return SGQ_OK;
    }
};

}  // namespace

extern "C" {

const char *sgq_last_error(void) { return g_err; }
const char *sgq_version(void) { return "sgq 0.1 (gfx950)"; }

int sgq_ctx_create(int device, sgq_ctx **out) {
    if (!out) return fail(SGQ_ERR_VALIDATION, "out is NULL");
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0)
        return fail(SGQ_ERR_NO_DEVICE, "no HIP device");
    if (device < 0 || device >= count) return fail(SGQ_ERR_NO_DEVICE, "device %d absent", device);
    SGQ_HIP(hipSetDevice(device));
    hipDeviceProp_t p;
    SGQ_HIP(hipGetDeviceProperties(&p, device));
    if (std::strncmp(p.gcnArchName, "gfx950", 6) != 0)
        return fail(SGQ_ERR_NO_DEVICE, "device %d is %s, libsgq is built for gfx950", device,
                    p.gcnArchName);
    auto *c = new sgq_ctx;
    c->device = device;
    if (hipEventCreate(&c->t0) != hipSuccess || hipEventCreate(&c->t1) != hipSuccess ||
        hipMalloc(&c->workspace, kWorkspaceBytes) != hipSuccess ||
        hipMemset(c->workspace, 0, kWorkspaceBytes) != hipSuccess) {
        sgq_ctx_destroy(c);
        return fail(SGQ_ERR_HIP, "context resources (events / %zu-byte workspace) failed",
                    kWorkspaceBytes);
    }
    *out = c;
    return SGQ_OK;
}

int sgq_ctx_destroy(sgq_ctx *ctx) {
    if (!ctx) return SGQ_OK;
    if (ctx->t0) (void)hipEventDestroy(ctx->t0);
    if (ctx->t1) (void)hipEventDestroy(ctx->t1);
    if (ctx->workspace) (void)hipFree(ctx->workspace);
    delete ctx;
    return SGQ_OK;
}

int sgq_ctx_set_stream(sgq_ctx *ctx, void *hip_stream) {
    if (!ctx) return fail(SGQ_ERR_VALIDATION, "ctx is NULL");
    ctx->stream = static_cast<hipStream_t>(hip_stream);
    return SGQ_OK;
}

int sgq_sync(sgq_ctx *ctx) {
    if (!ctx) return fail(SGQ_ERR_VALIDATION, "ctx is NULL");
    SGQ_HIP(hipStreamSynchronize(ctx->stream));
    return SGQ_OK;
}

int sgq_buf_alloc(sgq_ctx *ctx, uint64_t bytes, void **dev_ptr) {
    if (!ctx || !dev_ptr) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    SGQ_HIP(hipSetDevice(ctx->device));
    SGQ_HIP(hipMalloc(dev_ptr, bytes ? bytes : 256));
    return SGQ_OK;
}

int sgq_buf_free(sgq_ctx *ctx, void *dev_ptr) {
    (void)ctx;
    if (dev_ptr) SGQ_HIP(hipFree(dev_ptr));
    return SGQ_OK;
}

int sgq_buf_upload(sgq_ctx *ctx, void *dst_dev, const void *src_host, uint64_t bytes) {
    if (!ctx) return fail(SGQ_ERR_VALIDATION, "ctx is NULL");
    SGQ_HIP(hipMemcpyAsync(dst_dev, src_host, bytes, hipMemcpyHostToDevice, ctx->stream));
    SGQ_HIP(hipStreamSynchronize(ctx->stream));
    return SGQ_OK;
}

int sgq_buf_download(sgq_ctx *ctx, void *dst_host, const void *src_dev, uint64_t bytes) {
    if (!ctx) return fail(SGQ_ERR_VALIDATION, "ctx is NULL");
    SGQ_HIP(hipMemcpyAsync(dst_host, src_dev, bytes, hipMemcpyDeviceToHost, ctx->stream));
    SGQ_HIP(hipStreamSynchronize(ctx->stream));
    return SGQ_OK;
}

int sgq_buf_fill_zero(sgq_ctx *ctx, void *dev_ptr, uint64_t bytes) {
    if (!ctx) return fail(SGQ_ERR_VALIDATION, "ctx is NULL");
    // A memset node recorded into a graph has given wrong results on replays
    // after the first on this hardware pool: refuse instead of capturing one.
    if (ctx->capturing)
        return fail(SGQ_ERR_VALIDATION, "sgq_buf_fill_zero: not allowed while a graph capture is open");
    SGQ_HIP(hipMemsetAsync(dev_ptr, 0, bytes, ctx->stream));
    return SGQ_OK;
}

uint32_t sgq_kernel_count(void) { return (uint32_t)(sizeof kNames / sizeof kNames[0]); }

const char *sgq_kernel_name(uint32_t i) {
    return i < sgq_kernel_count() ? kNames[i] : nullptr;
}

int sgq_kernel_lookup(sgq_ctx *ctx, const char *name, const sgq_kernel **out,
                      sgq_kernel_info *info) {
    (void)ctx;
    if (!name || !out) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    auto *k = new sgq_kernel;
    if (!resolve(name, k)) {
        delete k;
        return fail(SGQ_ERR_UNKNOWN_KERNEL, "unknown kernel variant '%s'", name);
    }
    {
        Registry &r = registry();
        std::lock_guard<std::mutex> lock(r.mu);
        r.loaded.push_back(k);
    }
    *out = k;
    if (info) *info = k->info;
    return SGQ_OK;
}

int sgq_dispatch(sgq_ctx *ctx, const sgq_kernel *kernel, const sgq_binding *bindings,
                 uint32_t n_bindings, const void *push, uint32_t push_bytes,
                 const uint32_t groups[3]) {
    if (!ctx || !kernel || !groups) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    if (push_bytes != kernel->info.push_bytes)
        return fail(SGQ_ERR_VALIDATION, "%s: push constants are %u bytes, got %u",
                    kernel->name.c_str(), kernel->info.push_bytes, push_bytes);
    if (push_bytes && !push) return fail(SGQ_ERR_VALIDATION, "push is NULL");
    Binds B;
    for (uint32_t i = 0; i < n_bindings; i++) {
        if (bindings[i].binding >= kMaxBindings || bindings[i].binding >= kernel->info.bindings)
            return fail(SGQ_ERR_VALIDATION, "%s: binding %u out of range",
                        kernel->name.c_str(), bindings[i].binding);
        B.b[bindings[i].binding] = &bindings[i];
    }
    hipStream_t st = ctx->stream;
    void *p0, *p1, *p2, *p3, *p4;
    uint64_t r0, r1, r2, r3, r4;
    int rc;
    switch (kernel->kind) {
        case Kind::Gemv: {
            // bindings: 0 weights, 1 x, 2 y; groups [N, 1, 1] (one WG per row)
            if ((rc = B.get(0, &p0, &r0)) || (rc = B.get(1, &p1, &r1)) || (rc = B.get(2, &p2, &r2)))
                return rc;
            uint32_t k = kernel->k;
            if (!k) std::memcpy(&k, push, 4);
            const uint32_t n = groups[0];
            const uint64_t es = kernel->f16 ? 2 : 4;
            if (r0 && r0 < (uint64_t)n * (k / 32) * 18)
                return fail(SGQ_ERR_VALIDATION, "%s: weights binding too small", kernel->name.c_str());
            if (r1 && r1 < (uint64_t)k * es)
                return fail(SGQ_ERR_VALIDATION, "%s: x binding too small", kernel->name.c_str());
            if (r2 && r2 < (uint64_t)n * es)
                return fail(SGQ_ERR_VALIDATION, "%s: y binding too small", kernel->name.c_str());
            if (kernel->f16)
                return launch_gemv_q4_0(st, p0, static_cast<const uint16_t *>(p1),
                                        static_cast<uint16_t *>(p2), n, k, ctx->workspace);
            return launch_gemv_q4_0(st, p0, static_cast<const float *>(p1), static_cast<float *>(p2),
                                    n, k, ctx->workspace);
        }
        case Kind::GemvQ6kLogits: {
            // bindings: 0 padded Q6_K rows, 1 x (f16; fp32 for the _f32
            // form), 2 logits fp32; groups [N, 1, 1] (one per vocabulary row)
            if ((rc = B.get(0, &p0, &r0)) || (rc = B.get(1, &p1, &r1)) || (rc = B.get(2, &p2, &r2)))
                return rc;
            const uint32_t n = groups[0];
            if (r0 && r0 < (uint64_t)n * kernel->param)
                return fail(SGQ_ERR_VALIDATION, "%s: weights binding too small", kernel->name.c_str());
            if (r1 && r1 < (uint64_t)kernel->k * (kernel->f16 ? 2 : 4))
                return fail(SGQ_ERR_VALIDATION, "%s: x binding too small", kernel->name.c_str());
            if (r2 && r2 < (uint64_t)n * 4)
                return fail(SGQ_ERR_VALIDATION, "%s: logits binding too small", kernel->name.c_str());
            if (kernel->f16)
                return launch_gemv_q6_k(st, p0, kernel->param, static_cast<const uint16_t *>(p1),
                                        static_cast<float *>(p2), n, kernel->k, 30.0f);
            return launch_gemv_q6_k(st, p0, kernel->param, static_cast<const float *>(p1),
                                    static_cast<float *>(p2), n, kernel->k, 30.0f);
        }
        case Kind::RmsNorm: {
            // bindings: 0 x, 1 w, 2 y; one workgroup per row (groups[0] rows)
            if ((rc = B.get(0, &p0, &r0)) || (rc = B.get(1, &p1, &r1)) || (rc = B.get(2, &p2, &r2)))
                return rc;
            const uint64_t need = (uint64_t)groups[0] * kernel->k * (kernel->f16 ? 2 : 4);
            if ((r0 && r0 < need) || (r2 && r2 < need) || (r1 && r1 < (uint64_t)kernel->k * 4))
                return fail(SGQ_ERR_VALIDATION, "%s: binding too small", kernel->name.c_str());
            if (kernel->f16)
                return launch_rmsnorm(st, static_cast<const uint16_t *>(p0),
                                      static_cast<const float *>(p1), static_cast<uint16_t *>(p2),
                                      groups[0], kernel->k, (int)kernel->param, 1e-6f);
            return launch_rmsnorm(st, static_cast<const float *>(p0), static_cast<const float *>(p1),
                                  static_cast<float *>(p2), groups[0], kernel->k, (int)kernel->param,
                                  1e-6f);
        }
        case Kind::Rope: {
            // bindings: 0 xs (in place) [token × n_heads × head_dim], 1 cos_sin
            // [token × rot/2] (cos, sin); pairs = arrayLength(xs)/head_dim·rot/2
            if ((rc = B.get(0, &p0, &r0)) || (rc = B.get(1, &p1, &r1))) return rc;
            if (!r0) return fail(SGQ_ERR_VALIDATION, "%s: xs range required", kernel->name.c_str());
            const uint64_t rows = r0 / (kernel->f16 ? 2 : 4) / kernel->k;
            const uint64_t tokens = (rows + kernel->n - 1) / kernel->n;
            if (r1 && r1 < tokens * (kernel->param / 2) * 8)
                return fail(SGQ_ERR_VALIDATION, "%s: cos_sin binding too small", kernel->name.c_str());
            if (kernel->f16)
                return launch_rope(st, static_cast<uint16_t *>(p0), static_cast<const float *>(p1),
                                   rows, kernel->k, kernel->param, kernel->n);
            return launch_rope(st, static_cast<float *>(p0), static_cast<const float *>(p1), rows,
                               kernel->k, kernel->param, kernel->n);
        }
        case Kind::Geglu:
        case Kind::AddScaled: {
            // bindings: 0 a (gate), 1 b (up), 2 y; elements = arrayLength(y)
            if ((rc = B.get(0, &p0, &r0)) || (rc = B.get(1, &p1, &r1)) || (rc = B.get(2, &p2, &r2)))
                return rc;
            if (!r2) return fail(SGQ_ERR_VALIDATION, "%s: y range required", kernel->name.c_str());
            const uint64_t es = kernel->f16 ? 2 : 4;
            const uint64_t n = r2 / es;
            if ((r0 && r0 < n * es) || (r1 && r1 < n * es))
                return fail(SGQ_ERR_VALIDATION, "%s: binding too small", kernel->name.c_str());
            if (kernel->f16) {
                const auto *a = static_cast<const uint16_t *>(p0);
                const auto *b = static_cast<const uint16_t *>(p1);
                auto *y = static_cast<uint16_t *>(p2);
                if (kernel->kind == Kind::Geglu) return launch_geglu(st, a, b, y, n);
                float sc;
                std::memcpy(&sc, push, 4);
                return launch_add_scaled(st, a, b, y, n, sc);
            }
            if (kernel->kind == Kind::Geglu)
                return launch_geglu(st, static_cast<const float *>(p0), static_cast<const float *>(p1),
                                    static_cast<float *>(p2), n);
            float sc;
            std::memcpy(&sc, push, 4);
            return launch_add_scaled(st, static_cast<const float *>(p0),
                                     static_cast<const float *>(p1), static_cast<float *>(p2), n, sc);
        }
        case Kind::QuantQ8: {
            // bindings: 0 src fp32, 1 scales f16, 2 quants; blocks = arrayLength(src)/32
            if ((rc = B.get(0, &p0, &r0)) || (rc = B.get(1, &p1, &r1)) || (rc = B.get(2, &p2, &r2)))
                return rc;
            if (!r0) return fail(SGQ_ERR_VALIDATION, "kv_quant_q8: src range required");
            const uint64_t es = kernel->f16 ? 2 : 4;
            const uint64_t n = r0 / es / 32 * 32;
            if ((r1 && r1 < n / 32 * 2) || (r2 && r2 < n))
                return fail(SGQ_ERR_VALIDATION, "%s: scales/quants binding too small",
                            kernel->name.c_str());
            if (kernel->f16)
                return launch_quant_q8_0(st, static_cast<const uint16_t *>(p0),
                                         static_cast<uint16_t *>(p1), static_cast<int8_t *>(p2), n);
            return launch_quant_q8_0(st, static_cast<const float *>(p0), static_cast<uint16_t *>(p1),
                                     static_cast<int8_t *>(p2), n);
        }
        case Kind::DequantQ8: {
            // bindings: 0 scales, 1 quants, 2 out fp32; elements = arrayLength(quants)
            if ((rc = B.get(0, &p0, &r0)) || (rc = B.get(1, &p1, &r1)) || (rc = B.get(2, &p2, &r2)))
                return rc;
            if (!r1) return fail(SGQ_ERR_VALIDATION, "kv_dequant_q8: quants range required");
            if (r2 && r2 < r1 / 32 * 32 * (kernel->f16 ? 2 : 4))
                return fail(SGQ_ERR_VALIDATION, "%s: out binding too small", kernel->name.c_str());
            if (kernel->f16)
                return launch_dequant_q8_0(st, static_cast<const uint16_t *>(p0),
                                           static_cast<const int8_t *>(p1),
                                           static_cast<uint16_t *>(p2), r1 / 32 * 32);
            return launch_dequant_q8_0(st, static_cast<const uint16_t *>(p0),
                                       static_cast<const int8_t *>(p1), static_cast<float *>(p2),
                                       r1 / 32 * 32);
        }
        case Kind::AppendQ8: {
            // bindings: 0 src fp32 [n_tokens × row], 1 scales, 2 quants, 3 step;
            // groups cover n_tokens × row/32 blocks; row length is the group
            // count's y extent when given, else the kv row of the BASELINE
            // geometry (16 kv heads × 128).
            if ((rc = B.get(0, &p0, &r0)) || (rc = B.get(1, &p1, &r1)) || (rc = B.get(2, &p2, &r2)) ||
                (rc = B.get(3, &p3, &r3)))
                return rc;
            const uint32_t row = groups[1] > 1 ? groups[1] * 32 : 2048;
            const uint64_t es = kernel->f16 ? 2 : 4;
            if (!r0 || r0 % (row * es))
                return fail(SGQ_ERR_VALIDATION, "%s: src range must be whole rows of %u",
                            kernel->name.c_str(), row);
            const uint32_t ntok = (uint32_t)(r0 / es / row);
            if (kernel->f16)
                return launch_kv_append_q8(st, static_cast<const uint16_t *>(p0),
                                           static_cast<uint16_t *>(p1), static_cast<int8_t *>(p2),
                                           static_cast<const uint32_t *>(p3), ntok, row,
                                           kernel->param);
            return launch_kv_append_q8(st, static_cast<const float *>(p0),
                                       static_cast<uint16_t *>(p1), static_cast<int8_t *>(p2),
                                       static_cast<const uint32_t *>(p3), ntok, row, kernel->param);
        }
        case Kind::GemmI8:
        case Kind::GemmI8Down:
        case Kind::GemmI8Split: {
            // bindings: 0 weights, 1 xq, 2 x_scales, 3 y (+4 partials for split-K);
            // groups [M/64, N/16] (swizzled, M_TILES=4) — M from groups.
            if ((rc = B.get(0, &p0, &r0)) || (rc = B.get(1, &p1, &r1)) || (rc = B.get(2, &p2, &r2)) ||
                (rc = B.get(3, &p3, &r3)))
                return rc;
            const uint32_t m = groups[0] * 64;
            const uint32_t n = kernel->n, k = kernel->k;
            if (kernel->kind == Kind::GemmI8Down && groups[1] != n / 16)
                return fail(SGQ_ERR_VALIDATION, "%s: groups.y must be %u", kernel->name.c_str(), n / 16);
            if (r1 && r1 < (uint64_t)m * k)
                return fail(SGQ_ERR_VALIDATION, "%s: x binding too small for M=%u", kernel->name.c_str(), m);
            if (r3 && r3 < (uint64_t)m * n * (kernel->f16 ? 2 : 4))
                return fail(SGQ_ERR_VALIDATION, "%s: y binding too small", kernel->name.c_str());
            if (kernel->f16)
                return launch_gemm_q4_0_q8(st, p0, static_cast<const int8_t *>(p1),
                                           static_cast<const uint16_t *>(p2),
                                           static_cast<uint16_t *>(p3), m, n, k);
            uint32_t split = 1;
            float *partials = nullptr;
            if (kernel->kind == Kind::GemmI8Split) {
                split = kernel->param;
                if (split > 1) {
                    if ((rc = B.get(4, &p4, &r4))) return rc;
                    partials = static_cast<float *>(p4);
                }
            }
            return launch_gemm_q4_0_q8(st, p0, static_cast<const int8_t *>(p1),
                                       static_cast<const uint16_t *>(p2), static_cast<float *>(p3),
                                       m, n, k, split, partials);
        }
        case Kind::AppendVQ8: {
            if ((rc = B.get(0, &p0, &r0)) || (rc = B.get(1, &p1, &r1)) || (rc = B.get(2, &p2, &r2)) ||
                (rc = B.get(3, &p3, &r3)))
                return rc;
            // row = groups.y·32 when groups.y > 1, else 2048; src must hold
            // whole rows; quants cover the appended rows and scales their
            // 32-key blocks (from pos = step[0], a multiple of 32)
            const uint32_t row = groups[1] > 1 ? groups[1] * 32 : 2048;
            const uint64_t es = kernel->f16 ? 2 : 4;
            if (!r0 || r0 % (row * es))
                return fail(SGQ_ERR_VALIDATION, "%s: src range must be whole rows of %u",
                            kernel->name.c_str(), row);
            const uint32_t ntok = (uint32_t)(r0 / es / row);
            if ((r1 && r1 < (uint64_t)(ntok + 31) / 32 * row * 2) || (r2 && r2 < (uint64_t)ntok * row))
                return fail(SGQ_ERR_VALIDATION, "%s: scales/quants binding too small for %u rows",
                            kernel->name.c_str(), ntok);
            if (kernel->f16)
                return launch_kv_append_v_q8(st, static_cast<const uint16_t *>(p0),
                                             static_cast<uint16_t *>(p1), static_cast<int8_t *>(p2),
                                             static_cast<const uint32_t *>(p3), 0, ntok, row);
            return launch_kv_append_v_q8(st, static_cast<const float *>(p0),
                                         static_cast<uint16_t *>(p1), static_cast<int8_t *>(p2),
                                         static_cast<const uint32_t *>(p3), 0, ntok, row);
        }
        case Kind::AttnPrefillIpv: {
            void *pp[7];
            uint64_t rr[7];
            for (uint32_t i = 0; i < 7; i++)
                if ((rc = B.get(i, &pp[i], &rr[i]))) return rc;
            const uint32_t nq = kernel->k, nkv = kernel->n;
            if (!rr[5])
                return fail(SGQ_ERR_VALIDATION, "%s: out range required (it gives M)",
                            kernel->name.c_str());
            const uint64_t m = rr[5] / ((uint64_t)nq * 128 * 4);
            if (m == 0 || m >= (1u << 30) || rr[5] != m * nq * 128 * 4)
                return fail(SGQ_ERR_VALIDATION, "%s: out range is not a whole number of tokens",
                            kernel->name.c_str());
            if (groups[0] != nq || groups[1] != (m + 15) / 16 || groups[2] != 1)
                return fail(SGQ_ERR_VALIDATION, "%s: groups must be [%u, %llu, 1]",
                            kernel->name.c_str(), nq, (unsigned long long)((m + 15) / 16));
            if ((rr[0] && rr[0] < m * nq * 128 * 4) || (rr[6] && rr[6] < 16))
                return fail(SGQ_ERR_VALIDATION, "%s: binding too small", kernel->name.c_str());
            float scale;
            std::memcpy(&scale, push, 4);
            return launch_attn_prefill_ipv(
                st, static_cast<const float *>(pp[0]), static_cast<const int8_t *>(pp[1]),
                static_cast<const uint16_t *>(pp[2]), static_cast<const int8_t *>(pp[3]),
                static_cast<const uint16_t *>(pp[4]), static_cast<float *>(pp[5]), (int)m, 0,
                (int)nq, (int)nkv, 128, scale, static_cast<const uint32_t *>(pp[6]));
        }
        case Kind::AttnDecode: {
            void *p5, *p6;
            uint64_t r5, r6;
            if ((rc = B.get(0, &p0, &r0)) || (rc = B.get(1, &p1, &r1)) || (rc = B.get(2, &p2, &r2)) ||
                (rc = B.get(3, &p3, &r3)) || (rc = B.get(4, &p4, &r4)) || (rc = B.get(5, &p5, &r5)) ||
                (rc = B.get(6, &p6, &r6)))
                return rc;
            uint32_t n_splits;
            float scale;
            std::memcpy(&n_splits, push, 4);
            std::memcpy(&scale, static_cast<const uint8_t *>(push) + 4, 4);
            const uint32_t nq = kernel->k, nkv = kernel->n;
            if (groups[0] != nkv || groups[1] != n_splits || groups[2] != 1)
                return fail(SGQ_ERR_VALIDATION, "%s: groups must be [%u, n_splits=%u, 1]",
                            kernel->name.c_str(), nkv, n_splits);
            if (r0 && r0 < (uint64_t)nq * 128 * 4)
                return fail(SGQ_ERR_VALIDATION, "%s: q binding too small", kernel->name.c_str());
            if (r5 && r5 < (uint64_t)nq * n_splits * 130 * 4)
                return fail(SGQ_ERR_VALIDATION, "%s: part binding too small", kernel->name.c_str());
            if (r6 && r6 < 16)
                return fail(SGQ_ERR_VALIDATION, "%s: step binding too small", kernel->name.c_str());
            return launch_attn_decode_parts(
                st, static_cast<const float *>(p0), static_cast<const int8_t *>(p1),
                static_cast<const uint16_t *>(p2), static_cast<const int8_t *>(p3),
                static_cast<const uint16_t *>(p4), static_cast<const uint32_t *>(p6),
                (int)kernel->param, (int)nq, (int)nkv, (int)n_splits, scale, static_cast<float *>(p5));
        }
        case Kind::AttnReduce: {
            if ((rc = B.get(0, &p0, &r0)) || (rc = B.get(1, &p1, &r1))) return rc;
            uint32_t n_splits;
            std::memcpy(&n_splits, push, 4);
            const uint32_t nq = kernel->k;
            if (groups[0] != nq || groups[1] != 1 || groups[2] != 1)
                return fail(SGQ_ERR_VALIDATION, "%s: groups must be [%u, 1, 1]",
                            kernel->name.c_str(), nq);
            if ((r0 && r0 < (uint64_t)nq * n_splits * 130 * 4) || (r1 && r1 < (uint64_t)nq * 128 * 4))
                return fail(SGQ_ERR_VALIDATION, "%s: binding too small", kernel->name.c_str());
            return launch_attn_reduce(st, static_cast<const float *>(p0), (int)nq, (int)kernel->n,
                                      (int)n_splits, static_cast<float *>(p1));
        }
        case Kind::AttnDecodePages: {
            const bool q8k = kernel->param & 4;
            const uint32_t nb = kernel->info.bindings;
            void *pp[6];
            uint64_t rr[6];
            for (uint32_t i = 0; i < nb; i++)
                if ((rc = B.get(i, &pp[i], &rr[i]))) return rc;
            uint32_t n_splits;
            float scale;
            std::memcpy(&n_splits, push, 4);
            std::memcpy(&scale, static_cast<const uint8_t *>(push) + 4, 4);
            const uint32_t hd = kernel->k, nkv = kernel->n;
            if (n_splits == 0 || groups[0] != nkv || groups[1] != n_splits || groups[2] != 1)
                return fail(SGQ_ERR_VALIDATION, "%s: groups must be [%u, n_splits=%u, 1]",
                            kernel->name.c_str(), nkv, n_splits);
            const uint32_t part_b = nb - 2, step_b = nb - 1;
            if (rr[0] && rr[0] < (uint64_t)kRealNQ * hd * 2)
                return fail(SGQ_ERR_VALIDATION, "%s: q binding too small", kernel->name.c_str());
            if (rr[part_b] && rr[part_b] < (uint64_t)kRealNQ * n_splits * (hd + 2) * 4)
                return fail(SGQ_ERR_VALIDATION, "%s: part binding too small", kernel->name.c_str());
            if (rr[step_b] && rr[step_b] < 12)
                return fail(SGQ_ERR_VALIDATION, "%s: step binding too small", kernel->name.c_str());
            return launch_attn_decode_pages(
                st, static_cast<const uint16_t *>(pp[0]), pp[1],
                q8k ? static_cast<const uint16_t *>(pp[2]) : nullptr,
                static_cast<const uint16_t *>(pp[q8k ? 3 : 2]), static_cast<float *>(pp[part_b]),
                static_cast<const uint32_t *>(pp[step_b]), (int)(kernel->param & 3), (int)hd,
                (int)kRealNQ, (int)nkv, (int)n_splits, scale);
        }
        case Kind::AttnReducePages: {
            if ((rc = B.get(0, &p0, &r0)) || (rc = B.get(1, &p1, &r1))) return rc;
            uint32_t n_splits;
            std::memcpy(&n_splits, push, 4);
            const uint32_t hd = kernel->k;
            if (n_splits == 0 || n_splits > 65535 || groups[0] != kRealNQ || groups[1] != 1 ||
                groups[2] != 1)
                return fail(SGQ_ERR_VALIDATION,
                            "%s: groups must be [%u, 1, 1], 0 < n_splits <= 65535",
                            kernel->name.c_str(), kRealNQ);
            if ((r0 && r0 < (uint64_t)kRealNQ * n_splits * (hd + 2) * 4) ||
                (r1 && r1 < (uint64_t)kRealNQ * hd * 2))
                return fail(SGQ_ERR_VALIDATION, "%s: binding too small", kernel->name.c_str());
            return launch_attn_reduce_pages(st, static_cast<const float *>(p0), (int)kRealNQ,
                                            (int)hd, (int)n_splits, static_cast<uint16_t *>(p1));
        }
        case Kind::AppendF16: {
            if ((rc = B.get(0, &p0, &r0)) || (rc = B.get(1, &p1, &r1)) || (rc = B.get(2, &p2, &r2)))
                return rc;
            const uint32_t row = kernel->k;
            if (!r0 || r0 % ((uint64_t)row * 2))
                return fail(SGQ_ERR_VALIDATION, "%s: src range must be whole rows of %u halves",
                            kernel->name.c_str(), row);
            const uint64_t n_tok = r0 / ((uint64_t)row * 2);
            if ((uint64_t)groups[0] * groups[1] * groups[2] * 256 < n_tok * row)
                return fail(SGQ_ERR_VALIDATION, "%s: groups cover fewer than %llu elements",
                            kernel->name.c_str(), (unsigned long long)(n_tok * row));
            if (kernel->param && n_tok > kernel->param)
                return fail(SGQ_ERR_VALIDATION, "%s: %llu rows exceed the %u-slot ring",
                            kernel->name.c_str(), (unsigned long long)n_tok, kernel->param);
            if ((r1 && r1 < (uint64_t)(kernel->param ? kernel->param : n_tok) * row * 2) ||
                (r2 && r2 < 4))
                return fail(SGQ_ERR_VALIDATION, "%s: binding too small", kernel->name.c_str());
            return launch_kv_append_f16(st, static_cast<const uint16_t *>(p0),
                                        static_cast<uint16_t *>(p1),
                                        static_cast<const uint32_t *>(p2), (uint32_t)n_tok, row,
                                        kernel->param);
        }
        case Kind::AttnPrefillPages: {
            const PrefillVariant &pv = kPrefill[kernel->param];
            void *pp[8];
            uint64_t rr[8];
            for (uint32_t i = 0; i < pv.bindings; i++)
                if ((rc = B.get(i, &pp[i], &rr[i]))) return rc;
            const uint32_t hd = pv.head_dim, nkv = pv.n_kv, nb = pv.bindings;
            const uint32_t gx = pv.per_token ? nkv : kRealNQ;
            if (groups[0] != gx || groups[1] == 0 || groups[2] != 1)
                return fail(SGQ_ERR_VALIDATION, "%s: groups must be [%u, %s, 1]",
                            kernel->name.c_str(), gx, pv.per_token ? "M" : "M/16");
            const uint64_t m = pv.per_token ? groups[1] : 16ull * groups[1];
            if (m >= (1u << 24))
                return fail(SGQ_ERR_VALIDATION, "%s: M %llu too large", kernel->name.c_str(),
                            (unsigned long long)m);
            const uint64_t row = (uint64_t)kRealNQ * hd;  // q / out elements per query
            const bool iq = pv.fmt == 3 || pv.fmt == 4, ring = pv.ring != 0;
            if ((rr[nb - 2] && rr[nb - 2] < m * row * 2) || (rr[nb - 1] && rr[nb - 1] < 16) ||
                (rr[0] && rr[0] < m * row * (iq ? 1 : 2)) ||
                (iq && rr[1] && rr[1] < m * row / 32 * 2))
                return fail(SGQ_ERR_VALIDATION, "%s: binding too small for M=%llu",
                            kernel->name.c_str(), (unsigned long long)m);
            const uint64_t kv_row = (uint64_t)nkv * hd * 2;
            if (ring && ((rr[1] && rr[1] < pv.ring * kv_row) || (rr[2] && rr[2] < pv.ring * kv_row) ||
                         (rr[3] && rr[3] < m * kv_row) || (rr[4] && rr[4] < m * kv_row)))
                return fail(SGQ_ERR_VALIDATION, "%s: ring or chunk pages too small",
                            kernel->name.c_str());
            float scale;
            std::memcpy(&scale, push, 4);
            const void *q = pp[0], *k, *v, *ck = nullptr, *cv = nullptr;
            const uint16_t *qs = nullptr, *ks = nullptr, *vs = nullptr;
            if (iq) {
                qs = static_cast<const uint16_t *>(pp[1]);
                k = pp[2], ks = static_cast<const uint16_t *>(pp[3]), v = pp[4];
                if (pv.fmt == 4) vs = static_cast<const uint16_t *>(pp[5]);
            } else if (pv.fmt == 1) {
                k = pp[1], ks = static_cast<const uint16_t *>(pp[2]);
                v = pp[3], vs = static_cast<const uint16_t *>(pp[4]);
            } else {
                k = pp[1], v = pp[2];
                if (ring) ck = pp[3], cv = pp[4];
            }
            return launch_attn_prefill_pages(st, (int)pv.fmt, q, qs, k, ks, v, vs, (int)pv.ring, ck, cv,
                                             nullptr, nullptr, pp[nb - 2], (int)m,
                                             static_cast<const uint32_t *>(pp[nb - 1]), (int)kRealNQ,
                                             (int)nkv, (int)hd, (int)pv.window, scale);
        }
        case Kind::AttnPrefill: {
            const bool ring = kernel->param != 0;
            void *pp[11];
            uint64_t rr[11];
            for (uint32_t i = 0; i < kernel->info.bindings; i++)
                if ((rc = B.get(i, &pp[i], &rr[i]))) return rc;
            const uint32_t out_b = ring ? 9 : 5, step_b = ring ? 10 : 6;
            const uint32_t nq = kernel->k, nkv = kernel->n;
            if (!rr[out_b])
                return fail(SGQ_ERR_VALIDATION, "%s: out range required (it gives M)",
                            kernel->name.c_str());
            const uint64_t m = rr[out_b] / ((uint64_t)nq * 128 * 4);
            if (m == 0 || m >= (1u << 30) || rr[out_b] != m * nq * 128 * 4)
                return fail(SGQ_ERR_VALIDATION, "%s: out range is not a whole number of tokens",
                            kernel->name.c_str());
            const uint64_t gy = ring ? m : (m + 15) / 16;
            if (groups[0] != (ring ? nkv : nq) || groups[1] != gy || groups[2] != 1)
                return fail(SGQ_ERR_VALIDATION, "%s: groups must be [%u, %llu, 1]",
                            kernel->name.c_str(), ring ? nkv : nq, (unsigned long long)gy);
            if (rr[0] && rr[0] < m * nq * 128 * 4)
                return fail(SGQ_ERR_VALIDATION, "%s: q binding too small", kernel->name.c_str());
            if (ring && ((rr[5] && rr[5] < m * nkv * 128) || (rr[7] && rr[7] < m * nkv * 128)))
                return fail(SGQ_ERR_VALIDATION, "%s: chunk pages too small", kernel->name.c_str());
            if (rr[step_b] && rr[step_b] < 16)
                return fail(SGQ_ERR_VALIDATION, "%s: step binding too small", kernel->name.c_str());
            float scale;
            std::memcpy(&scale, push, 4);
            return launch_attn_prefill_q8(
                st, static_cast<const float *>(pp[0]), static_cast<const int8_t *>(pp[1]),
                static_cast<const uint16_t *>(pp[2]), static_cast<const int8_t *>(pp[3]),
                static_cast<const uint16_t *>(pp[4]), static_cast<float *>(pp[out_b]), (int)m, 0,
                (int)nq, (int)nkv, 128, ring ? (int)kAttnWindow : 0, scale,
                ring ? (int)kernel->param : 0, ring ? static_cast<const int8_t *>(pp[5]) : nullptr,
                ring ? static_cast<const uint16_t *>(pp[6]) : nullptr,
                ring ? static_cast<const int8_t *>(pp[7]) : nullptr,
                ring ? static_cast<const uint16_t *>(pp[8]) : nullptr,
                static_cast<const uint32_t *>(pp[step_b]));
        }
    }
    return fail(SGQ_ERR_LIBRARY, "unhandled kernel kind");
}

int sgq_graph_begin(sgq_ctx *ctx) {
    if (!ctx) return fail(SGQ_ERR_VALIDATION, "ctx is NULL");
    if (!ctx->stream) SGQ_HIP(hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking));
    SGQ_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    ctx->capturing = true;
    return SGQ_OK;
}

int sgq_graph_end(sgq_ctx *ctx, sgq_graph **out) {
    if (!ctx || !out) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    if (!ctx->capturing) return fail(SGQ_ERR_VALIDATION, "no capture in progress");
    auto *g = new sgq_graph;
    ctx->capturing = false;
    hipError_t e = hipStreamEndCapture(ctx->stream, &g->graph);
    if (e != hipSuccess) {
        delete g;
        return check_hip(e, "hipStreamEndCapture");
    }
    e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(g->graph);
        delete g;
        return check_hip(e, "hipGraphInstantiate");
    }
    *out = g;
    return SGQ_OK;
}

int sgq_graph_submit(sgq_ctx *ctx, sgq_graph *graph) {
    if (!ctx || !graph) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    SGQ_HIP(hipGraphLaunch(graph->exec, ctx->stream));
    return SGQ_OK;
}

int sgq_graph_destroy(sgq_graph *graph) {
    if (!graph) return SGQ_OK;
    if (graph->exec) (void)hipGraphExecDestroy(graph->exec);
    if (graph->graph) (void)hipGraphDestroy(graph->graph);
    delete graph;
    return SGQ_OK;
}

}  // extern "C"

namespace {
__global__ void step_write_kernel(uint32_t *step, uint32_t a, uint32_t b, uint32_t c,
                                  uint32_t d) {
    const uint32_t t = threadIdx.x;
    if (t < 4) step[t] = t == 0 ? a : t == 1 ? b : t == 2 ? c : d;
}
}  // namespace

extern "C" {

int sgq_step_write(sgq_ctx *ctx, void *step_dev, uint32_t pos, uint32_t kv_len_sliding,
                   uint32_t kv_len_global, uint32_t q0) {
    if (!ctx || !step_dev) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    hipLaunchKernelGGL(step_write_kernel, dim3(1), dim3(64), 0, ctx->stream,
                       static_cast<uint32_t *>(step_dev), pos, kv_len_sliding, kv_len_global, q0);
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}

int sgq_timer_start(sgq_ctx *ctx) {
    if (!ctx) return fail(SGQ_ERR_VALIDATION, "ctx is NULL");
    SGQ_HIP(hipEventRecord(ctx->t0, ctx->stream));
    return SGQ_OK;
}

int sgq_timer_stop(sgq_ctx *ctx, float *ms) {
    if (!ctx || !ms) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    SGQ_HIP(hipEventRecord(ctx->t1, ctx->stream));
    SGQ_HIP(hipEventSynchronize(ctx->t1));
    SGQ_HIP(hipEventElapsedTime(ms, ctx->t0, ctx->t1));
    return SGQ_OK;
}

int sgq_gemv_q4_0(sgq_ctx *ctx, const void *w, const float *x, float *y, uint32_t n,
                  uint32_t k) {
    if (!ctx || !w || !x || !y) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    return launch_gemv_q4_0(ctx->stream, w, x, y, n, k, ctx->workspace);
}

int sgq_gemv_q6_k(sgq_ctx *ctx, const void *w, size_t row_stride, const float *x, float *y,
                  uint32_t n, uint32_t k, float softcap) {
    if (!ctx || !w || !x || !y) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    return launch_gemv_q6_k(ctx->stream, w, row_stride, x, y, n, k, softcap);
}

int sgq_x_limbs(sgq_ctx *ctx, const float *x, void *x_limbs, uint32_t k) {
    if (!ctx || !x || !x_limbs) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    return launch_quant_limbs(ctx->stream, x, x_limbs, k);
}

int sgq_gemv_q4_0_limbs(sgq_ctx *ctx, uint32_t n_targets, const void *const *w, float *const *y,
                        const uint32_t *rows, const void *x_limbs, uint32_t k, float softcap) {
    if (!ctx || !w || !y || !rows || !x_limbs) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    SGQ_CHECK(n_targets >= 1 && n_targets <= (uint32_t)kGemvMaxTargets,
              "gemv_q4_0_limbs: %u targets (1..%d)", n_targets, kGemvMaxTargets);
    SGQ_CHECK(softcap >= 0.f, "gemv_q4_0_limbs: negative softcap");
    GemvTargets tg{};
    uint64_t end = 0;
    for (uint32_t j = 0; j < n_targets; j++) {
        if (!w[j] || !y[j]) return fail(SGQ_ERR_VALIDATION, "NULL target %u", j);
        SGQ_CHECK(rows[j] > 0, "gemv_q4_0_limbs: target %u has no rows", j);
        end += rows[j];
        SGQ_CHECK(end < (1u << 31), "gemv_q4_0_limbs: too many rows");
        tg.w[j] = w[j];
        tg.y[j] = y[j];
        tg.end[j] = (int)end;
    }
    tg.count = (int)n_targets;
    tg.softcap = softcap;
    return launch_gemv_limbs(ctx->stream, tg, x_limbs, k);
}

int sgq_attn_prefill_q8(sgq_ctx *ctx, const float *q, const int8_t *k_quants,
                        const uint16_t *k_scales, const int8_t *v_quants, const uint16_t *v_scales,
                        uint32_t n_tokens, uint32_t q0, uint32_t n_q_heads, uint32_t n_kv_heads,
                        uint32_t head_dim, uint32_t window, float scale, float *out) {
    if (!ctx || !q || !k_quants || !k_scales || !v_quants || !v_scales || !out)
        return fail(SGQ_ERR_VALIDATION, "NULL argument");
    SGQ_CHECK(n_tokens < (1u << 30) && q0 < (1u << 30) && window < (1u << 30),
              "attn_prefill_q8: size out of range");
    return launch_attn_prefill_q8(ctx->stream, q, k_quants, k_scales, v_quants, v_scales, out,
                                  (int)n_tokens, (int)q0, (int)n_q_heads, (int)n_kv_heads,
                                  (int)head_dim, (int)window, scale);
}

int sgq_kv_append_v_q8(sgq_ctx *ctx, const float *src, uint32_t n_tokens, uint32_t row_len,
                       uint32_t pos, int8_t *v_quants, uint16_t *v_scales) {
    if (!ctx || (n_tokens && (!src || !v_quants || !v_scales)))
        return fail(SGQ_ERR_VALIDATION, "NULL argument");
    return launch_kv_append_v_q8(ctx->stream, src, v_scales, v_quants, nullptr, pos, n_tokens,
                                 row_len);
}

int sgq_attn_prefill_ipv(sgq_ctx *ctx, const float *q, const int8_t *k_quants,
                         const uint16_t *k_scales, const int8_t *v_quants,
                         const uint16_t *v_scales_kb, uint32_t n_tokens, uint32_t q0,
                         uint32_t n_q_heads, uint32_t n_kv_heads, uint32_t head_dim, float scale,
                         float *out) {
    if (!ctx || !q || !k_quants || !k_scales || !v_quants || !v_scales_kb || !out)
        return fail(SGQ_ERR_VALIDATION, "NULL argument");
    SGQ_CHECK(n_tokens < (1u << 30) && q0 < (1u << 30), "attn_prefill_ipv: size out of range");
    return launch_attn_prefill_ipv(ctx->stream, q, k_quants, k_scales, v_quants, v_scales_kb, out,
                                   (int)n_tokens, (int)q0, (int)n_q_heads, (int)n_kv_heads,
                                   (int)head_dim, scale, nullptr);
}

int sgq_rmsnorm(sgq_ctx *ctx, const float *x, const float *w, float *y, uint32_t rows,
                uint32_t row_len, int plus_one, float eps) {
    if (!ctx || !x || !y) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    return launch_rmsnorm(ctx->stream, x, w, y, rows, row_len, plus_one, eps);
}

int sgq_rope(sgq_ctx *ctx, float *x, const float *cos_sin, uint64_t n_tokens, uint32_t n_heads,
             uint32_t head_dim, uint32_t rot_dims) {
    if (!ctx || !x || !cos_sin) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    return launch_rope(ctx->stream, x, cos_sin, n_tokens * n_heads, head_dim, rot_dims, n_heads);
}

int sgq_geglu(sgq_ctx *ctx, const float *gate, const float *up, float *y, uint64_t n) {
    if (!ctx || !gate || !up || !y) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    return launch_geglu(ctx->stream, gate, up, y, n);
}

int sgq_add_scaled(sgq_ctx *ctx, const float *a, const float *b, float *y, uint64_t n, float s) {
    if (!ctx || !a || !b || !y) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    return launch_add_scaled(ctx->stream, a, b, y, n, s);
}

int sgq_quant_q8_0(sgq_ctx *ctx, const float *x, uint16_t *scales, int8_t *quants, uint64_t n) {
    if (!ctx || (n && (!x || !scales || !quants))) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    return launch_quant_q8_0(ctx->stream, x, scales, quants, n);
}

int sgq_dequant_q8_0(sgq_ctx *ctx, const uint16_t *scales, const int8_t *quants, float *out,
                     uint64_t n) {
    if (!ctx || (n && (!out || !scales || !quants))) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    return launch_dequant_q8_0(ctx->stream, scales, quants, out, n);
}

int sgq_gemm_q4_0_q8(sgq_ctx *ctx, const void *w, const int8_t *xq, const uint16_t *xs, float *y,
                     uint32_t m, uint32_t n, uint32_t k, uint32_t split_k, float *partials) {
    if (!ctx || !w || !xq || !xs || !y) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    return launch_gemm_q4_0_q8(ctx->stream, w, xq, xs, y, m, n, k, split_k, partials);
}

int sgq_attn_decode_q8(sgq_ctx *ctx, const float *q, const int8_t *k_quants,
                       const uint16_t *k_scales, const int8_t *v_quants, const uint16_t *v_scales,
                       uint32_t kv_len, uint32_t n_q_heads, uint32_t n_kv_heads,
                       uint32_t head_dim, uint32_t n_splits, float scale, float *out) {
    if (!ctx || !q || !k_quants || !k_scales || !v_quants || !v_scales || !out)
        return fail(SGQ_ERR_VALIDATION, "NULL argument");
    return launch_attn_decode_q8(ctx->stream, q, k_quants, k_scales, v_quants, v_scales, nullptr, 0,
                                 kv_len, (int)n_q_heads, (int)n_kv_heads, (int)head_dim,
                                 (int)n_splits, scale, out, ctx->workspace, kWorkspaceBytes);
}

int sgq_fill_q4_0_random(sgq_ctx *ctx, void *w, uint64_t n_blocks, uint64_t seed, float sigma) {
    if (!ctx || (n_blocks && !w)) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    return launch_fill_q4_0(ctx->stream, w, n_blocks, seed, sigma);
}

int sgq_fill_normal(sgq_ctx *ctx, float *x, uint64_t n, uint64_t seed, float mean, float sigma) {
    if (!ctx || (n && !x)) return fail(SGQ_ERR_VALIDATION, "NULL argument");
    return launch_fill_normal(ctx->stream, x, n, seed, mean, sigma);
}

}  // extern "C"
