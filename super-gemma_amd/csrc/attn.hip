// Q8_0-KV split-K decode attention kernels and launchers.  The split work
// item (attn_chunk, int8-MFMA QK) is in attn_mfma.h; the split merge
// (attn_merge) in attn_body.h.
#include "attn_mfma.h"

namespace sgq {
namespace {

// Workgroup order (a 1-D grid of n_splits·n_kv): workgroup i runs on XCD
// i % 8, and each XCD takes 4 kv heads of one split side by side, then the
// next split (split ≡ XCD mod 8), then the next 4 heads.  The f16 scale
// pages hold the 16 heads of a slot in one 128-byte line, so heads of the
// same slots that run at the same time on the same XCD share its fetch
// (128K: 946 -> 820 MB of HBM reads per launch against 570 MB
// algorithmic), while consecutive splits of a head keep the K/V rows
// streaming (side by side, 16 heads per split read the cache 4.7 against
// 5.7 TB/s in a read-only probe).  Measured: 128K 140.5 -> 135.0 us, 32K
// 40.2 -> 40.5 us, against consecutive splits of one head; all 16 heads
// side by side: 134.6 and 41.3 us.
__device__ __forceinline__ void attn_work_item(int n_kv, int n_splits, int *kvh, int *split) {
    constexpr int HG = 4;
    const int id = blockIdx.x;
    if (n_splits % 8 == 0 && n_kv % HG == 0) {
        const int x = id % 8, a = id / 8, S8 = n_splits / 8;
        const int t = a / HG;
        *split = (t % S8) * 8 + x;
        *kvh = (t / S8) * HG + a % HG;
    } else {
        *split = id % n_splits;
        *kvh = id / n_splits;
    }
}

template <int QPK, bool FUSED, int W>
__global__ __launch_bounds__(W * kWave) void attn_decode_q8_kernel(
    const float *__restrict__ q, const int8_t *__restrict__ kq, const uint16_t *__restrict__ ks,
    const int8_t *__restrict__ vq, const uint16_t *__restrict__ vs,
    const uint32_t *__restrict__ step, int step_word, uint32_t kv_len_direct, int n_kv,
    int n_splits, float scale, float *__restrict__ part, float *__restrict__ out,
    BlockLimbs *__restrict__ limbs_out, AttnPost post) {
    const uint32_t kv_len = step ? step[step_word] : kv_len_direct;
    int kvh, split;
    attn_work_item(n_kv, n_splits, &kvh, &split);
    attn_chunk<QPK, FUSED, W>(q, kq, ks, vq, vs, kv_len, n_kv, n_splits, scale, part, out,
                              limbs_out, post, kvh, split, FUSED ? step[0] : 0u);
}

// One wave per (kv head, split) work item (attn_split_per_wave): workgroup
// = the 4 adjacent kv heads 4g..4g+3 of one split, consecutive workgroups
// take consecutive splits of one group.  Partials only (n_splits >= 1).
// Used when that gives at least 4 waves per CU (n_splits·n_kv >= 1024,
// decided from host-side counts only, so that the typed call and the
// dispatch by name pick the same kernel): config 4 at 4K / 32K / 128K with
// 64 / 128 / 256 splits 11.2 / 34.4 / 117.4 us against 11.5 / 40.2 / 130.2
// for the four-waves-per-item kernel at its best split counts; with few
// splits (the decode step's 16) it leaves most of the GPU idle.  (The 4
// head groups of a split side by side on one XCD: 11.4 / 37.6 / 121.9 us.)
template <int QPK>
__global__ __launch_bounds__(4 * kWave) void attn_decode_q8_hw_kernel(
    const float *__restrict__ q, const int8_t *__restrict__ kq, const uint16_t *__restrict__ ks,
    const int8_t *__restrict__ vq, const uint16_t *__restrict__ vs,
    const uint32_t *__restrict__ step, int step_word, uint32_t kv_len_direct, int n_kv,
    int n_splits, float scale, float *__restrict__ part) {
    __shared__ __align__(16) int8_t ql_s[4][2][4][kHD];
    __shared__ float qn_s[4][2];
    __shared__ __align__(16) float pw_s[4][32 * 4 * 2];
    const int wave = threadIdx.x / kWave;
    const uint32_t kv_len = step ? step[step_word] : kv_len_direct;
    const int split = blockIdx.x % n_splits, kvh = (blockIdx.x / n_splits) * 4 + wave;
    attn_split_per_wave<QPK>(q, kq, ks, vq, vs, kv_len, n_kv, n_splits, scale, part, kvh, split,
                             ql_s[wave], qn_s[wave], pw_s[wave]);
}
constexpr int kAttnPerWaveMinWaves = 1024;
inline bool attn_per_wave(int n_kv, int n_splits) {
    return n_kv % 4 == 0 && n_splits * n_kv >= kAttnPerWaveMinWaves;
}

// Merge of the split partials (attn_reduce.wgsl:24-57): for query head h,
// out = Σ_s a_s·e^(m_s−M) / Σ_s l_s·e^(m_s−M), M = max_s m_s.  One
// workgroup per query head (attn_merge_head): 4 waves up to 64 splits, 16
// above, so that each wave's share of the rows is one batch of loads (the
// config-4 step at 128K with 256 splits: 117.8 -> 116.1 us).  The kernel
// boundary after the split kernel makes the partials visible.  Optionally
// writes the x limbs of the output rows for the next GEMV.
template <int NW>
__global__ __launch_bounds__(NW * 64) void attn_merge_kernel(const float *__restrict__ part,
                                                             int n_splits, float *__restrict__ out,
                                                             BlockLimbs *__restrict__ limbs_out) {
    __shared__ float merge_s[merge_smem(NW)];
    attn_merge_head<NW>(part, n_splits, blockIdx.x, out, limbs_out, merge_s);
}
constexpr int kMergeWideSplits = 64;  // above: 16-wave merge workgroups

// The same merge for up to 16 splits: one workgroup per kv head, thread
// (head, dim) loads all splits' (m, l, acc[dim]) in one batch and folds
// them in split order (attn_merge): a single round trip.
template <int QPK>
__global__ __launch_bounds__(QPK * kHD) void attn_merge_fold_kernel(
    const float *__restrict__ part, int n_splits, float *__restrict__ out,
    BlockLimbs *__restrict__ limbs_out) {
    __shared__ __align__(16) float o_s[QPK * kHD];
    attn_merge<QPK, false>(part, n_splits, blockIdx.x, out, limbs_out, o_s);
}

void launch_merge(hipStream_t st, int qpk, int n_q, int n_kv, int n_splits, const float *part,
                  float *out, BlockLimbs *lo) {
    if (n_splits > kMergeWideSplits)
        hipLaunchKernelGGL(attn_merge_kernel<16>, dim3(n_q), dim3(16 * 64), 0, st, part, n_splits,
                           out, lo);
    else if (n_splits > 16)
        hipLaunchKernelGGL(attn_merge_kernel<4>, dim3(n_q), dim3(4 * 64), 0, st, part, n_splits,
                           out, lo);
    else if (qpk == 1)
        hipLaunchKernelGGL(attn_merge_fold_kernel<1>, dim3(n_kv), dim3(kHD), 0, st, part, n_splits,
                           out, lo);
    else
        hipLaunchKernelGGL(attn_merge_fold_kernel<2>, dim3(n_kv), dim3(2 * kHD), 0, st, part,
                           n_splits, out, lo);
}

}  // namespace

int launch_attn_decode_q8(hipStream_t st, const float *q, const int8_t *kq, const uint16_t *ks,
                          const int8_t *vq, const uint16_t *vs, const uint32_t *step,
                          int step_word, uint32_t kv_len, int n_q, int n_kv, int head_dim,
                          int n_splits, float scale, float *out, void *workspace,
                          size_t workspace_bytes, void *limbs_out) {
    SGQ_CHECK(head_dim == kHD, "attn_decode_q8: head_dim %d unsupported (128)", head_dim);
    SGQ_CHECK(n_kv > 0 && n_q % n_kv == 0, "attn_decode_q8: n_q %% n_kv != 0");
    SGQ_CHECK(n_splits >= 1 && n_splits <= kMergeMaxSplits, "attn_decode_q8: n_splits %d out of range", n_splits);
    SGQ_CHECK(step != nullptr || kv_len > 0, "attn_decode_q8: kv_len must be > 0");
    SGQ_CHECK(((uintptr_t)kq & 15) == 0 && ((uintptr_t)vq & 3) == 0 && ((uintptr_t)ks & 7) == 0 &&
                  ((uintptr_t)vs & 7) == 0,
              "attn_decode_q8: misaligned cache");
    SGQ_CHECK(n_kv <= kAttnMaxKv, "attn_decode_q8: n_kv %d > %d", n_kv, kAttnMaxKv);
    const size_t part_bytes = (size_t)n_q * n_splits * (kHD + 2) * 4;
    SGQ_CHECK(kAttnPartOff + part_bytes <= workspace_bytes,
              "attn_decode_q8: workspace too small (%zu < %zu)", workspace_bytes,
              kAttnPartOff + part_bytes);
    float *part = reinterpret_cast<float *>(static_cast<uint8_t *>(workspace) + kAttnPartOff);
    const int qpk = n_q / n_kv;
    const dim3 grid(n_splits * n_kv);
    SGQ_CHECK(qpk == 1 || qpk == 2, "attn_decode_q8: %d q heads per kv head unsupported", qpk);
    BlockLimbs *lo = static_cast<BlockLimbs *>(limbs_out);
    if (attn_per_wave(n_kv, n_splits)) {
        const dim3 g4(n_splits * (n_kv / 4));
        if (qpk == 1)
            hipLaunchKernelGGL(attn_decode_q8_hw_kernel<1>, g4, dim3(4 * kWave), 0, st, q, kq, ks, vq,
                               vs, step, step_word, kv_len, n_kv, n_splits, scale, part);
        else
            hipLaunchKernelGGL(attn_decode_q8_hw_kernel<2>, g4, dim3(4 * kWave), 0, st, q, kq, ks, vq,
                               vs, step, step_word, kv_len, n_kv, n_splits, scale, part);
        SGQ_HIP(hipGetLastError());
        launch_merge(st, qpk, n_q, n_kv, n_splits, part, out, lo);
        SGQ_HIP(hipGetLastError());
        return SGQ_OK;
    }
    float *out1 = n_splits == 1 ? out : nullptr;
    BlockLimbs *lo1 = n_splits == 1 ? lo : nullptr;
#define SGQ_ATTN(Q, W)                                                                            \
    hipLaunchKernelGGL((attn_decode_q8_kernel<Q, false, W>), grid, dim3(W * kWave), 0, st, q, kq, \
                       ks, vq, vs, step, step_word, kv_len, n_kv, n_splits, scale, part, out1,    \
                       lo1, AttnPost{})
    if (qpk == 1) SGQ_ATTN(1, kAttnWaves);
    else SGQ_ATTN(2, kAttnWaves);
    SGQ_HIP(hipGetLastError());
    if (n_splits > 1) {
        launch_merge(st, qpk, n_q, n_kv, n_splits, part, out, lo);
    }
#undef SGQ_ATTN
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}

int launch_attn_decode_parts(hipStream_t st, const float *q, const int8_t *kq,
                             const uint16_t *ks, const int8_t *vq, const uint16_t *vs,
                             const uint32_t *step, int step_word, int n_q, int n_kv, int n_splits,
                             float scale, float *part) {
    SGQ_CHECK(step != nullptr && part != nullptr, "attn_decode (parts): step and part required");
    SGQ_CHECK(n_kv > 0 && n_q % n_kv == 0 && (n_q / n_kv == 1 || n_q / n_kv == 2),
              "attn_decode (parts): %d q heads over %d kv heads unsupported", n_q, n_kv);
    SGQ_CHECK(n_splits >= 1 && n_splits <= kMergeMaxSplits,
              "attn_decode (parts): n_splits %d out of range (1..%d)", n_splits, kMergeMaxSplits);
    SGQ_CHECK(((uintptr_t)kq & 15) == 0 && ((uintptr_t)vq & 3) == 0 && ((uintptr_t)ks & 7) == 0 &&
                  ((uintptr_t)vs & 7) == 0 && ((uintptr_t)part & 3) == 0,
              "attn_decode (parts): misaligned operand");
    if (attn_per_wave(n_kv, n_splits)) {
        const dim3 g4(n_splits * (n_kv / 4));
        if (n_q == n_kv)
            hipLaunchKernelGGL(attn_decode_q8_hw_kernel<1>, g4, dim3(4 * kWave), 0, st, q, kq, ks, vq,
                               vs, step, step_word, 0u, n_kv, n_splits, scale, part);
        else
            hipLaunchKernelGGL(attn_decode_q8_hw_kernel<2>, g4, dim3(4 * kWave), 0, st, q, kq, ks, vq,
                               vs, step, step_word, 0u, n_kv, n_splits, scale, part);
        SGQ_HIP(hipGetLastError());
        return SGQ_OK;
    }
    const dim3 grid(n_splits * n_kv);
    if (n_q == n_kv)
        hipLaunchKernelGGL((attn_decode_q8_kernel<1, false, kAttnWaves>), grid,
                           dim3(kAttnWaves * kWave), 0, st, q, kq, ks, vq, vs, step, step_word, 0u,
                           n_kv, n_splits, scale, part, nullptr, nullptr, AttnPost{});
    else
        hipLaunchKernelGGL((attn_decode_q8_kernel<2, false, kAttnWaves>), grid,
                           dim3(kAttnWaves * kWave), 0, st, q, kq, ks, vq, vs, step, step_word, 0u,
                           n_kv, n_splits, scale, part, nullptr, nullptr, AttnPost{});
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}

int launch_attn_reduce(hipStream_t st, const float *part, int n_q, int n_kv, int n_splits,
                       float *out) {
    SGQ_CHECK(part != nullptr && out != nullptr, "attn_reduce: NULL operand");
    SGQ_CHECK(n_kv > 0 && n_q % n_kv == 0 && (n_q / n_kv == 1 || n_q / n_kv == 2),
              "attn_reduce: %d q heads over %d kv heads unsupported", n_q, n_kv);
    SGQ_CHECK(n_splits >= 1 && n_splits <= kMergeMaxSplits,
              "attn_reduce: n_splits %d out of range (1..%d)", n_splits, kMergeMaxSplits);
    launch_merge(st, n_q / n_kv, n_q, n_kv, n_splits, part, out, nullptr);
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}

int attn_prepare() { return SGQ_OK; }  // all variants fit the default LDS limit

int launch_attn_decode_fused(hipStream_t st, const float *q_raw, const float *k_raw,
                             const float *v_src, const float *wq_norm, const float *wk_norm,
                             const float *rope_cs, float eps, const uint32_t *step, int step_word,
                             uint32_t ring, int8_t *kq, uint16_t *ks, int8_t *vq, uint16_t *vs,
                             int n_q, int n_kv, int n_splits, float scale, float *out,
                             void *workspace, size_t workspace_bytes, void *limbs_out) {
    SGQ_CHECK(step != nullptr, "attn (fused): needs the step buffer");
    SGQ_CHECK(n_kv > 0 && n_q % n_kv == 0, "attn (fused): n_q %% n_kv != 0");
    SGQ_CHECK(n_splits >= 1 && n_splits <= kMergeMaxSplits, "attn (fused): n_splits %d", n_splits);
    SGQ_CHECK(((uintptr_t)kq & 15) == 0 && ((uintptr_t)vq & 15) == 0 && ((uintptr_t)ks & 7) == 0 &&
                  ((uintptr_t)vs & 7) == 0,
              "attn (fused): misaligned cache");
    const size_t part_bytes = (size_t)n_q * n_splits * (kHD + 2) * 4;
    SGQ_CHECK(kAttnPartOff + part_bytes <= workspace_bytes, "attn (fused): workspace too small");
    float *part = reinterpret_cast<float *>(static_cast<uint8_t *>(workspace) + kAttnPartOff);
    const AttnPost post{q_raw, k_raw, v_src, wq_norm, wk_norm, rope_cs, eps, (int)ring,
                        kq, vq, ks, vs};
    if (int rc = attn_prepare()) return rc;
    const dim3 grid(n_splits * n_kv);
    const int qpk = n_q / n_kv;
    SGQ_CHECK(qpk == 1 || qpk == 2, "attn (fused): %d q heads per kv head unsupported", qpk);
    BlockLimbs *lo = static_cast<BlockLimbs *>(limbs_out);
    float *out1 = n_splits == 1 ? out : nullptr;
    BlockLimbs *lo1 = n_splits == 1 ? lo : nullptr;
#define SGQ_ATTN(Q, W)                                                                            \
    hipLaunchKernelGGL((attn_decode_q8_kernel<Q, true, W>), grid, dim3(W * kWave), 0, st, nullptr, \
                       kq, ks, vq, vs, step, step_word, 0u, n_kv, n_splits, scale, part, out1,    \
                       lo1, post)
    if (qpk == 1) SGQ_ATTN(1, kAttnWaves);
    else SGQ_ATTN(2, kAttnWaves);
    SGQ_HIP(hipGetLastError());
    if (n_splits > 1) {
        launch_merge(st, qpk, n_q, n_kv, n_splits, part, out, lo);
    }
#undef SGQ_ATTN
    SGQ_HIP(hipGetLastError());
    return SGQ_OK;
}

}  // namespace sgq
