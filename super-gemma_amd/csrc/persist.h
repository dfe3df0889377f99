// Parameters of the persistent decode kernel (persist.hip), built by the
// model driver (model.hip).
#pragma once
#include "sgq_internal.h"

namespace sgq {

// One decoder layer's tensors (device pointers), as the kernel reads them.
struct PLayer {
    const void *wq, *wk, *wv, *wo, *wg, *wu, *wd;  // Q4_0; wv null: V from K
    const float *attn_norm, *q_norm, *k_norm, *post_attn_norm, *ffn_norm, *post_ffw_norm;
    const float *out_scale;
    int8_t *kq, *vq;
    uint16_t *ks, *vs;
    uint32_t slots;
    int global;
};

// Byte offsets of one layer's activation region in the arena (each region
// is written once per launch; region n_layers holds the head's input).
struct PArena {
    size_t stride;
    size_t x, xl_attn, ss_attn;  // residual in, its norm's limbs, block Σx²
    size_t qkv, part, xl_o;      // raw q|k|v, attention partials, o limbs
    size_t y, xm, xl_ffn, ss_ffn;  // O output, post-attention residual, FFN norm
    size_t h, xl_h, d;           // GeGLU output, its limbs, down output
};

// Sync words: [0] global barrier count, [16 (1 + g)] group counts g < 8,
// [kSyncMergeOff + layer·n_kv + kv head] attention merge counts.
constexpr int kSyncMergeOff = 256;

struct PParams {
    const PLayer *layers;
    int n_layers;
    const uint8_t *embd;
    const float *out_norm;
    int H, F, QD, KD, n_kv, vocab;
    int s_h, slice_h, s_q, slice_q, s_f, slice_f;  // GEMV K-slices for K = H, QD, F
    int n_splits;                                  // attention splits per kv head
    float eps, attn_scale, softcap, embed_scale;
    const uint32_t *step;  // [pos, kv_len_sliding, kv_len_global, q0, token]
    const float *rope_cs;  // [2 kinds][64][cos, sin]
    float *logits;
    unsigned *sync;
    int *err;
    uint8_t *arena;
    PArena ar;
};

int persist_lds_bytes();
int persist_prepare(int qpk);
int launch_decode_persistent(hipStream_t st, const PParams &p, int qpk, int grid);

}  // namespace sgq
