"""Write reference_kats.json: the known-answer vectors held by the reference's
own unit tests for this path, transcribed as data (inputs and expected
outputs), each with the file:line it comes from.

The reference is Rust and cannot be built here (no rustc/cargo), so these
vectors are what its tests assert, copied as numbers; the oracle and the HIP
kernels are checked against them in tests/test_oracle.py and the GPU tests.

Run:  python tests/golden/make_reference_kats.py
"""
import json
import math
import os

HERE = os.path.dirname(os.path.abspath(__file__))

kats = {
    # crates/sg-gguf/src/q4_0.rs:79-96 dequantize_known_block
    "q4_0_known_block": {
        "src": "crates/sg-gguf/src/q4_0.rs:79-96",
        "d": 2.0,
        "qs": [0x39] + [0x88] * 15,
        "expect": {"0": 2.0, "16": -10.0, "others": 0.0},
    },
    # crates/sg-gguf/src/q4_0.rs:98-110 dequantize_extremes
    "q4_0_extremes": {
        "src": "crates/sg-gguf/src/q4_0.rs:98-110",
        "d": 1.5,
        "qs": [0xF0] * 16,
        "expect": {"0": -12.0, "16": 10.5},
    },
    # crates/sg-gguf/src/q4_0.rs:112-118 blocks_from_bytes_validates_length
    "q4_0_block_bytes": {"src": "crates/sg-gguf/src/q4_0.rs:72-76,112-118", "block_bytes": 18},
    # crates/sg-model/src/reference.rs:561-570 gelu_tanh_reference_values
    "gelu_tanh": {
        "src": "crates/sg-model/src/reference.rs:561-570",
        "abs_tol": 1e-6,
        "points": [[0.0, 0.0], [1.0, 0.841192], [-2.0, -0.0454023]],
        "exact": [[20.0, 20.0], [-20.0, -0.0]],
    },
    # crates/sg-model/src/reference.rs:572-586 softmax_attention_uniform_when_keys_equal
    "attention_uniform": {
        "src": "crates/sg-model/src/reference.rs:572-586",
        "n_q_heads": 4, "n_kv": 2, "hd": 2, "kv_len": 3, "q0": 2,
        "ck": [1.0] * 12,
        "cv": [float(i) for i in range(12)],
        "q": [1.0] * 8,
        "expect": [[0, 4.0], [4, 6.0]],  # (flat output index, value)
        "abs_tol": 1e-6,
    },
    # crates/sg-model/src/reference.rs:588-596 sliding_window_masks_old_keys
    "attention_window": {
        "src": "crates/sg-model/src/reference.rs:588-596",
        "n_q_heads": 1, "n_kv": 1, "hd": 1, "q0": 2, "window": 2,
        "ck": [1.0, 1.0, 1.0], "cv": [10.0, 20.0, 30.0], "q": [1.0],
        "expect": [[0, 25.0]],
        "abs_tol": 1e-6,
    },
    # crates/sg-model/src/rope.rs:70-79 pos_zero_is_identity
    "rope_pos_zero": {"src": "crates/sg-model/src/rope.rs:70-79", "pos": 0, "head_dim": 256,
                      "theta": 10000.0},
    # crates/sg-model/src/rope.rs:81-87 first_pair_rotates_by_pos_radians
    "rope_first_pair": {"src": "crates/sg-model/src/rope.rs:81-87", "pos": 3, "head_dim": 256,
                        "theta": 10000.0,
                        "expect_cos0": float(math.cos(3.0)), "expect_sin0": float(math.sin(3.0))},
    # crates/sg-model/src/rope.rs:89-104 proportional_factors_freeze_tail_pairs
    "rope_proportional": {
        "src": "crates/sg-model/src/rope.rs:89-104",
        "pos": 100000, "head_dim": 512, "theta": 1000000.0,
        "factors": {"live": 64, "live_value": 1.0, "frozen_value": 1e30, "frozen": 192},
        "expect_cos0": float(math.cos(100000.0)),
        "pair63_angle": 100000.0 * (1e6 ** (-2.0 * 63.0 / 512.0)),
    },
    # crates/sg-model/src/rope.rs:106-113 apply_rope_neox_pairing
    "rope_neox_pairing": {
        "src": "crates/sg-model/src/rope.rs:106-113",
        "cs": [0.0, 1.0, 1.0, 0.0], "row": [1.0, 5.0, 2.0, 7.0],
        "expect": [-2.0, 5.0, 1.0, 7.0],
    },
    # crates/sg-gpu/tests/parity_kv.rs:131-144 — an all-zero block quantizes to
    # d = 0 and q = 0 (the id = 0 path).
    "q8_zero_block": {"src": "crates/sg-gpu/tests/parity_kv.rs:138-144", "d_bits": 0, "q": 0},
    # crates/sg-gpu/tests/coop_i8_smoke.rs: the 16x16x16 int8 tile with
    # a[i][k] = (i+k)%7-3 and b[k][j] = (k*j)%11-5 (inputs; the expected C is
    # their integer product, which the test computes the same way).
    "coop_i8_tile": {"src": "crates/sg-gpu/tests/coop_i8_smoke.rs", "m": 16, "n": 16, "k": 16},
    # crates/sg-gguf/src/q6_k.rs:92-124 dequantize_known_block: a block with
    # ql = 0, qh = 0, scales = 1, d = 0.5 dequantizes to -16 everywhere; then
    # edits of single bytes set weights 0 and 96 (weight 64 is unchanged).
    "q6_k_known_block": {
        "src": "crates/sg-gguf/src/q6_k.rs:92-124",
        "d": 0.5, "scales": [1] * 16,
        "all_zero_expect": -16.0,
        "steps": [
            {"set": {"ql": [[0, 0x0F]], "qh": [[0, 0x03]], "scales": [[0, 2]]},
             "expect": [[0, 31.0], [64, -16.0]]},
            {"set": {"ql": [[32, 0xA0]], "qh_or": [[0, 0xC0]], "scales": [[6, -3]]},
             "expect": [[96, -39.0]]},
        ],
    },
    # crates/sg-gguf/src/q6_k.rs:126-138 negative_scales_and_signed_range
    "q6_k_negative_scales": {"src": "crates/sg-gguf/src/q6_k.rs:126-138", "d": 1.0,
                             "ql": 0xFF, "qh": 0xFF, "scale": -128, "expect_all": -3968.0},
    # crates/sg-gguf/src/q6_k.rs:25-38, 86-90: 210-byte blocks of 256 weights;
    # crates/sg-gpu/build.rs:322-327 rows padded 4410 -> 4416 bytes (ROW_WORDS 1104)
    "q6_k_block_bytes": {"src": "crates/sg-gguf/src/q6_k.rs:25-38,86-90; crates/sg-gpu/build.rs:322-327",
                         "block_bytes": 210, "block_weights": 256, "row_bytes_k5376": 4410,
                         "row_stride_k5376": 4416},
}

if __name__ == "__main__":
    out = os.path.join(HERE, "reference_kats.json")
    with open(out, "w") as f:
        json.dump(kats, f, indent=1, sort_keys=True)
    print("wrote", out)
