"""numpy/ctypes front end of the CPU oracle (``libsgo.so`` built from sgo.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of bench.py, never by the product library.  Every
function here forwards to the C restatement in sgo.c, which cites the
reference file:line it follows.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libsgo.so")
_lib = None

P = C.c_void_p
U64 = C.c_uint64
SZ = C.c_size_t


def build() -> str:
    """Compile sgo.c into libsgo.so (gcc, a few seconds)."""
    subprocess.run(["make", "-s", "-C", _HERE, "-B", "libsgo.so"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        sigs = {
            "sgo_rng_next": (U64, [C.POINTER(U64)]),
            "sgo_rng_f32_vec": (U64, [U64, P, SZ]),
            "sgo_rng_u64_vec": (U64, [U64, P, SZ]),
            "sgo_f32_to_f16": (C.c_uint16, [C.c_float]),
            "sgo_f16_to_f32": (C.c_float, [C.c_uint16]),
            "sgo_f32_to_f16_vec": (None, [P, P, SZ]),
            "sgo_f16_to_f32_vec": (None, [P, P, SZ]),
            "sgo_through_f16": (None, [P, SZ]),
            "sgo_q4_0_dequant_block": (None, [P, P]),
            "sgo_q4_0_dequant_rows": (None, [P, SZ, SZ, P]),
            "sgo_random_q4_0": (U64, [U64, P, SZ]),
            "sgo_gemv_q4_0_rows": (None, [P, P, SZ, P, SZ, P]),
            "sgo_q6_k_dequant_block": (None, [P, P]),
            "sgo_q6_k_dequant_rows": (None, [P, SZ, SZ, SZ, P]),
            "sgo_random_q6_k_rows": (U64, [U64, P, SZ, SZ, SZ]),
            "sgo_gemv_q6_k_logits": (None, [P, SZ, P, SZ, SZ, C.c_double, P]),
            "sgo_dot_f64": (C.c_double, [P, P, SZ]),
            "sgo_matmul_q4_0": (None, [P, P, SZ, SZ, SZ, P, C.c_int]),
            "sgo_quant_q8_0": (None, [P, SZ, P, P]),
            "sgo_q8_quant_div": (None, [P, SZ, P, P, P]),
            "sgo_q8_quant_v": (None, [P, SZ, SZ, SZ, P, P, P]),
            "sgo_kv_append_v_q8": (None, [P, SZ, SZ, SZ, P, P]),
            "sgo_attention_head_ipv": (None, [P, P, P, SZ, SZ, SZ, SZ, SZ, C.c_double, SZ, SZ,
                                              P]),
            "sgo_dequant_q8_0_f16": (None, [P, P, SZ, P]),
            "sgo_dequant_q8_0": (None, [P, P, SZ, P]),
            "sgo_block_dot_q4_q8": (C.c_int32, [P, P]),
            "sgo_mmq_pairs": (None, [P, P, P, SZ, P, P, SZ, P]),
            "sgo_mmq_q4_0_q8": (None, [P, P, SZ, SZ, SZ, P]),
            "sgo_mmq_block_dots": (None, [P, P, SZ, SZ, SZ, P]),
            "sgo_rmsnorm": (None, [P, P, SZ, SZ, C.c_double, C.c_int, P]),
            "sgo_cos_sin_table": (None, [P, SZ, SZ, C.c_float, P, P]),
            "sgo_rope": (None, [P, SZ, SZ, SZ, SZ, P]),
            "sgo_apply_rope_f32": (None, [P, SZ, P]),
            "sgo_gelu_tanh": (C.c_float, [C.c_float]),
            "sgo_geglu": (None, [P, P, SZ, P]),
            "sgo_add_scaled": (None, [P, P, SZ, C.c_float, P]),
            "sgo_attention_head": (None, [P, P, P, SZ, SZ, SZ, SZ, SZ, C.c_double, SZ, SZ, P]),
            "sgo_attention": (None, [P, P, P, SZ, SZ, SZ, SZ, SZ, SZ, C.c_float, P]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(C.c_void_p)


# --- RNG (mod.rs:7-32) -------------------------------------------------------
class Rng:
    """xorshift64* with the reference's seed.max(1) rule."""

    def __init__(self, seed: int):
        self.state = max(int(seed), 1)

    def next_u64(self) -> int:
        s = U64(self.state)
        v = lib().sgo_rng_next(C.byref(s))
        self.state = s.value
        return v

    def f32_vec(self, n: int) -> np.ndarray:
        out = np.empty(n, np.float32)
        self.state = lib().sgo_rng_f32_vec(self.state, _p(out), n)
        return out

    def u64_vec(self, n: int) -> np.ndarray:
        out = np.empty(n, np.uint64)
        self.state = lib().sgo_rng_u64_vec(self.state, _p(out), n)
        return out

    def random_q6_k_rows(self, n_rows: int, k: int, row_stride: int) -> np.ndarray:
        """parity_logits.rs:31-51 rows in a padded layout (row_stride bytes)."""
        out = np.empty(n_rows * row_stride, np.uint8)
        self.state = lib().sgo_random_q6_k_rows(self.state, _p(out), n_rows, k, row_stride)
        return out

    def random_q4_0(self, n_blocks: int) -> np.ndarray:
        out = np.empty(n_blocks * 18, np.uint8)
        self.state = lib().sgo_random_q4_0(self.state, _p(out), n_blocks)
        return out


# --- f16 ---------------------------------------------------------------------
def f32_to_f16_bits(x) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().sgo_f32_to_f16_vec(_p(x), _p(out), x.size)
    return out


def f16_bits_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().sgo_f16_to_f32_vec(_p(h), _p(out), h.size)
    return out


def through_f16(x) -> np.ndarray:
    out = np.array(x, np.float32, copy=True, order="C")
    lib().sgo_through_f16(_p(out), out.size)
    return out


# --- Q4_0 --------------------------------------------------------------------
def q4_0_dequant(w: np.ndarray, n_rows: int, k: int) -> np.ndarray:
    w = np.ascontiguousarray(w, np.uint8)
    assert w.size == n_rows * k // 32 * 18
    out = np.empty((n_rows, k), np.float32)
    lib().sgo_q4_0_dequant_rows(_p(w), n_rows, k, _p(out))
    return out


def q6_k_dequant(w: np.ndarray, n_rows: int, k: int, row_stride: int | None = None) -> np.ndarray:
    """q6_k.rs:41-62 over rows of k/256 blocks at row_stride bytes."""
    row_stride = row_stride or (k // 256) * 210
    w = np.ascontiguousarray(w, np.uint8)
    out = np.empty((n_rows, k), np.float32)
    lib().sgo_q6_k_dequant_rows(_p(w), row_stride, n_rows, k, _p(out))
    return out


def gemv_q6_k_logits(w: np.ndarray, row_stride: int, x, n: int, k: int,
                     softcap: float = 30.0) -> np.ndarray:
    """parity_logits.rs:84-98: f64 dot per row, softcap*tanh(dot/softcap)."""
    w = np.ascontiguousarray(w, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(n, np.float32)
    lib().sgo_gemv_q6_k_logits(_p(w), row_stride, _p(x), n, k, float(softcap), _p(y))
    return y


def gemv_rows(w: np.ndarray, x: np.ndarray, k: int, rows) -> np.ndarray:
    w = np.ascontiguousarray(w, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    rows = np.ascontiguousarray(rows, np.int64)
    out = np.empty(rows.size, np.float32)
    lib().sgo_gemv_q4_0_rows(_p(w), _p(x), k, _p(rows), rows.size, _p(out))
    return out


def matmul_q4_0(w: np.ndarray, x: np.ndarray, n_tokens: int, n_out: int, n_in: int,
                threads: int = 1) -> np.ndarray:
    w = np.ascontiguousarray(w, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty((n_tokens, n_out), np.float32)
    lib().sgo_matmul_q4_0(_p(w), _p(x), n_tokens, n_out, n_in, _p(y), threads)
    return y


def dot_f64(a, b) -> float:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return lib().sgo_dot_f64(_p(a), _p(b), a.size)


# --- Q8_0 --------------------------------------------------------------------
def quant_q8_0(x) -> tuple[np.ndarray, np.ndarray]:
    """(f16 scale bits [n/32], int8 quants [n]) — mod.rs:272-286."""
    x = np.ascontiguousarray(x, np.float32)
    n = x.size
    s = np.empty(n // 32, np.uint16)
    q = np.empty(n, np.int8)
    lib().sgo_quant_q8_0(_p(x), n, _p(s), _p(q))
    return s.reshape(x.shape[:-1] + (x.shape[-1] // 32,)), q.reshape(x.shape)


def q8_quant_div(x):
    x = np.ascontiguousarray(x, np.float32)
    n = x.size
    s = np.empty(n // 32, np.uint16)
    q = np.empty(n, np.int8)
    d = np.empty(n, np.float32)
    lib().sgo_q8_quant_div(_p(x), n, _p(s), _p(q), _p(d))
    return s, q, d


def q8_quant_v(v, keys, n_kv_heads, head_dim):
    v = np.ascontiguousarray(v, np.float32)
    kblk = (keys + 31) // 32
    q = np.empty(v.size, np.int8)
    s = np.empty(kblk * n_kv_heads * head_dim, np.uint16)
    d = np.empty(v.size, np.float32)
    lib().sgo_q8_quant_v(_p(v), keys, n_kv_heads, head_dim, _p(q), _p(s), _p(d))
    return q, s, d


def kv_append_v_q8(src, n_tok, row, pos, quants, scales):
    """kv_append_global_v_q8.wgsl:32-75 into (quants int8 [slots*row],
    scales uint16 [slot_blocks*row]), in place."""
    src = np.ascontiguousarray(src, np.float32)
    assert quants.flags["C_CONTIGUOUS"] and scales.flags["C_CONTIGUOUS"]
    assert quants.dtype == np.int8 and scales.dtype == np.uint16
    assert quants.size >= (pos + n_tok) * row and scales.size >= ((pos + n_tok + 31) // 32) * row
    lib().sgo_kv_append_v_q8(_p(src), n_tok, row, pos, _p(quants), _p(scales))


def dequant_v_keyblocked(quants, scales, keys, row):
    """Dequantize key-blocked V: x[t, c] = f16 scale[t//32, c] * q[t, c]."""
    q = np.asarray(quants, np.int8)[:keys * row].reshape(keys, row).astype(np.float32)
    s = f16_bits_to_f32(np.asarray(scales, np.uint16)[:((keys + 31) // 32) * row]).reshape(-1, row)
    return (q * s[np.arange(keys) // 32]).astype(np.float32).reshape(-1)


def dequant_q8_0(scales, quants) -> np.ndarray:
    scales = np.ascontiguousarray(scales, np.uint16)
    quants = np.ascontiguousarray(quants, np.int8)
    out = np.empty(quants.shape, np.float32)
    lib().sgo_dequant_q8_0(_p(scales), _p(quants), quants.size, _p(out))
    return out


def dequant_q8_0_f16(scales, quants) -> np.ndarray:
    scales = np.ascontiguousarray(scales, np.uint16)
    quants = np.ascontiguousarray(quants, np.int8)
    out = np.empty(quants.shape, np.float32)
    lib().sgo_dequant_q8_0_f16(_p(scales), _p(quants), quants.size, _p(out))
    return out


# --- MMQ ---------------------------------------------------------------------
def block_dot(wblk, xq) -> int:
    wblk = np.ascontiguousarray(wblk, np.uint8)
    xq = np.ascontiguousarray(xq, np.int8)
    return lib().sgo_block_dot_q4_q8(_p(wblk), _p(xq))


def mmq_pairs(w, xq, xs, k, ms, ns) -> np.ndarray:
    w = np.ascontiguousarray(w, np.uint8)
    xq = np.ascontiguousarray(xq, np.int8)
    xs = np.ascontiguousarray(xs, np.uint16)
    ms = np.ascontiguousarray(ms, np.int64)
    ns = np.ascontiguousarray(ns, np.int64)
    out = np.empty(ms.size, np.float32)
    lib().sgo_mmq_pairs(_p(w), _p(xq), _p(xs), k, _p(ms), _p(ns), ms.size, _p(out))
    return out


def mmq_q4_0_q8(w, x, m, k, n) -> np.ndarray:
    w = np.ascontiguousarray(w, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty((m, n), np.float32)
    lib().sgo_mmq_q4_0_q8(_p(w), _p(x), m, k, n, _p(out))
    return out


def mmq_block_dots(w, xq, k, mi, ni) -> np.ndarray:
    w = np.ascontiguousarray(w, np.uint8)
    xq = np.ascontiguousarray(xq, np.int8)
    out = np.empty(k // 32, np.int32)
    lib().sgo_mmq_block_dots(_p(w), _p(xq), k, mi, ni, _p(out))
    return out


# --- elementwise -------------------------------------------------------------
def rmsnorm(x, w, row_len, eps=1e-6, plus_one=False) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.float32)
    if w is None:
        wp = None
    else:
        w = np.ascontiguousarray(w, np.float32)
        wp = _p(w)
    lib().sgo_rmsnorm(_p(x), wp, x.size // row_len, row_len, eps, int(plus_one), _p(out))
    return out


def cos_sin_table(positions, head_dim, theta, factors=None) -> np.ndarray:
    pos = np.ascontiguousarray(positions, np.uint32)
    out = np.empty((pos.size, head_dim // 2, 2), np.float32)
    if factors is None:
        fp = None
    else:
        factors = np.ascontiguousarray(factors, np.float32)
        fp = _p(factors)
    lib().sgo_cos_sin_table(_p(pos), pos.size, head_dim, theta, fp, _p(out))
    return out


def rope(x, head_dim, rot_dims, n_heads, cos_sin) -> np.ndarray:
    out = np.array(x, np.float32, copy=True, order="C")
    cs = np.ascontiguousarray(cos_sin, np.float32)
    lib().sgo_rope(_p(out), out.size // head_dim, head_dim, rot_dims, n_heads, _p(cs))
    return out


def apply_rope_f32(row, cs) -> np.ndarray:
    out = np.array(row, np.float32, copy=True, order="C")
    cs = np.ascontiguousarray(cs, np.float32)
    lib().sgo_apply_rope_f32(_p(out), out.size, _p(cs))
    return out


def gelu_tanh(x: float) -> float:
    return lib().sgo_gelu_tanh(x)


def geglu(g, u) -> np.ndarray:
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    out = np.empty(g.shape, np.float32)
    lib().sgo_geglu(_p(g), _p(u), g.size, _p(out))
    return out


def add_scaled(a, b, s) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    out = np.empty(a.shape, np.float32)
    lib().sgo_add_scaled(_p(a), _p(b), a.size, s, _p(out))
    return out


# --- attention ---------------------------------------------------------------
def attention_head(q, k, v, i, qh, n_q_heads, n_kv_heads, head_dim, scale, t0, t1):
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    out = np.empty(head_dim, np.float32)
    lib().sgo_attention_head(_p(q), _p(k), _p(v), i, qh, n_q_heads, n_kv_heads, head_dim,
                             scale, t0, t1, _p(out))
    return out


def attention_head_ipv(q, k, v, i, qh, n_q_heads, n_kv_heads, head_dim, scale, t0, t1):
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    out = np.empty(head_dim, np.float32)
    lib().sgo_attention_head_ipv(_p(q), _p(k), _p(v), i, qh, n_q_heads, n_kv_heads, head_dim,
                                 scale, t0, t1, _p(out))
    return out


def attention(q, ck, cv, n, q0, n_q_heads, n_kv, hd, window, scale) -> np.ndarray:
    q = np.ascontiguousarray(q, np.float32)
    ck = np.ascontiguousarray(ck, np.float32)
    cv = np.ascontiguousarray(cv, np.float32)
    out = np.empty((n, n_q_heads, hd), np.float32)
    lib().sgo_attention(_p(q), _p(ck), _p(cv), n, q0, n_q_heads, n_kv, hd, window or 0,
                        scale, _p(out))
    return out
