"""sgq — Python host mirror of super-gemma's sg-gpu dispatch surface over libsgq.

The reference host API (crates/sg-gpu/src/lib.rs:20-44) is::

    ctx = GpuContext::new()?;                    // NoDevice → tests skip
    let k = ctx.load_kernel("gemv_q4_0_k5376")?; // UnknownKernel on a bad name
    ctx.dispatch_blocking(&k, vec![BufferBinding::buffer(0, w), ...], push, groups)?;

This module exposes the same calls (``GpuContext``, ``load_kernel``,
``dispatch``, ``dispatch_blocking``, ``BufferBinding``, ``StepState``,
``GraphRecorder``) with torch device tensors as buffers, plus the typed entry
points of include/sgq.h.  Everything goes through the C ABI of
``libsgq.so`` via ctypes; there is no Python or CPU fallback: if the library
or a gfx950 device is missing, calls raise.

torch is imported first so that libsgq binds to the HIP runtime torch
already loaded (one runtime per process).
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass
from typing import Optional, Sequence

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
# SGQ_LIB_PATH names another build of the same library (e.g. an A/B variant);
# by default the in-tree libsgq.so next to this file.
LIB_PATH = os.environ.get("SGQ_LIB_PATH") or os.path.join(_HERE, "libsgq.so")

SGQ_OK = 0
ERRORS = {
    1: "Library",
    2: "Hip",
    3: "NoDevice",
    4: "UnknownKernel",
    5: "Pipeline",
    6: "Validation",
}


class GpuError(RuntimeError):
    """Mirrors sg_gpu::GpuError (crates/sg-gpu/src/lib.rs:31-44)."""

    def __init__(self, code: int, msg: str):
        self.code = code
        self.kind = ERRORS.get(code, f"code{code}")
        super().__init__(f"{self.kind}: {msg}")


class NoDevice(GpuError):
    pass


class UnknownKernel(GpuError):
    pass


class ValidationError(GpuError):
    pass


_lib = None


class _Info(C.Structure):
    _fields_ = [("workgroup", C.c_uint32 * 3), ("bindings", C.c_uint32),
                ("push_bytes", C.c_uint32), ("subgroup_size", C.c_uint32)]


class _Binding(C.Structure):
    _fields_ = [("binding", C.c_uint32), ("_pad", C.c_uint32), ("ptr", C.c_void_p),
                ("offset", C.c_uint64), ("range", C.c_uint64)]


class ModelConfig(C.Structure):
    """sgq_model_config (include/sgq.h)."""
    _fields_ = [(n, C.c_uint32) for n in (
        "n_layers", "hidden", "ffn", "n_q_heads", "n_kv_heads", "head_dim", "vocab",
        "sliding_window", "global_every", "max_ctx")] + [(n, C.c_float) for n in (
        "rope_theta_sliding", "rope_theta_global", "global_rope_frac", "eps", "attn_scale",
        "final_softcap", "weight_sigma")] + [("global_k_eq_v", C.c_uint32),
                                             ("prefill_chunk", C.c_uint32), ("seed", C.c_uint64)] + [
        (n, C.c_uint32) for n in ("head_dim_global", "n_kv_heads_global", "embed_q6k",
                                  "reserved")]

    def as_dict(self):
        return {n: getattr(self, n) for n, _ in self._fields_}


class _GgufTensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("type", C.c_uint32), ("n_dims", C.c_uint32),
                ("dims", C.c_uint64 * 4), ("offset", C.c_uint64), ("bytes", C.c_uint64),
                ("data", C.c_void_p)]


# Exported symbols and their ctypes signatures (checked against include/sgq.h
# by tests/test_abi.py).
P, U32, U64, I = C.c_void_p, C.c_uint32, C.c_uint64, C.c_int
SIGNATURES = {
    "sgq_last_error": (C.c_char_p, []),
    "sgq_version": (C.c_char_p, []),
    "sgq_ctx_create": (I, [I, C.POINTER(P)]),
    "sgq_ctx_destroy": (I, [P]),
    "sgq_ctx_set_stream": (I, [P, P]),
    "sgq_sync": (I, [P]),
    "sgq_buf_alloc": (I, [P, U64, C.POINTER(P)]),
    "sgq_buf_free": (I, [P, P]),
    "sgq_buf_upload": (I, [P, P, P, U64]),
    "sgq_buf_download": (I, [P, P, P, U64]),
    "sgq_buf_fill_zero": (I, [P, P, U64]),
    "sgq_gemv_q4_0_noalloc": (I, [P, P, P, P, U32, U32]),
    "sgq_kv_append_v_q8": (I, [P, P, U32, U32, U32, P, P]),
    "sgq_attn_prefill_ipv": (I, [P, P, P, P, P, P, U32, U32, U32, U32, U32, C.c_float, P]),
    "sgq_kernel_lookup": (I, [P, C.c_char_p, C.POINTER(P), C.POINTER(_Info)]),
    "sgq_kernel_count": (U32, []),
    "sgq_kernel_name": (C.c_char_p, [U32]),
    "sgq_dispatch": (I, [P, P, C.POINTER(_Binding), U32, P, U32, C.POINTER(U32)]),
    "sgq_graph_begin": (I, [P]),
    "sgq_graph_end": (I, [P, C.POINTER(P)]),
    "sgq_graph_submit": (I, [P, P]),
    "sgq_graph_destroy": (I, [P]),
    "sgq_step_write": (I, [P, P, U32, U32, U32, U32]),
    "sgq_timer_start": (I, [P]),
    "sgq_timer_stop": (I, [P, C.POINTER(C.c_float)]),
    "sgq_gemv_q4_0": (I, [P, P, P, P, U32, U32]),
    "sgq_gemv_q6_k": (I, [P, P, C.c_size_t, P, P, U32, U32, C.c_float]),
    "sgq_x_limbs": (I, [P, P, P, U32]),
    "sgq_gemv_q4_0_limbs": (I, [P, U32, C.POINTER(P), C.POINTER(P), C.POINTER(U32), P, U32,
                                C.c_float]),
    "sgq_attn_prefill_q8": (I, [P, P, P, P, P, P, U32, U32, U32, U32, U32, U32, C.c_float, P]),
    "sgq_rmsnorm": (I, [P, P, P, P, U32, U32, I, C.c_float]),
    "sgq_rope": (I, [P, P, P, U64, U32, U32, U32]),
    "sgq_geglu": (I, [P, P, P, P, U64]),
    "sgq_add_scaled": (I, [P, P, P, P, U64, C.c_float]),
    "sgq_quant_q8_0": (I, [P, P, P, P, U64]),
    "sgq_dequant_q8_0": (I, [P, P, P, P, U64]),
    "sgq_gemm_q4_0_q8": (I, [P, P, P, P, P, U32, U32, U32, U32, P]),
    "sgq_attn_decode_q8": (I, [P, P, P, P, P, P, U32, U32, U32, U32, U32, C.c_float, P]),
    "sgq_model_default_config": (None, [C.POINTER(ModelConfig)]),
    "sgq_model_create": (I, [P, C.POINTER(ModelConfig), C.POINTER(P)]),
    "sgq_model_destroy": (I, [P]),
    "sgq_model_reset": (I, [P]),
    "sgq_model_position": (U32, [P]),
    "sgq_model_decode": (I, [P, U32, P]),
    "sgq_model_decode_graph": (I, [P, U32, P]),
    "sgq_model_set_decode_mode": (I, [P, I]),
    "sgq_model_decode_mode": (I, [P]),
    "sgq_model_status": (I, [P]),
    "sgq_model_fill_cache": (I, [P, U32, U64]),
    "sgq_model_prefill": (I, [P, C.POINTER(U32), U32, P]),
    "sgq_model_tensor": (I, [P, I, C.c_char_p, C.POINTER(P), C.POINTER(U64)]),
    "sgq_gguf_open": (I, [C.c_char_p, C.POINTER(P)]),
    "sgq_gguf_close": (I, [P]),
    "sgq_gguf_tensor_count": (U64, [P]),
    "sgq_gguf_tensor_at": (I, [P, U64, C.POINTER(_GgufTensor)]),
    "sgq_gguf_tensor_find": (I, [P, C.c_char_p, C.POINTER(_GgufTensor)]),
    "sgq_gguf_meta_int": (I, [P, C.c_char_p, C.POINTER(C.c_int64)]),
    "sgq_gguf_meta_float": (I, [P, C.c_char_p, C.POINTER(C.c_double)]),
    "sgq_gguf_meta_string": (I, [P, C.c_char_p, C.POINTER(C.c_char_p)]),
    "sgq_model_load_gguf": (I, [P, P]),
    "sgq_fill_q4_0_random": (I, [P, P, U64, U64, C.c_float]),
    "sgq_fill_normal": (I, [P, P, U64, U64, C.c_float, C.c_float]),
}


def lib():
    """Load libsgq.so (built by super-gemma_amd/build.py); raises if absent."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise GpuError(1, f"{LIB_PATH} is not built (run __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _check(rc: int):
    if rc != SGQ_OK:
        msg = lib().sgq_last_error().decode(errors="replace")
        cls = {3: NoDevice, 4: UnknownKernel, 6: ValidationError}.get(rc, GpuError)
        raise cls(rc, msg)


def _ptr(t: Optional[torch.Tensor]):
    if t is None:
        return None
    if not t.is_cuda:
        raise ValidationError(6, "buffers must be device tensors")
    if not t.is_contiguous():
        raise ValidationError(6, "buffers must be contiguous")
    return C.c_void_p(t.data_ptr())


def _nbytes(t: torch.Tensor) -> int:
    return t.numel() * t.element_size()


@dataclass
class Kernel:
    """A looked-up variant: KernelBlob's name/workgroup/bindings/push_bytes."""
    name: str
    handle: C.c_void_p
    workgroup: tuple
    bindings: int
    push_bytes: int

    def groups_for(self, n: int):
        """Kernel::groups_for (crates/sg-gpu/src/kernel.rs:56-58)."""
        return [(n + self.workgroup[0] - 1) // self.workgroup[0], 1, 1]


@dataclass
class BufferBinding:
    """BufferBinding{binding, buffer, offset, range} over a torch tensor."""
    binding: int
    buffer: torch.Tensor
    offset: int = 0
    range: Optional[int] = None

    @staticmethod
    def buffer(binding: int, t: torch.Tensor) -> "BufferBinding":
        return BufferBinding(binding, t)


@dataclass
class StepState:
    """StepState (crates/sg-gpu/src/graph.rs:33-61)."""
    pos: int = 0
    kv_len_sliding: int = 0
    kv_len_global: int = 0
    q0: int = 0


class GpuContext:
    """GpuContext over one gfx950 device; work goes on torch's current stream."""

    def __init__(self, device: int = 0):
        if not torch.cuda.is_available():
            raise NoDevice(3, "no HIP device visible to torch")
        h = C.c_void_p()
        _check(lib().sgq_ctx_create(device, C.byref(h)))
        self._h = h
        self.device = device
        self.set_stream(torch.cuda.current_stream(device))

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and _lib is not None:
            _lib.sgq_ctx_destroy(h)
            self._h = None

    @property
    def handle(self):
        return self._h

    def set_stream(self, stream: Optional[torch.cuda.Stream]):
        """Enqueue on a torch stream from now on (None: the null stream)."""
        h = None if stream is None else stream.cuda_stream
        _check(lib().sgq_ctx_set_stream(self._h, C.c_void_p(h)))

    def synchronize(self):
        _check(lib().sgq_sync(self._h))

    # -- kernel registry / dispatch (the reference's name-based surface) --
    def load_kernel(self, name: str) -> Kernel:
        h = C.c_void_p()
        info = _Info()
        _check(lib().sgq_kernel_lookup(self._h, name.encode(), C.byref(h), C.byref(info)))
        return Kernel(name, h, tuple(info.workgroup), info.bindings, info.push_bytes)

    def dispatch(self, kernel: Kernel, bindings: Sequence[BufferBinding], push: Optional[bytes],
                 groups: Sequence[int]):
        arr = (_Binding * max(1, len(bindings)))()
        keep = []
        for i, b in enumerate(bindings):
            nbytes = _nbytes(b.buffer)
            rng = b.range if b.range is not None else nbytes - b.offset
            if b.offset + rng > nbytes:
                raise ValidationError(6, f"binding {b.binding}: range past the end of the buffer")
            arr[i] = _Binding(b.binding, 0, _ptr(b.buffer), b.offset, rng)
            keep.append(b.buffer)
        pb = push or b""
        pbuf = C.create_string_buffer(pb, len(pb)) if pb else None
        g = (C.c_uint32 * 3)(*[int(v) for v in groups])
        _check(lib().sgq_dispatch(self._h, kernel.handle, arr, len(bindings),
                                  C.cast(pbuf, C.c_void_p) if pbuf else None, len(pb), g))

    def dispatch_blocking(self, kernel, bindings, push, groups):
        """crates/sg-gpu/src/exec.rs:9-23: record one dispatch, submit, wait."""
        self.dispatch(kernel, bindings, push, groups)
        self.synchronize()

    def step_write(self, step_buf: torch.Tensor, s: StepState):
        _check(lib().sgq_step_write(self._h, _ptr(step_buf), s.pos, s.kv_len_sliding,
                                    s.kv_len_global, s.q0))

    # -- typed entry points -------------------------------------------------
    def gemv_q4_0(self, w: torch.Tensor, x: torch.Tensor, y: torch.Tensor, n: int, k: int):
        _need(w, torch.uint8, n * (k // 32) * 18, "w")
        _need(x, torch.float32, k, "x")
        _need(y, torch.float32, n, "y")
        _check(lib().sgq_gemv_q4_0(self._h, _ptr(w), _ptr(x), _ptr(y), n, k))

    def gemv_q6_k(self, w: torch.Tensor, row_stride: int, x: torch.Tensor, y: torch.Tensor,
                  n: int, k: int, softcap: float = 30.0):
        """Q6_K logits GEMV (gemv_q6_k_logits.wgsl): y = softcap·tanh(E·x/softcap)."""
        _need(w, torch.uint8, n * row_stride, "w")
        _need(x, torch.float32, k, "x")
        _need(y, torch.float32, n, "y")
        _check(lib().sgq_gemv_q6_k(self._h, _ptr(w), row_stride, _ptr(x), _ptr(y), n, k,
                                   float(softcap)))

    X_LIMBS_BYTES_PER_BLOCK = 80

    def x_limbs(self, x: torch.Tensor, xl: torch.Tensor, k: int):
        """x [k] fp32 -> its limb table (k/32 × 80 bytes, uint8 tensor)."""
        _need(x, torch.float32, k, "x")
        _need(xl, torch.uint8, k // 32 * self.X_LIMBS_BYTES_PER_BLOCK, "x_limbs")
        _check(lib().sgq_x_limbs(self._h, _ptr(x), _ptr(xl), k))

    def gemv_q4_0_limbs(self, ws, ys, rows, xl: torch.Tensor, k: int, softcap: float = 0.0):
        """One launch over up to 4 matrices sharing x: ys[j][:rows[j]] = ws[j]·x."""
        n = len(ws)
        if not (len(ys) == len(rows) == n):
            raise ValidationError(6, "ws, ys and rows differ in length")
        for w, y, r in zip(ws, ys, rows):
            _need(w, torch.uint8, r * (k // 32) * 18, "w")
            _need(y, torch.float32, r, "y")
        _need(xl, torch.uint8, k // 32 * self.X_LIMBS_BYTES_PER_BLOCK, "x_limbs")
        wp = (P * n)(*[_ptr(w) for w in ws])
        yp = (P * n)(*[_ptr(y) for y in ys])
        rp = (U32 * n)(*rows)
        _check(lib().sgq_gemv_q4_0_limbs(self._h, n, wp, yp, rp, _ptr(xl), k, softcap))

    def quant_q8_0(self, x: torch.Tensor, scales: torch.Tensor, quants: torch.Tensor):
        n = x.numel()
        _need(x, torch.float32, n, "x")
        _need(scales, (torch.uint16, torch.int16, torch.float16), n // 32, "scales")
        _need(quants, torch.int8, n, "quants")
        _check(lib().sgq_quant_q8_0(self._h, _ptr(x), _ptr(scales), _ptr(quants), n))

    def dequant_q8_0(self, scales, quants, out):
        n = quants.numel()
        _need(out, torch.float32, n, "out")
        _need(scales, (torch.uint16, torch.int16, torch.float16), n // 32, "scales")
        _check(lib().sgq_dequant_q8_0(self._h, _ptr(scales), _ptr(quants), _ptr(out), n))

    def gemm_q4_0_q8(self, w, xq, xs, y, m, n, k, split_k=1, partials=None):
        _need(w, torch.uint8, n * (k // 32) * 18, "w")
        _need(xq, torch.int8, m * k, "xq")
        _need(xs, (torch.uint16, torch.int16, torch.float16), m * (k // 32), "xs")
        _need(y, torch.float32, m * n, "y")
        if split_k > 1:
            _need(partials, torch.float32, split_k * m * n, "partials")
        elif partials is not None:  # optional: lets the last part-filled round split over K
            _need(partials, torch.float32, m * n, "partials")
        _check(lib().sgq_gemm_q4_0_q8(self._h, _ptr(w), _ptr(xq), _ptr(xs), _ptr(y), m, n, k,
                                      split_k, _ptr(partials)))

    def attn_decode_q8(self, q, kq, ks, vq, vs, kv_len, n_q, n_kv, out, n_splits=16,
                       scale=None, head_dim=128):
        """Split-K decode attention over a Q8_0 K/V cache (fp32 q/out)."""
        _need(q, torch.float32, n_q * head_dim, "q")
        _need(out, torch.float32, n_q * head_dim, "out")
        _need(kq, torch.int8, kv_len * n_kv * head_dim, "k_quants")
        _need(vq, torch.int8, kv_len * n_kv * head_dim, "v_quants")
        _need(ks, (torch.uint16, torch.int16, torch.float16), kv_len * n_kv * head_dim // 32, "k_scales")
        _need(vs, (torch.uint16, torch.int16, torch.float16), kv_len * n_kv * head_dim // 32, "v_scales")
        if scale is None:
            scale = 1.0 / head_dim ** 0.5
        _check(lib().sgq_attn_decode_q8(self._h, _ptr(q), _ptr(kq), _ptr(ks), _ptr(vq), _ptr(vs),
                                        kv_len, n_q, n_kv, head_dim, n_splits, scale, _ptr(out)))

    def kv_append_v_q8(self, src, n_tok, row, pos, vq, vs):
        """Key-blocked V append (sgq_kv_append_v_q8)."""
        _need(src, torch.float32, n_tok * row, "src")
        _need(vq, torch.int8, (pos + n_tok) * row, "v_quants")
        _need(vs, (torch.uint16, torch.int16, torch.float16), ((pos + n_tok + 31) // 32) * row,
              "v_scales")
        _check(lib().sgq_kv_append_v_q8(self._h, _ptr(src), n_tok, row, pos, _ptr(vq), _ptr(vs)))

    def attn_prefill_ipv(self, q, kq, ks, vq, vs_kb, n_tok, q0, n_q, n_kv, out, scale=None,
                         head_dim=128):
        """Causal prefill attention with int8 PV over a linear cache of
        positions 0..q0+n_tok-1 (V scales key-blocked)."""
        n_slots = q0 + n_tok
        _need(q, torch.float32, n_tok * n_q * head_dim, "q")
        _need(out, torch.float32, n_tok * n_q * head_dim, "out")
        _need(kq, torch.int8, n_slots * n_kv * head_dim, "k_quants")
        _need(vq, torch.int8, n_slots * n_kv * head_dim, "v_quants")
        _need(vs_kb, (torch.uint16, torch.int16, torch.float16),
              ((n_slots + 31) // 32) * n_kv * head_dim, "v_scales")
        sc = 1.0 / head_dim ** 0.5 if scale is None else scale
        _check(lib().sgq_attn_prefill_ipv(self._h, _ptr(q), _ptr(kq), _ptr(ks), _ptr(vq),
                                          _ptr(vs_kb), n_tok, q0, n_q, n_kv, head_dim, sc,
                                          _ptr(out)))

    def attn_prefill_q8(self, q, kq, ks, vq, vs, n_tok, q0, n_q, n_kv, out, window=0,
                        scale=None, head_dim=128):
        """Prefill attention for positions q0..q0+n_tok-1 over a linear Q8_0
        cache holding positions 0..q0+n_tok-1."""
        n_slots = q0 + n_tok
        _need(q, torch.float32, n_tok * n_q * head_dim, "q")
        _need(out, torch.float32, n_tok * n_q * head_dim, "out")
        _need(kq, torch.int8, n_slots * n_kv * head_dim, "k_quants")
        _need(vq, torch.int8, n_slots * n_kv * head_dim, "v_quants")
        _need(ks, (torch.uint16, torch.int16, torch.float16), n_slots * n_kv * head_dim // 32, "k_scales")
        _need(vs, (torch.uint16, torch.int16, torch.float16), n_slots * n_kv * head_dim // 32, "v_scales")
        if scale is None:
            scale = 1.0 / head_dim ** 0.5
        _check(lib().sgq_attn_prefill_q8(self._h, _ptr(q), _ptr(kq), _ptr(ks), _ptr(vq), _ptr(vs),
                                         n_tok, q0, n_q, n_kv, head_dim, window, scale, _ptr(out)))

    def rmsnorm(self, x, w, y, rows, row_len, plus_one=False, eps=1e-6):
        _need(x, torch.float32, rows * row_len, "x")
        _need(y, torch.float32, rows * row_len, "y")
        if w is not None:
            _need(w, torch.float32, row_len, "w")
        _check(lib().sgq_rmsnorm(self._h, _ptr(x), _ptr(w), _ptr(y), rows, row_len,
                                 int(plus_one), eps))

    def rope(self, x, cos_sin, n_tokens, n_heads, head_dim, rot_dims):
        _need(x, torch.float32, n_tokens * n_heads * head_dim, "x")
        _need(cos_sin, torch.float32, n_tokens * rot_dims, "cos_sin")
        _check(lib().sgq_rope(self._h, _ptr(x), _ptr(cos_sin), n_tokens, n_heads, head_dim,
                              rot_dims))

    def geglu(self, g, u, y):
        n = y.numel()
        _need(g, torch.float32, n, "gate")
        _need(u, torch.float32, n, "up")
        _check(lib().sgq_geglu(self._h, _ptr(g), _ptr(u), _ptr(y), n))

    def add_scaled(self, a, b, y, s):
        n = y.numel()
        _need(a, torch.float32, n, "a")
        _need(b, torch.float32, n, "b")
        _check(lib().sgq_add_scaled(self._h, _ptr(a), _ptr(b), _ptr(y), n, s))

    def fill_q4_0_random(self, w: torch.Tensor, n_blocks: int, seed: int, sigma: float = 0.02):
        _need(w, torch.uint8, n_blocks * 18, "w")
        _check(lib().sgq_fill_q4_0_random(self._h, _ptr(w), n_blocks, seed, sigma))

    def fill_normal(self, x: torch.Tensor, seed: int, mean: float = 0.0, sigma: float = 1.0):
        _need(x, torch.float32, x.numel(), "x")
        _check(lib().sgq_fill_normal(self._h, _ptr(x), x.numel(), seed, mean, sigma))

    # -- timing -------------------------------------------------------------
    def timer_start(self):
        _check(lib().sgq_timer_start(self._h))

    def timer_stop(self) -> float:
        ms = C.c_float()
        _check(lib().sgq_timer_stop(self._h, C.byref(ms)))
        return ms.value


class Graph:
    """A recorded, re-submittable command graph (CommandGraph)."""

    def __init__(self, ctx: GpuContext, handle):
        self.ctx = ctx
        self.handle = handle

    def submit(self):
        _check(lib().sgq_graph_submit(self.ctx.handle, self.handle))

    def __del__(self):
        if getattr(self, "handle", None) is not None and _lib is not None:
            _lib.sgq_graph_destroy(self.handle)
            self.handle = None


class GraphRecorder:
    """Context manager capturing every dispatch on ctx's stream into a Graph.

    The context's stream must not be the null stream while recording; use a
    side torch stream (``with torch.cuda.stream(s): ctx.set_stream(s)``).
    """

    def __init__(self, ctx: GpuContext):
        self.ctx = ctx
        self.graph: Optional[Graph] = None

    def __enter__(self):
        _check(lib().sgq_graph_begin(self.ctx.handle))
        return self

    def __exit__(self, exc_type, exc, tb):
        h = C.c_void_p()
        rc = lib().sgq_graph_end(self.ctx.handle, C.byref(h))
        if exc_type is None:
            _check(rc)
            self.graph = Graph(self.ctx, h)
        return False


@dataclass
class GgufTensor:
    name: str
    type: int
    dims: tuple
    offset: int
    nbytes: int
    data_ptr: int


class Gguf:
    """A GGUF v3 file (sgq_gguf_*, crates/sg-gguf/src/parse.rs): tensor table,
    metadata, zero-copy tensor bytes.  No GPU needed."""

    def __init__(self, path: str):
        h = C.c_void_p()
        _check(lib().sgq_gguf_open(os.fsencode(path), C.byref(h)))
        self._h = h

    def close(self):
        if getattr(self, "_h", None) is not None and _lib is not None:
            _lib.sgq_gguf_close(self._h)
            self._h = None

    def __del__(self):
        self.close()

    @staticmethod
    def _wrap(t: _GgufTensor) -> GgufTensor:
        return GgufTensor(t.name.decode(), t.type, tuple(t.dims[:t.n_dims]), t.offset, t.bytes,
                          t.data)

    def tensors(self):
        out = []
        for i in range(lib().sgq_gguf_tensor_count(self._h)):
            t = _GgufTensor()
            _check(lib().sgq_gguf_tensor_at(self._h, i, C.byref(t)))
            out.append(self._wrap(t))
        return out

    def find(self, name: str) -> GgufTensor:
        t = _GgufTensor()
        _check(lib().sgq_gguf_tensor_find(self._h, name.encode(), C.byref(t)))
        return self._wrap(t)

    def data(self, t: GgufTensor) -> bytes:
        return C.string_at(t.data_ptr, t.nbytes)

    def meta_int(self, key: str) -> int:
        v = C.c_int64()
        _check(lib().sgq_gguf_meta_int(self._h, key.encode(), C.byref(v)))
        return v.value

    def meta_float(self, key: str) -> float:
        v = C.c_double()
        _check(lib().sgq_gguf_meta_float(self._h, key.encode(), C.byref(v)))
        return v.value

    def meta_string(self, key: str) -> str:
        v = C.c_char_p()
        _check(lib().sgq_gguf_meta_string(self._h, key.encode(), C.byref(v)))
        return v.value.decode()


def default_model_config(**overrides) -> ModelConfig:
    """The benchmark decoder shape (sgq_model_default_config), with overrides."""
    cfg = ModelConfig()
    lib().sgq_model_default_config(C.byref(cfg))
    for k, v in overrides.items():
        if not hasattr(cfg, k):
            raise ValidationError(6, f"unknown model config field {k}")
        setattr(cfg, k, v)
    return cfg


class Model:
    """The decode-step driver (sgq_model_*): a random-init decoder resident on
    the context's device.  ``decode(token, logits)`` runs one step at the
    current position and advances it; ``graph=True`` replays a recorded
    hipGraph of the step (the context needs a non-null stream)."""

    def __init__(self, ctx: GpuContext, cfg: Optional[ModelConfig] = None):
        self.ctx = ctx
        self.cfg = cfg if cfg is not None else default_model_config()
        h = C.c_void_p()
        _check(lib().sgq_model_create(ctx.handle, C.byref(self.cfg), C.byref(h)))
        self._h = h

    def close(self):
        if getattr(self, "_h", None) is not None and _lib is not None:
            _lib.sgq_model_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    @property
    def position(self) -> int:
        return int(lib().sgq_model_position(self._h))

    def reset(self):
        _check(lib().sgq_model_reset(self._h))

    def decode(self, token: int, logits: torch.Tensor, graph: bool = False):
        _need(logits, torch.float32, self.cfg.vocab, "logits")
        fn = lib().sgq_model_decode_graph if graph else lib().sgq_model_decode
        _check(fn(self._h, int(token), _ptr(logits)))

    @property
    def decode_mode(self) -> int:
        """0: one kernel per operator; 2: five fused launches per layer;
        3: one kernel per operator at any supported geometry."""
        return int(lib().sgq_model_decode_mode(self._h))

    @decode_mode.setter
    def decode_mode(self, mode: int):
        _check(lib().sgq_model_set_decode_mode(self._h, int(mode)))

    def status(self):
        """Wait for the stream."""
        _check(lib().sgq_model_status(self._h))

    def prefill(self, tokens, logits: Optional[torch.Tensor] = None):
        """Run a prompt (host token ids) through the model at the current
        position; logits of its last token into `logits` when given."""
        import numpy as np
        toks = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32))
        if logits is not None:
            _need(logits, torch.float32, self.cfg.vocab, "logits")
        _check(lib().sgq_model_prefill(self._h, toks.ctypes.data_as(C.POINTER(U32)), toks.size,
                                       _ptr(logits)))

    def load_gguf(self, gguf: "Gguf"):
        """Upload a GGUF's weights (sgq_model_load_gguf)."""
        _check(lib().sgq_model_load_gguf(self._h, gguf._h))

    def fill_cache(self, n_tokens: int, seed: int = 0xCAC4E):
        """Synthetic Q8_0 K/V for positions [0, n_tokens); position = n_tokens."""
        _check(lib().sgq_model_fill_cache(self._h, n_tokens, seed))

    def tensor_ptr(self, name: str, layer: int = -1):
        p, b = C.c_void_p(), C.c_uint64()
        _check(lib().sgq_model_tensor(self._h, layer, name.encode(), C.byref(p), C.byref(b)))
        return p.value, b.value

    def write_tensor(self, name: str, data, layer: int = -1):
        """Overwrite a named device tensor with host bytes of exactly its size."""
        import numpy as np
        a = np.ascontiguousarray(data)
        p, b = self.tensor_ptr(name, layer)
        if a.nbytes != b:
            raise ValidationError(6, f"{name}[{layer}]: {a.nbytes} bytes given, tensor has {b}")
        _check(lib().sgq_buf_upload(self.ctx.handle, p, a.ctypes.data, b))

    def read_tensor(self, name: str, layer: int = -1, dtype=None):
        """Host copy (numpy) of a named device tensor."""
        import numpy as np
        p, b = self.tensor_ptr(name, layer)
        out = np.empty(b, np.uint8)
        _check(lib().sgq_buf_download(self.ctx.handle, out.ctypes.data, p, b))
        if dtype is None:
            dtype = np.uint8 if name.startswith(("attn_", "ffn_", "token_embd")) and \
                not name.endswith("norm") else np.float32
        return out.view(dtype)


def _need(t, dtypes, numel, name):
    if t is None:
        raise ValidationError(6, f"{name} is required")
    if not isinstance(dtypes, tuple):
        dtypes = (dtypes,)
    if t.dtype not in dtypes:
        raise ValidationError(6, f"{name}: dtype {t.dtype} not in {dtypes}")
    if t.numel() < numel:
        raise ValidationError(6, f"{name}: {t.numel()} elements < required {numel}")
    if not t.is_contiguous():
        raise ValidationError(6, f"{name}: must be contiguous")
