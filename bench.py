"""Benchmark of the super-gemma quantized compute core on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Prints ONE JSON line (rank 0).  A "step" is one pass of the hot path over one
batch of synthetic input, already resident in HBM:

  prefill BASELINE config 5's prefill: a 4096-token prompt from position 0;
          value = prompt tok/s.
  decode  BASELINE config 5 (default): one bs=1 decode step of the 62-layer
          random-init decoder at an 8K context (synthetic Q8_0 K/V pages for
          positions 0..8191), replayed as one hipGraph; value = tok/s.
  gemv    BASELINE config 1: Q4_0 GEMV K=5376, N=21504 (decode), rotating over
          8 weight copies (520 MB > the 256 MB MALL) so every launch streams
          its weights from HBM.
  mmq     BASELINE config 2: Q4_0×Q8 int8-MFMA GEMM M=512, K=5376, N=21504.
  splitk  BASELINE config 3: down-proj M=2048, K=21504, N=5376, split-K 4
          (--split-k 1/2/4/8).
  attn_prefill, attn_prefill_sliding
          BASELINE config 4 prefill: 4096 queries, causal / sliding-1024.
  attn_prefill_ipv
          the same causal prefill with int8 PV over key-blocked V.
  attn_decode_4k, attn_decode_32k, attn_decode_128k
          BASELINE config 4 decode over a 4K / 32K / 128K Q8_0 context.
  head_q6k
          the real checkpoint's tied Q6_K LM head (262144 x 5376, rows padded
          to 4416 B) with the 30*tanh softcap (gemv_q6_k_logits).

The timed region is bracketed by torch.cuda.synchronize() and measured with
HIP events on the stream the kernels run on.  The cpu_baseline leg times the
CPU restatement of the reference's Q4_0 matmul (oracle/, reference.rs:402-444)
on a bounded sample on the host cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "super-gemma_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E, GB/s
INT8_PEAK_TOPS = 5000.0    # MI355X dense int8 MFMA, TOP/s
METRIC = "decode tok/s (31B Q4_0 shape, bs=1) + Q4_0 GEMV GB/s vs HBM peak"


def q4_bytes(n, k):
    return n * (k // 32) * 18


class Gemv:
    name = "gemv_q4_0 K=5376 N=21504 (BASELINE config 1), 8 rotating weight copies"
    kernel = "gemv_q4_0_ring_kernel"

    def __init__(self, ctx, torch, n=21504, k=5376):
        self.ctx, self.torch = ctx, torch
        self.k, self.n = k, n
        if n != 21504 or k != 5376:
            self.name = f"gemv_q4_0 K={k} N={n} (shape sweep around config 1), 8 rotating copies"
        self.copies = 8
        nbytes = q4_bytes(self.n, self.k)
        self.w = [torch.empty(nbytes, dtype=torch.uint8, device="cuda") for _ in range(self.copies)]
        for i, w in enumerate(self.w):
            ctx.fill_q4_0_random(w, nbytes // 18, seed=100 + i, sigma=0.02)
        self.x = torch.empty(self.k, dtype=torch.float32, device="cuda")
        ctx.fill_normal(self.x, seed=7)
        self.y = torch.empty(self.n, dtype=torch.float32, device="cuda")
        # algorithmic bytes per launch: W + x (fp32) + y (fp32)
        self.bytes = nbytes + self.k * 4 + self.n * 4

    def step(self, i):
        self.ctx.gemv_q4_0(self.w[i % self.copies], self.x, self.y, self.n, self.k)

    def result(self, ms_per_step):
        gbs = self.bytes / (ms_per_step * 1e-3) / 1e9
        return {
            "value": gbs, "unit": "GB/s",
            "dtype": "q4_0 weights, fp32 x/y; x enters the i4 dot8 as 15-bit fixed point per "
                     "32-block (4 limbs)",
            "roofline": ring_roofline(self.ctx, self.torch, [w.data_ptr() for w in self.w],
                                      self.k, self.n,
                                      traffic=(self.k, self.n) == (5376, 21504)),
            "config": {"workload": self.name, "m": 1, "k": self.k, "n": self.n,
                       "bytes_per_launch": self.bytes},
        }


class Mmq:
    kernel = "mmq_kernel"

    def __init__(self, ctx, torch, m=512, k=5376, n=21504, split=1, label="BASELINE config 2"):
        self.ctx, self.torch = ctx, torch
        self.m, self.k, self.n, self.split = m, k, n, split
        self.name = f"gemm_q4_0_q8 int8 MFMA M={m} K={k} N={n} split_k={split} ({label})"
        self.w = torch.empty(q4_bytes(n, k), dtype=torch.uint8, device="cuda")
        ctx.fill_q4_0_random(self.w, n * k // 32, seed=21, sigma=0.02)
        x = torch.empty(m * k, dtype=torch.float32, device="cuda")
        ctx.fill_normal(x, seed=22)
        if split > 1:  # config 3: GeGLU-like activations gelu(N(0,1))*N(0,1)
            u = torch.empty_like(x)
            ctx.fill_normal(u, seed=23)
            x = (torch.nn.functional.gelu(x, approximate="tanh") * u).contiguous()
        self.xs = torch.empty(m * k // 32, dtype=torch.int16, device="cuda")
        self.xq = torch.empty(m * k, dtype=torch.int8, device="cuda")
        ctx.quant_q8_0(x, self.xs, self.xq)
        del x
        self.y = torch.empty(m * n, dtype=torch.float32, device="cuda")
        # split > 1: the K-slice partials; split 1: the workspace that lets the
        # last part-filled round of tiles split over K
        self.part = torch.empty(split * m * n, dtype=torch.float32, device="cuda")
        self.ops = 2.0 * m * n * k

    def step(self, i):
        self.ctx.gemm_q4_0_q8(self.w, self.xq, self.xs, self.y, self.m, self.n, self.k,
                              self.split, self.part)

    def result(self, ms_per_step):
        tops = self.ops / (ms_per_step * 1e-3) / 1e12
        return {
            "value": tops, "unit": "TOP/s", "dtype": "int8 x q4_0 -> i32 MFMA, fp32 rescale",
            "roofline": {"bound": "mfma", "achieved": tops, "peak": INT8_PEAK_TOPS,
                         "unit": "TOP/s", "frac": tops / INT8_PEAK_TOPS, "traffic": None},
            "config": {"workload": self.name, "m": self.m, "k": self.k, "n": self.n,
                       "split_k": self.split, "ops_per_launch": self.ops},
        }


F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA


class AttnPrefill:
    """BASELINE config 4 prefill: 4096 queries, 32 q / 16 kv heads, hd 128,
    causal (window 0) or sliding-1024, over a Q8_0 cache of N(0,1) K/V."""
    kernel = "attn_prefill_kernel"

    def __init__(self, ctx, torch, window=0, n_tok=4096, ipv=False):
        self.ctx, self.torch, self.window, self.n_tok = ctx, torch, window, n_tok
        self.ipv = ipv
        n_q, n_kv, hd = 32, 16, 128
        self.n_q, self.n_kv = n_q, n_kv
        kv = torch.empty(n_tok * n_kv * hd, dtype=torch.float32, device="cuda")
        self.kq = torch.empty(kv.numel(), dtype=torch.int8, device="cuda")
        self.vq = torch.empty(kv.numel(), dtype=torch.int8, device="cuda")
        self.ks = torch.empty(kv.numel() // 32, dtype=torch.int16, device="cuda")
        self.vs = torch.empty(kv.numel() // 32, dtype=torch.int16, device="cuda")
        ctx.fill_normal(kv, seed=41)
        ctx.quant_q8_0(kv, self.ks, self.kq)
        ctx.fill_normal(kv, seed=42)
        if ipv:  # V with key-blocked scales (int8 PV)
            self.vs_kb = torch.empty(((n_tok + 31) // 32) * n_kv * hd, dtype=torch.int16,
                                     device="cuda")
            ctx.kv_append_v_q8(kv, n_tok, n_kv * hd, 0, self.vq, self.vs_kb)
        else:
            ctx.quant_q8_0(kv, self.vs, self.vq)
        self.q = torch.empty(n_tok * n_q * hd, dtype=torch.float32, device="cuda")
        ctx.fill_normal(self.q, seed=43)
        self.out = torch.empty_like(self.q)
        pairs = sum(min(i + 1, window) if window else i + 1 for i in range(n_tok))
        self.flops = 4.0 * hd * n_q * pairs  # QK^T and PV, 2 flops per MAC
        self.name = (f"attn_prefill_{'ipv' if ipv else 'q8'} {n_tok} queries, 32q/16kv, hd 128, "
                     f"{'sliding-%d' % window if window else 'causal'} (BASELINE config 4)"
                     + (", int8 PV with key-blocked V" if ipv else ""))

    def step(self, i):
        if self.ipv:
            self.ctx.attn_prefill_ipv(self.q, self.kq, self.ks, self.vq, self.vs_kb, self.n_tok, 0,
                                      self.n_q, self.n_kv, self.out)
            return
        self.ctx.attn_prefill_q8(self.q, self.kq, self.ks, self.vq, self.vs, self.n_tok, 0,
                                 self.n_q, self.n_kv, self.out, window=self.window)

    def result(self, ms_per_step):
        tf = self.flops / (ms_per_step * 1e-3) / 1e12
        return {
            "value": tf, "unit": "TFLOP/s",
            "dtype": ("f16 MFMA QK, int8 MFMA PV (P quantized per 32-key block), fp32 acc"
                      if self.ipv else "f16 MFMA (K/V dequantized from Q8_0), fp32 acc"),
            "roofline": {"bound": "mfma", "achieved": tf, "peak": F16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": tf / F16_PEAK_TFLOPS, "traffic": None},
            "config": {"workload": self.name, "flops_per_launch": self.flops},
        }


class AttnDecode:
    """BASELINE config 4 decode: bs 1, 32 q / 16 kv heads, hd 128, Q8_0 K/V
    over a context of `ctx_len` (4K/32K/128K), split over the sequence."""
    kernel = "attn_decode_q8_kernel"

    def __init__(self, ctx, torch, ctx_len=32768, splits=None):
        import sgq

        self.ctx, self.torch, self.ctx_len = ctx, torch, ctx_len
        n_q, n_kv, hd = 32, 16, 128
        self.n_q, self.n_kv = n_q, n_kv
        # rotate copies so the KV pages stream from HBM (>= 512 MB in total)
        self.copies = max(1, (512 << 20) // (ctx_len * 4352))
        kv = torch.empty(ctx_len * n_kv * hd, dtype=torch.float32, device="cuda")
        self.pages = []
        for c in range(self.copies):
            kq = torch.empty(kv.numel(), dtype=torch.int8, device="cuda")
            vq = torch.empty(kv.numel(), dtype=torch.int8, device="cuda")
            ks = torch.empty(kv.numel() // 32, dtype=torch.int16, device="cuda")
            vs = torch.empty(kv.numel() // 32, dtype=torch.int16, device="cuda")
            ctx.fill_normal(kv, seed=50 + 2 * c)
            ctx.quant_q8_0(kv, ks, kq)
            ctx.fill_normal(kv, seed=51 + 2 * c)
            ctx.quant_q8_0(kv, vs, vq)
            self.pages.append((kq, ks, vq, vs))
        del kv
        self.q = torch.empty(n_q * hd, dtype=torch.float32, device="cuda")
        ctx.fill_normal(self.q, seed=52)
        self.out = torch.empty_like(self.q)
        # 256 slots per split, 64..256 splits: the one-wave-per-(kv head,
        # split) kernel (sweep: 4K best at 64, 32K at 128, 128K at 128-256)
        self.splits = splits or min(256, max(64, ctx_len // 256))
        self.bytes = ctx_len * n_kv * (2 * hd + 2 * (hd // 32) * 2) + 2 * n_q * hd * 4
        # one graph replays the split + merge pair over every cache copy, as
        # the decode step's graph does (no host launch cost between pairs); a
        # step is one replay, reported per pair
        self.stream = torch.cuda.Stream()
        ctx.set_stream(self.stream)
        self._pair(0)  # eager first call: any lazy set-up happens outside the capture
        ctx.synchronize()
        with sgq.GraphRecorder(ctx) as rec:
            for c in range(self.copies):
                self._pair(c)
        self.graph = rec.graph

    def _pair(self, c):
        kq, ks, vq, vs = self.pages[c]
        self.ctx.attn_decode_q8(self.q, kq, ks, vq, vs, self.ctx_len, self.n_q, self.n_kv,
                                self.out, n_splits=self.splits, scale=1.0)

    def step(self, i):
        self.graph.submit()

    def result(self, ms_per_step):
        ms_per_step = ms_per_step / self.copies
        gbs = self.bytes / (ms_per_step * 1e-3) / 1e9
        return {
            "value": gbs, "unit": "GB/s", "dtype": "q8_0 K/V, fp32 q/out",
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": gbs / HBM_PEAK_GBS, "traffic": None},
            "config": {"workload": f"attn_decode_q8 ctx {self.ctx_len}, 32q/16kv, hd 128, "
                                   f"{self.splits} splits, {self.copies} rotating caches "
                                   "(BASELINE config 4), one hipGraph replay over the copies",
                       "bytes_per_launch": self.bytes, "us_per_pair": ms_per_step * 1e3},
        }


class AttnPages:
    """The released checkpoint's decode attention by name over f16 pages, as
    the reference's record_layer dispatches it (crates/sg-model/src/graph.rs:
    572-650): attn_decode_global_q8k (Q8_0 K, f16 V, head_dim 512, 4 kv
    heads, 32 splits) or attn_decode_sliding (f16 K/V, head_dim 256, 16 kv
    heads, the full 1024-slot ring, 16 splits), then its attn_reduce.  One
    graph replays the pair over rotating caches (>= 512 MB) so the pages
    stream from HBM; a step is one replay, reported per pair."""
    kernel = "attn_decode_pages_kernel"

    def __init__(self, ctx, torch, kind="global_q8k", ctx_len=8192):
        import struct
        import sgq

        self.ctx, self.torch, self.kind, self.ctx_len = ctx, torch, kind, ctx_len
        if kind == "sliding":
            hd, n_kv, self.splits, word = 256, 16, 16, 1
        else:
            hd, n_kv, self.splits, word = 512, 4, 32, 2
        n_q, row = 32, n_kv * hd
        k_bytes = ctx_len * row * (1 + 2 / 32) if kind == "global_q8k" else ctx_len * row * 2
        self.bytes = int(k_bytes + ctx_len * row * 2)
        self.copies = max(1, (512 << 20) // self.bytes)
        tmp = torch.empty(ctx_len * row, dtype=torch.float32, device="cuda")
        q = torch.empty(n_q * hd, dtype=torch.float32, device="cuda")
        ctx.fill_normal(q, seed=60)
        q16 = q.half().view(torch.int16)
        step = torch.zeros(8, dtype=torch.int32, device="cuda")
        kvs = [ctx_len - 1, ctx_len if word == 1 else 0, ctx_len if word == 2 else 0, 0]
        ctx.step_write(step, sgq.StepState(*kvs))
        part = torch.empty(n_q * self.splits * (hd + 2), dtype=torch.float32, device="cuda")
        out = torch.empty(n_q * hd, dtype=torch.int16, device="cuda")
        attn = ctx.load_kernel(f"attn_decode_{kind}")
        red = ctx.load_kernel(f"attn_reduce_d{hd}")
        self.pages = []
        for c in range(self.copies):
            ctx.fill_normal(tmp, seed=61 + 2 * c)
            if kind == "global_q8k":
                kq = torch.empty(tmp.numel(), dtype=torch.int8, device="cuda")
                ks = torch.empty(tmp.numel() // 32, dtype=torch.int16, device="cuda")
                ctx.quant_q8_0(tmp, ks, kq)
                kb = (kq, ks)
            else:
                kb = (tmp.half().view(torch.int16),)
            ctx.fill_normal(tmp, seed=62 + 2 * c)
            self.pages.append((kb, tmp.half().view(torch.int16)))
        del tmp
        torch.cuda.synchronize()
        self.stream = torch.cuda.Stream()
        ctx.set_stream(self.stream)

        def bind(*ts):
            return [sgq.BufferBinding.buffer(i, t) for i, t in enumerate(ts)]

        with sgq.GraphRecorder(ctx) as rec:
            for kb, v in self.pages:
                ctx.dispatch(attn, bind(q16, *kb, v, part, step),
                             struct.pack("<If", self.splits, 1.0), [n_kv, self.splits, 1])
                ctx.dispatch(red, bind(part, out), struct.pack("<I", self.splits), [n_q, 1, 1])
        self.graph = rec.graph
        self.hd, self.n_kv = hd, n_kv

    def step(self, i):
        self.graph.submit()

    def result(self, ms_per_step):
        ms = ms_per_step / self.copies
        gbs = self.bytes / (ms * 1e-3) / 1e9
        return {
            "value": gbs, "unit": "GB/s",
            "dtype": "f16 q / V" + (", Q8_0 K" if self.kind == "global_q8k" else ", f16 K")
                     + "; fp32 MFMA accumulation, f16 out",
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": gbs / HBM_PEAK_GBS, "traffic": None},
            "config": {"workload": f"attn_decode_{self.kind} + attn_reduce_d{self.hd} by name, "
                                   f"{self.ctx_len} slots, 32 q / {self.n_kv} kv heads, "
                                   f"{self.splits} splits, {self.copies} rotating caches",
                       "bytes_per_launch": self.bytes, "us_per_pair": ms * 1e3},
        }


class AttnPrefillPages:
    """The released checkpoint's prefill attention by name, as the
    reference's record_prefill_layer dispatches it (crates/sg-model/src/
    graph.rs:1176-1225) for a 4096-token prompt from position 0 (q0 =
    step[3] = 0): attn_prefill_global_flash_sp_iq (int8 q with f16 scales,
    Q8_0 K, f16 V, head_dim 512, 4 kv heads, causal; groups [32, M/16, 1]) or
    attn_prefill_sliding_ring (f16 q / K / V, head_dim 256, 16 kv heads,
    window 1024: the ring holds the slots before the chunk, the chunk's own
    K/V come from its pages; groups [16, M, 1]).  One dispatch per step,
    replayed from a graph."""
    kernel = "attn_prefill_wide_kernel"

    def __init__(self, ctx, torch, kind="global_flash_sp_iq", n_tok=4096):
        import struct
        import sgq

        self.ctx, self.kind, self.n_tok = ctx, kind, n_tok
        n_q = 32
        if kind == "sliding_ring":
            hd, n_kv, window, scale = 256, 16, 1024, 1.0 / (256 ** 0.5)
        else:
            hd, n_kv, window, scale = 512, 4, 0, 1.0
        self.hd, self.n_kv, self.window = hd, n_kv, window
        row = n_kv * hd
        f = torch.empty(n_tok * max(n_q * hd, row), dtype=torch.float32, device="cuda")

        def normal(n, seed):
            ctx.fill_normal(f[:n], seed=seed)
            return f[:n]

        step = torch.zeros(8, dtype=torch.int32, device="cuda")
        ctx.step_write(step, sgq.StepState(0, 0, 0, 0))
        out = torch.empty(n_tok * n_q * hd, dtype=torch.int16, device="cuda")
        if kind == "sliding_ring":
            q16 = normal(n_tok * n_q * hd, 70).half().view(torch.int16)
            ring_k = torch.zeros(1024 * row, dtype=torch.int16, device="cuda")
            ring_v = torch.zeros_like(ring_k)
            ck = normal(n_tok * row, 71).half().view(torch.int16)
            cv = normal(n_tok * row, 72).half().view(torch.int16)
            binds = [q16, ring_k, ring_v, ck, cv, out, step]
            groups = [n_kv, n_tok, 1]
        else:
            qq = torch.empty(n_tok * n_q * hd, dtype=torch.int8, device="cuda")
            qs = torch.empty(qq.numel() // 32, dtype=torch.int16, device="cuda")
            ctx.quant_q8_0(normal(qq.numel(), 73), qs, qq)
            kq = torch.empty(n_tok * row, dtype=torch.int8, device="cuda")
            ks = torch.empty(kq.numel() // 32, dtype=torch.int16, device="cuda")
            ctx.quant_q8_0(normal(kq.numel(), 74), ks, kq)
            v16 = normal(n_tok * row, 75).half().view(torch.int16)
            binds = [qq, qs, kq, ks, v16, out, step]
            groups = [n_q, n_tok // 16, 1]
        del f
        self._keep = binds
        torch.cuda.synchronize()
        self.stream = torch.cuda.Stream()
        ctx.set_stream(self.stream)
        k = ctx.load_kernel(f"attn_prefill_{kind}")
        with sgq.GraphRecorder(ctx) as rec:
            ctx.dispatch(k, [sgq.BufferBinding.buffer(i, t) for i, t in enumerate(binds)],
                         struct.pack("<f", scale), groups)
        self.graph = rec.graph
        pairs = sum(min(i + 1, window) if window else i + 1 for i in range(n_tok))
        self.flops = 4.0 * hd * n_q * pairs  # QK^T and PV, 2 flops per MAC

    def step(self, i):
        self.graph.submit()

    def result(self, ms_per_step):
        tf = self.flops / (ms_per_step * 1e-3) / 1e12
        iq = self.kind != "sliding_ring"
        return {
            "value": tf, "unit": "TFLOP/s",
            "dtype": ("int8 q / Q8_0 K as exact f16 on the f16 MFMA (block dots scaled), f16 V"
                      if iq else "f16 q / K / V") + "; fp32 acc, f16 out",
            "roofline": {"bound": "mfma", "achieved": tf, "peak": F16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": tf / F16_PEAK_TFLOPS, "traffic": None},
            "config": {"workload": f"attn_prefill_{self.kind} by name, {self.n_tok} queries "
                                   f"from position 0, 32 q / {self.n_kv} kv heads, head_dim "
                                   f"{self.hd}, " + (f"window {self.window}" if self.window
                                                     else "causal"),
                       "flops_per_launch": self.flops},
        }


class HeadQ6K:
    """The Q6_K tied LM head of the real checkpoint (gemv_q6_k_logits.wgsl):
    262144 vocabulary rows x K=5376, rows padded to 4416 bytes, 30*tanh
    softcap; 1.16 GB per launch, so it streams from HBM."""
    kernel = "gemv_q6_k_kernel"

    def __init__(self, ctx, torch, n=262144, k=5376, stride=4416):
        self.ctx, self.torch = ctx, torch
        self.n, self.k, self.stride = n, k, stride
        self.w = torch.zeros(n * stride, dtype=torch.uint8, device="cuda")
        # random bytes, then bounded sub-scales and small d (parity_logits.rs:31-51)
        g = torch.Generator(device="cuda").manual_seed(61)
        self.w.copy_(torch.randint(0, 256, (n * stride,), dtype=torch.uint8, device="cuda",
                                   generator=g))
        blk = self.w.view(n, stride)[:, :(k // 256) * 210].reshape(n, k // 256, 210)
        blk[:, :, 192:208] = (blk[:, :, 192:208] & 15).to(torch.int16).sub(8).to(torch.int8).view(torch.uint8)
        d = (torch.rand(n, k // 256, device="cuda", generator=g) * 1e-3).to(torch.float16)
        blk[:, :, 208:210] = d.view(torch.uint8).view(n, k // 256, 2)
        self.x = torch.empty(k, dtype=torch.float32, device="cuda")
        ctx.fill_normal(self.x, seed=62)
        self.y = torch.empty(n, dtype=torch.float32, device="cuda")
        self.bytes = n * stride + k * 4 + n * 4

    def step(self, i):
        self.ctx.gemv_q6_k(self.w, self.stride, self.x, self.y, self.n, self.k, 30.0)

    def result(self, ms_per_step):
        gbs = self.bytes / (ms_per_step * 1e-3) / 1e9
        return {
            "value": gbs, "unit": "GB/s", "dtype": "q6_k weights, f16 x (from fp32), f32 dot",
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": gbs / HBM_PEAK_GBS, "traffic": None},
            "config": {"workload": f"gemv_q6_k_logits N={self.n} K={self.k} stride {self.stride} "
                                   "(the real checkpoint's tied Q6_K head)",
                       "bytes_per_launch": self.bytes},
        }


class Prefill:
    """BASELINE config 5 prefill: a 4096-token prompt of seeded random ids
    through the 62-layer random-init decoder from position 0 (one chunk),
    last-token logits.  value = prompt tokens per second."""
    kernel = "mmq_kernel"

    def __init__(self, ctx, torch, n_tok=4096, real=False):
        import numpy as np
        import sgq

        self.ctx, self.torch, self.n_tok, self.real = ctx, torch, n_tok, real
        self.stream = torch.cuda.Stream()
        ctx.set_stream(self.stream)
        if real:  # the released checkpoint's geometry (crates/sg-gguf/src/desc.rs:66-93)
            self.cfg = sgq.default_model_config(
                n_layers=60, global_every=6, head_dim=256, head_dim_global=512, n_kv_heads=16,
                n_kv_heads_global=4, embed_q6k=1, max_ctx=n_tok, prefill_chunk=n_tok)
        else:
            self.cfg = sgq.default_model_config(max_ctx=n_tok, prefill_chunk=n_tok)
        self.model = sgq.Model(ctx, self.cfg)
        self.tokens = np.random.default_rng(11).integers(0, self.cfg.vocab, n_tok).astype(np.uint32)
        self.logits = torch.empty(self.cfg.vocab, dtype=torch.float32, device="cuda")
        c = self.cfg
        H, F = c.hidden, c.ffn
        self.mmq_ops, self.attn_flops = 0, 0.0
        for l in range(c.n_layers):
            glob = l % c.global_every == c.global_every - 1
            hd = (c.head_dim_global or c.head_dim) if glob else c.head_dim
            nkv = (c.n_kv_heads_global or c.n_kv_heads) if glob else c.n_kv_heads
            QD, KD = c.n_q_heads * hd, nkv * hd
            kv_proj = KD if glob and c.global_k_eq_v else 2 * KD
            self.mmq_ops += 2 * n_tok * H * (QD + kv_proj + 2 * F) + 2 * n_tok * QD * H \
                + 2 * n_tok * F * H
            w = 0 if glob else c.sliding_window
            self.attn_flops += 4.0 * hd * c.n_q_heads * sum(min(i + 1, w) if w else i + 1
                                                            for i in range(n_tok))

    def step(self, i):
        self.model.reset()
        self.model.prefill(self.tokens, self.logits)

    def mmq_roofline(self):
        """The dominant kernel alone: the MMQ at the prefill's gate/up shape
        (M=4096, K=5376, N=21504), timed with HIP events over 10 launches."""
        t = self.torch
        m, k, n = self.n_tok, 5376, 21504
        mm = Mmq(self.ctx, t, m=m, k=k, n=n, label="prefill gate/up shape")
        mm.step(0)
        self.ctx.synchronize()
        self.ctx.timer_start()
        for i in range(10):
            mm.step(i)
        ms = self.ctx.timer_stop() / 10
        r = mm.result(ms)["roofline"]
        r["kernel"] = f"mmq_kernel M={m} K={k} N={n} (int8 ops only)"
        r["us_per_launch"] = ms * 1e3
        del mm
        return r

    def result(self, ms_per_step):
        tops = (self.mmq_ops + self.attn_flops) / (ms_per_step * 1e-3) / 1e12
        c = self.cfg
        return {
            "value": self.n_tok / (ms_per_step * 1e-3), "unit": "tok/s (prefill)",
            "dtype": "q4_0 weights x q8_0 activations (int8 MFMA), f16 attention",
            "roofline": self.mmq_roofline(),
            "whole_prefill_rate": {"achieved": tops, "unit": "TOP/s",
                                   "note": "MMQ int8 ops + attention f16 flops per second "
                                           "over the whole prefill (mixed units: no peak)"},
            "config": {"workload": (f"prefill {self.n_tok} tokens from position 0, released-"
                                    "checkpoint geometry (60 layers, head_dim 256/512, 16/4 kv "
                                    "heads, Q6_K embedding/head), random init") if self.real else
                                   (f"prefill {self.n_tok} tokens from position 0, 62-layer "
                                    "random-init decoder (BASELINE config 5)"),
                       "n_layers": c.n_layers, "hidden": c.hidden, "ffn": c.ffn,
                       "mmq_ops": self.mmq_ops, "attn_flops": self.attn_flops},
        }


class Decode:
    """one bs=1 decode step of the full 62-layer random-init
    decoder at an 8K-token context, replayed as one hipGraph per step."""
    kernel = "gemv_q4_0_ring_kernel"

    def __init__(self, ctx, torch, context=8192, mode="fused"):
        import sgq

        self.ctx, self.torch, self.sgq = ctx, torch, sgq
        self.stream = torch.cuda.Stream()
        ctx.set_stream(self.stream)
        self.cfg = sgq.default_model_config(max_ctx=16384)
        self.model = sgq.Model(ctx, self.cfg)
        self.mode = mode
        self.model.decode_mode = {"kernels": 0, "fused": 2}[mode]
        self.context = context
        self.model.fill_cache(context)
        self.logits = torch.empty(self.cfg.vocab, dtype=torch.float32, device="cuda")
        c = self.cfg
        H, F, QD, KD = c.hidden, c.ffn, c.n_q_heads * 128, c.n_kv_heads * 128
        n_glob = sum(1 for l in range(c.n_layers) if l % c.global_every == c.global_every - 1)
        n_slide = c.n_layers - n_glob
        per_layer = q4_bytes(QD, H) + q4_bytes(KD, H) + q4_bytes(H, QD) + 2 * q4_bytes(F, H) \
            + q4_bytes(H, F)
        self.weight_bytes = c.n_layers * per_layer + n_slide * q4_bytes(KD, H) \
            + (0 if c.global_k_eq_v else n_glob * q4_bytes(KD, H)) + q4_bytes(c.vocab, H)
        kv_row = KD * (1 + 2 / 32) * 2  # K and V quants + f16 scales per position
        ctx_pos = context + 1
        self.kv_bytes = int(kv_row * (n_slide * min(ctx_pos, c.sliding_window) + n_glob * ctx_pos))
        self.bytes = self.weight_bytes + self.kv_bytes
        self.rng = __import__("random").Random(5)

    def step(self, i):
        self.model.decode(self.rng.randrange(self.cfg.vocab), self.logits, graph=True)

    def kernel_roofline(self):
        return ring_roofline(self.ctx, self.torch,
                             [self.model.tensor_ptr("ffn_gate", l)[0]
                              for l in range(self.cfg.n_layers)], 5376, 21504)

    def result(self, ms_per_step):
        tok_s = 1000.0 / ms_per_step
        step_gbs = self.bytes / (ms_per_step * 1e-3) / 1e9
        c = self.cfg
        return {
            "value": tok_s, "unit": "tok/s",
            "dtype": "q4_0 weights x i4-limb activations (15-bit fixed point per 32-block) "
                     "in every GEMV, q8_0 kv, fp32 elsewhere",
            "roofline": self.kernel_roofline(),
            "step_roofline": {"bound": "hbm", "achieved": step_gbs, "peak": HBM_PEAK_GBS,
                              "unit": "GB/s", "frac": step_gbs / HBM_PEAK_GBS,
                              "bytes_per_step": self.bytes},
            "config": {"workload": "decode step, bs=1, 8K context (BASELINE config 5), "
                                   "62-layer random-init decoder, hipGraph per step",
                       "decode_mode": self.mode,
                       "n_layers": c.n_layers, "hidden": c.hidden, "ffn": c.ffn,
                       "n_q_heads": c.n_q_heads, "n_kv_heads": c.n_kv_heads, "head_dim": 128,
                       "vocab": c.vocab, "sliding_window": c.sliding_window,
                       "global_every": c.global_every, "context": self.context,
                       "weight_bytes": self.weight_bytes, "kv_bytes_read": self.kv_bytes},
        }


class DecodeReal:
    """One decode step at the released checkpoint's geometry (crates/sg-gguf/
    src/desc.rs:66-93): 60 layers, hidden 5376, ffn 21504, 32 query heads;
    sliding layers 16 kv heads of 256 (window 1024), every sixth layer global
    with 4 kv heads of 512 and K=V; the tied 262144-row head in Q6_K.  Random
    init, 8K context, decode mode 2 (the fused GEMVs around the any-geometry
    attention) or 3 (kernel per operator), replayed as a hipGraph.  Not a BASELINE config: the benchmark's config 5
    is `decode`."""

    kernel = "whole decode step (roofline over the step's algorithmic bytes)"

    def __init__(self, ctx, torch, context=8192, mode="fused"):
        import sgq

        self.ctx, self.torch = ctx, torch
        self.stream = torch.cuda.Stream()
        ctx.set_stream(self.stream)
        self.cfg = sgq.default_model_config(
            n_layers=60, global_every=6, sliding_window=1024, head_dim=256, head_dim_global=512,
            n_kv_heads=16, n_kv_heads_global=4, embed_q6k=1, max_ctx=16384)
        self.model = sgq.Model(ctx, self.cfg)
        self.mode = mode
        self.model.decode_mode = {"fused": 2, "kernels": 3}[mode]
        self.context = context
        self.model.fill_cache(context)
        self.logits = torch.empty(self.cfg.vocab, dtype=torch.float32, device="cuda")
        c = self.cfg
        H, F = c.hidden, c.ffn
        w = kv = 0
        for l in range(c.n_layers):
            glob = l % c.global_every == c.global_every - 1
            hd = c.head_dim_global if glob else c.head_dim
            QD, KD = c.n_q_heads * hd, (c.n_kv_heads_global if glob else c.n_kv_heads) * hd
            w += q4_bytes(QD, H) + q4_bytes(KD, H) * (1 if glob else 2) + q4_bytes(H, QD) \
                + 2 * q4_bytes(F, H) + q4_bytes(H, F)
            slots = context + 1 if glob else min(context + 1, c.sliding_window)
            kv += int(KD * (1 + 2 / 32) * 2 * slots)
        w += c.vocab * (H // 256) * 210
        self.weight_bytes, self.kv_bytes = w, kv
        self.bytes = w + kv
        self.rng = __import__("random").Random(5)

    def step(self, i):
        self.model.decode(self.rng.randrange(self.cfg.vocab), self.logits, graph=True)

    def result(self, ms_per_step):
        step_gbs = self.bytes / (ms_per_step * 1e-3) / 1e9
        c = self.cfg
        return {
            "value": 1000.0 / ms_per_step, "unit": "tok/s",
            "dtype": "q4_0 weights x i4-limb activations in every GEMV, q6_k head, q8_0 kv, "
                     "fp32 elsewhere",
            "roofline": {"bound": "hbm", "achieved": step_gbs, "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": step_gbs / HBM_PEAK_GBS, "traffic": None,
                         "bytes_per_step": self.bytes},
            "config": {"workload": "decode step, bs=1, 8K context, released-checkpoint geometry "
                                   "(60 layers, head_dim 256/512, 16/4 kv heads, Q6_K head), "
                                   "random init, hipGraph per step",
                       "decode_mode": self.mode,
                       "n_layers": c.n_layers, "hidden": c.hidden, "ffn": c.ffn,
                       "vocab": c.vocab, "context": self.context,
                       "weight_bytes": self.weight_bytes, "kv_bytes_read": self.kv_bytes},
        }


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "gemv_q4_0_ring_k5376_n21504_traffic.json")


def measured_traffic():
    """HBM bytes per launch of the streamed GEMV at K=5376, N=21504, from the
    committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes (scaled by a copy
    kernel of known size); None when that profile is absent."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            return json.load(f)["hbm_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def ring_roofline(ctx, torch, w_ptrs, k, n, steps=124, traffic=True):
    """The dominant kernel, gemv_q4_0_ring_kernel, alone at K x N: x limbs
    made once, then `steps` single-matrix launches rotating over w_ptrs (so
    each launch streams its weights from HBM), recorded once as a hipGraph
    and replayed with HIP events on the context's stream around the replay
    (back-to-back launches without host gaps).  Algorithmic bytes per
    launch: W (18 B per 32 weights) + the x limb table (80 B per 32 values)
    + y (fp32)."""
    import ctypes as C
    import sgq

    lib = sgq.lib()
    x = torch.empty(k, dtype=torch.float32, device="cuda")
    ctx.fill_normal(x, seed=3)
    xl = torch.empty(k // 32 * ctx.X_LIMBS_BYTES_PER_BLOCK, dtype=torch.uint8, device="cuda")
    ctx.x_limbs(x, xl, k)
    y = torch.empty(n, dtype=torch.float32, device="cuda")
    yp = (C.c_void_p * 1)(y.data_ptr())
    rows = (C.c_uint32 * 1)(n)

    def run(m):
        for j in range(m):
            wp = (C.c_void_p * 1)(w_ptrs[j % len(w_ptrs)])
            rc = lib.sgq_gemv_q4_0_limbs(ctx.handle, 1, wp, yp, rows, C.c_void_p(xl.data_ptr()),
                                         k, 0.0)
            assert rc == 0, sgq.lib().sgq_last_error()
    def full(m):  # the whole typed call: fp32 x in, the limbs built in the kernel
        for j in range(m):
            rc = lib.sgq_gemv_q4_0(ctx.handle, C.c_void_p(w_ptrs[j % len(w_ptrs)]),
                                   C.c_void_p(x.data_ptr()), C.c_void_p(y.data_ptr()), n, k)
            assert rc == 0, sgq.lib().sgq_last_error()

    def timed(fn):
        fn(len(w_ptrs))
        ctx.synchronize()
        with sgq.GraphRecorder(ctx) as rec:
            fn(steps)
        rec.graph.submit()  # warm replay
        ctx.synchronize()
        ctx.timer_start()
        rec.graph.submit()
        return ctx.timer_stop() / steps

    ms = timed(run)
    ms_full = timed(full)
    nbytes = q4_bytes(n, k) + (k // 32) * 80 + n * 4
    gbs = nbytes / (ms * 1e-3) / 1e9
    full_bytes = q4_bytes(n, k) + k * 4 + n * 4  # BASELINE's config-1 bytes (fp32 x in)
    full_gbs = full_bytes / (ms_full * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": gbs / HBM_PEAK_GBS, "traffic": measured_traffic() if traffic else None,
            "kernel": f"gemv_q4_0_ring_kernel K={k} N={n}", "bytes_per_launch": nbytes,
            "us_per_launch": ms * 1e3, "launches": steps,
            "full_call": {"what": "sgq_gemv_q4_0 (fp32 x; limbs built in the streamed kernel's prologue)",
                          "us_per_call": ms_full * 1e3, "achieved": full_gbs,
                          "frac": full_gbs / HBM_PEAK_GBS, "bytes_per_call": full_bytes}}


def measured_peaks(torch):
    """Roofline denominators measured on this box (libsgq_probe.so, no memory
    traffic for the MFMA probes): the dense int8 MFMA rate, the ceiling of an
    exact per-32-block rescale (16 cvt + 16 FMA per int8 MFMA, and with the
    f16 scale-product MFMA as the MMQ issues it), and a streaming HBM read of
    4 GiB.  Each is the best of 3 launches timed with HIP events on torch's
    current stream."""
    import ctypes as C

    path = os.path.join(ROOT, "super-gemma_amd", "sgq", "libsgq_probe.so")
    if not os.path.exists(path):
        return None
    P = C.CDLL(path)
    P.sgqp_mfma.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p]
    P.sgqp_mfma_count.restype = C.c_longlong
    P.sgqp_mfma_count.argtypes = [C.c_int, C.c_int, C.c_int]
    P.sgqp_hbm_read.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64, C.c_int, C.c_void_p]
    stream = torch.cuda.current_stream()
    sp = C.c_void_p(stream.cuda_stream)

    def best_ms(launch, reps=3):
        launch()
        best = None
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            launch()
            e1.record(stream)
            e1.synchronize()
            ms = e0.elapsed_time(e1)
            best = ms if best is None else min(best, ms)
        return best

    out = {}
    for label, mode, blocks, iters in (("int8_mfma", 0, 1024, 20000),
                                       ("int8_mfma_cvt_fma_ceiling", 1, 512, 20000),
                                       ("int8_mfma_cvt_fma_scale_mfma_ceiling", 2, 512, 20000)):
        buf = torch.empty(blocks * 256, dtype=torch.int32, device="cuda")
        ms = best_ms(lambda: P.sgqp_mfma(sp, mode, blocks, iters, C.c_void_p(buf.data_ptr())))
        ops = P.sgqp_mfma_count(mode, blocks, iters) * 2.0 * 32 * 32 * 32
        out[label + "_tops"] = ops / (ms * 1e-3) / 1e12
    nbytes = 4 << 30
    big = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    red = torch.empty(1024 * 256, dtype=torch.float32, device="cuda")
    ms = best_ms(lambda: P.sgqp_hbm_read(sp, C.c_void_p(big.data_ptr()), nbytes, 1024,
                                         C.c_void_p(red.data_ptr())))
    out["hbm_read_gbs"] = nbytes / (ms * 1e-3) / 1e9
    del big
    out["note"] = ("int8 MFMA 32x32x32 only (16 waves/CU); the same with 16 cvt + 16 FMA "
                   "per MFMA, and with the f16 scale MFMA (32x32x8) too (8 waves/CU, the MMQ's "
                   "occupancy); streaming read of 4 GiB (64 KB chunks, nontemporal 16-byte loads)")
    return out


def _time_reps(fn, budget_s):
    fn()  # warm
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        el = time.perf_counter() - t0
        if el > budget_s or reps >= 100000:
            return reps, el


def cpu_baseline(budget_s: float = 8.0):
    """Time the CPU restatement of CpuModel::matmul (dequant_row + 8-lane f64
    dot, row-parallel; reference.rs:402-475) on the host cores:
      - config 1 (GEMV K=5376, N=21504) at full size on min(16, host CPUs)
        threads, and on 1 thread;
      - configs 2 and 3 (the same matmul over M tokens, as the reference's
        CPU forward runs a prefill chunk) at reduced M, fitted as
        t(M) = a + b*M from two M values and extrapolated linearly to the
        configs' M (stated in the report)."""
    import numpy as np
    from oracle import oracle

    try:
        host_cpus = len(os.sched_getaffinity(0))
    except AttributeError:
        host_cpus = os.cpu_count() or 1
    threads = max(1, min(16, host_cpus))
    rng = oracle.Rng(0xBA5E)
    k, n = 5376, 21504
    w = rng.random_q4_0(n * k // 32)
    x = rng.f32_vec(k)
    reps, el = _time_reps(lambda: oracle.matmul_q4_0(w, x, 1, n, k, threads), budget_s)
    gbs = q4_bytes(n, k) * reps / el / 1e9
    reps1, el1 = _time_reps(lambda: oracle.matmul_q4_0(w, x, 1, n, k, 1), budget_s / 2)
    gbs1 = q4_bytes(n, k) * reps1 / el1 / 1e9

    def mmq_extrapolated(m_full, k_, n_, ms=(4, 16)):
        wq = rng.random_q4_0(n_ * k_ // 32)
        xs = rng.f32_vec(max(ms) * k_)
        t = []
        for m in ms:
            r, e = _time_reps(lambda: oracle.matmul_q4_0(wq, xs[:m * k_], m, n_, k_, threads),
                              budget_s / 4)
            t.append(e / r)
        b = (t[1] - t[0]) / (ms[1] - ms[0])
        a = t[0] - b * ms[0]
        t_full = a + b * m_full
        return {"m": m_full, "k": k_, "n": n_, "seconds": t_full,
                "tops": 2.0 * m_full * n_ * k_ / t_full / 1e12,
                "fit": f"t(M) = {a * 1e3:.1f} ms + {b * 1e3:.2f} ms * M from M = {ms[0]}, {ms[1]}"}

    return {"value": gbs, "unit": "GB/s", "cores": threads, "kind": "port",
            "host_cpus": host_cpus, "value_1_thread": gbs1,
            "sample": f"config 1 GEMV (K=5376, N=21504) full size: {reps} reps in {el:.1f} s on "
                      f"{threads} threads ({host_cpus} host CPUs), {reps1} reps in {el1:.1f} s on "
                      "1 thread; C restatement of reference.rs:402-444",
            "mmq_config2_extrapolated": mmq_extrapolated(512, 5376, 21504),
            "mmq_config3_extrapolated": mmq_extrapolated(2048, 21504, 5376)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--decode-mode", default="fused", choices=["kernels", "fused"],
                    help="decode workload: five fused launches per layer (default) or one "
                         "kernel per operator, each step replayed as a hipGraph")
    ap.add_argument("--workload", default="decode",
                    choices=["decode", "decode_real", "prefill_real", "prefill", "gemv", "mmq", "splitk", "attn_prefill",
                             "attn_prefill_ipv",
                             "attn_prefill_sliding", "attn_decode_4k", "attn_decode_32k",
                             "attn_decode_128k", "head_q6k", "attn_pages_sliding",
                             "attn_pages_q8k_4k", "attn_pages_q8k_8k", "attn_pages_q8k_32k",
                             "attn_prefill_pages_iq", "attn_prefill_pages_sliding"])
    ap.add_argument("--split-k", type=int, default=4, choices=[1, 2, 4, 8],
                    help="splitk workload: K split (BASELINE config 3 sweeps 1/2/4/8)")
    ap.add_argument("--gemv-rows", type=int, default=21504,
                    help="gemv workload: rows N (config 1 is 21504; other values sweep the "
                         "per-launch fixed cost against the streaming rate)")
    ap.add_argument("--mmq-m", type=int, default=512,
                    help="mmq / splitk workloads: M (512 keeps configs 2 and 3; other values sweep the tile rounds)")
    ap.add_argument("--gemv-k", type=int, default=5376,
                    help="gemv workload: K (config 1 is 5376; 21504 is the FFN down projection, "
                         "streamed as four K-slices)")
    ap.add_argument("--attn-splits", type=int, default=None,
                    help="attn_decode_* workloads: split count (default: 256 slots per split, "
                         "64..256 splits)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-peaks", action="store_true",
                    help="skip the measured MFMA / HBM peak probes")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus}: this build runs on one GPU only "
              "(no collectives, no multi-GPU path); use --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    import sgq

    ctx = sgq.GpuContext(0)
    if args.steps is None:
        args.steps = {"decode": 100, "decode_real": 50, "prefill": 5, "prefill_real": 3}.get(args.workload, 200)
    if args.warmup is None:
        args.warmup = {"decode": 10, "decode_real": 5, "prefill": 1, "prefill_real": 1}.get(args.workload, 20)
    if args.workload == "decode":
        wl = Decode(ctx, torch, mode=args.decode_mode)
    elif args.workload == "decode_real":
        wl = DecodeReal(ctx, torch, mode="kernels" if args.decode_mode == "kernels" else "fused")
    elif args.workload == "prefill":
        wl = Prefill(ctx, torch)
    elif args.workload == "prefill_real":
        wl = Prefill(ctx, torch, real=True)
    elif args.workload == "gemv":
        wl = Gemv(ctx, torch, n=args.gemv_rows, k=args.gemv_k)
    elif args.workload == "mmq":
        wl = (Mmq(ctx, torch) if args.mmq_m == 512 else
              Mmq(ctx, torch, m=args.mmq_m, label="M sweep around BASELINE config 2"))
    elif args.workload == "head_q6k":
        wl = HeadQ6K(ctx, torch)
    elif args.workload == "attn_prefill":
        wl = AttnPrefill(ctx, torch)
    elif args.workload == "attn_prefill_ipv":
        wl = AttnPrefill(ctx, torch, ipv=True)
    elif args.workload == "attn_prefill_sliding":
        wl = AttnPrefill(ctx, torch, window=1024)
    elif args.workload == "attn_prefill_pages_iq":
        wl = AttnPrefillPages(ctx, torch, "global_flash_sp_iq")
    elif args.workload == "attn_prefill_pages_sliding":
        wl = AttnPrefillPages(ctx, torch, "sliding_ring")
    elif args.workload == "attn_pages_sliding":
        wl = AttnPages(ctx, torch, "sliding", 1024)
    elif args.workload.startswith("attn_pages_q8k_"):
        wl = AttnPages(ctx, torch, "global_q8k",
                       {"4k": 4096, "8k": 8192, "32k": 32768}[args.workload[15:]])
    elif args.workload.startswith("attn_decode_"):
        wl = AttnDecode(ctx, torch, {"4k": 4096, "32k": 32768, "128k": 131072}[args.workload[12:]],
                        splits=args.attn_splits)
    else:
        wl = (Mmq(ctx, torch, m=2048, k=21504, n=5376, split=args.split_k, label="BASELINE config 3")
              if args.mmq_m == 512 else
              Mmq(ctx, torch, m=args.mmq_m, k=21504, n=5376, split=args.split_k,
                  label="M sweep around BASELINE config 3"))
    torch.cuda.synchronize()
    for i in range(args.warmup):
        wl.step(i)
    torch.cuda.synchronize()
    ctx.timer_start()
    for i in range(args.steps):
        wl.step(i)
    ms_total = ctx.timer_stop()
    torch.cuda.synchronize()
    ctx.synchronize()
    ms = ms_total / args.steps
    res = wl.result(ms)
    out = {
        "metric": METRIC,
        "value": res["value"],
        "unit": res["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": res["dtype"],
        "data": "synthetic (device-generated, seeded)",
        "config": res["config"],
        "roofline": res["roofline"],
        **({"step_roofline": res["step_roofline"]} if "step_roofline" in res else {}),
        **({"whole_prefill_rate": res["whole_prefill_rate"]} if "whole_prefill_rate" in res
           else {}),
        "kernel": wl.kernel,
    }
    if not args.no_peaks:
        out["measured_peaks"] = measured_peaks(torch)
        if out["measured_peaks"] and out["roofline"].get("unit") == "TOP/s":
            mp = out["measured_peaks"]
            a = out["roofline"]["achieved"]
            out["roofline"]["frac_of_measured_int8_peak"] = a / mp["int8_mfma_tops"]
            out["roofline"]["frac_of_rescale_ceiling"] = a / mp["int8_mfma_cvt_fma_scale_mfma_ceiling_tops"]
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
