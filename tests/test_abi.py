"""CPU checks of the C ABI: libsgq.so loads, exports exactly what
include/sgq.h declares, and the host-side validation paths fail loudly.
No compute runs here (no GPU in this container)."""
import ctypes as C
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sgq.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sgq_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    import sgq

    assert os.path.exists(sgq.LIB_PATH), "libsgq.so not built"
    L = C.CDLL(sgq.LIB_PATH)
    syms = declared_symbols()
    assert len(syms) >= 20
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, f"declared but not exported: {missing}"
    # the Python mirror binds every declared symbol with a signature
    assert set(syms) == set(sgq.SIGNATURES), set(syms) ^ set(sgq.SIGNATURES)


def test_exports_are_c_abi_and_gfx950_only():
    import sgq

    out = subprocess.run(["nm", "-D", "--defined-only", sgq.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    assert all(s in exported for s in declared_symbols())
    # code objects: gfx950 only
    blob = open(sgq.LIB_PATH, "rb").read()
    assert b"gfx950" in blob
    for other in (b"gfx942", b"gfx90a", b"gfx1100"):
        assert other not in blob


def test_registry_names_resolve_without_device():
    import sgq

    L = sgq.lib()
    names = [L.sgq_kernel_name(i).decode() for i in range(L.sgq_kernel_count())]
    assert "gemv_q4_0_k5376" in names and "kv_quant_q8" in names
    assert "gemm_q4_0_i8_swz_m4n1_k5376_n21504" in names and "gemm_q4_0_i8_bb_pfd4" in names
    for n in names:
        h = C.c_void_p()
        info = sgq._Info()
        rc = L.sgq_kernel_lookup(None, n.encode(), C.byref(h), C.byref(info))
        assert rc == 0, (n, L.sgq_last_error())
        assert info.bindings >= 2
    # binding / push layouts of the reference's variants (crates/sg-gpu/build.rs:64-190)
    want = {"rmsnorm_5376": (3, 0, 256), "rmsnorm_256_plus1": (3, 0, 256),
            "rope_sliding_q": (2, 0, 256), "rope_global_k": (2, 0, 256),
            "geglu": (3, 0, 256), "add_scaled": (3, 4, 256)}
    for n, (nb, pb, wg) in want.items():
        info = sgq._Info()
        assert L.sgq_kernel_lookup(None, n.encode(), C.byref(h), C.byref(info)) == 0
        assert (info.bindings, info.push_bytes, info.workgroup[0]) == (nb, pb, wg), n
    rc = L.sgq_kernel_lookup(None, b"gemv_q6_k_logits_nonexistent", C.byref(h), C.byref(info))
    assert rc == 4 and b"unknown kernel" in L.sgq_last_error()


def test_attention_variants_layouts_and_unbuilt_names():
    """The record_layer attention / KV-append surface (crates/sg-model/src/
    graph.rs:560-656): head_dim 128 with Q8_0 K/V, and the real checkpoint's
    decode side over f16 pages with the reference's binding and push layout
    (crates/sg-gpu/build.rs:255-438, :2206-2335); a name outside the
    registry fails with UnknownKernel."""
    import sgq

    L = sgq.lib()
    h = C.c_void_p()
    info = sgq._Info()
    want = {"kv_append_global_q8": (4, 0), "kv_append_sliding_q8": (4, 0),
            "attn_decode_global_q8_hd128": (7, 8), "attn_decode_sliding_q8_hd128": (7, 8),
            "attn_reduce_d128": (2, 4), "attn_prefill_global_flash_q8_hd128": (7, 4),
            "attn_prefill_sliding_ring_q8_hd128": (11, 4),
            "attn_decode_sliding": (5, 8), "attn_decode_global": (5, 8),
            "attn_decode_global_q8k": (6, 8), "attn_reduce_d256": (2, 4),
            "attn_reduce_d512": (2, 4), "kv_append_sliding": (3, 0), "kv_append_global": (3, 0),
            "attn_prefill_sliding": (5, 4), "attn_prefill_sliding_ring": (7, 4),
            "attn_prefill_global": (5, 4), "attn_prefill_global_flash": (5, 4),
            "attn_prefill_global_flash_sp": (5, 4), "attn_prefill_global_flash_sp_q8": (7, 4),
            "attn_prefill_global_flash_sp_iq": (7, 4), "attn_prefill_global_flash_sp_ipv": (8, 4),
            "attn_prefill_global_flash_sp_ipv_bcast": (8, 4)}
    for n, (nb, pb) in want.items():
        assert L.sgq_kernel_lookup(None, n.encode(), C.byref(h), C.byref(info)) == 0, n
        assert (info.bindings, info.push_bytes) == (nb, pb), n
    rc = L.sgq_kernel_lookup(None, b"attn_prefill_global_flash_sp_ipv_hd64", C.byref(h),
                             C.byref(info))
    assert rc == 4 and b"unknown kernel" in L.sgq_last_error()


def test_ctx_create_without_device_reports_no_device():
    import torch
    import sgq

    if torch.cuda.is_available():
        pytest.skip("device present")
    h = C.c_void_p()
    rc = sgq.lib().sgq_ctx_create(0, C.byref(h))
    assert rc == 3  # NoDevice: callers skip, as GpuContext::new's error does
    with pytest.raises(sgq.NoDevice):
        sgq.GpuContext(0)


# Every variant the reference's model loads (crates/sg-model/src/graph.rs,
# GraphKernels::load: its load("...") calls).
MODEL_VARIANTS = [
    "add_scaled", "attn_decode_global_q8k", "attn_decode_sliding",
    "attn_prefill_global_flash_sp_iq", "attn_prefill_sliding_ring", "attn_reduce_d256",
    "attn_reduce_d512", "geglu", "gemm_q4_0_i8_bb_pfd4", "gemm_q4_0_i8_swz_m4n1_k5376_n16384",
    "gemm_q4_0_i8_swz_m4n1_k5376_n2048", "gemm_q4_0_i8_swz_m4n1_k5376_n21504",
    "gemm_q4_0_i8_swz_m4n1_k5376_n4096", "gemm_q4_0_i8_swz_m4n1_k5376_n8192",
    "gemm_q4_0_i8_swz_m4n1_k8192_n5376", "gemm_q4_0_i8_swz_m4n1_s1_k16384_n5376",
    "gemv_q4_0_k16384", "gemv_q4_0_k21504", "gemv_q4_0_k5376", "gemv_q4_0_k8192",
    "gemv_q6_k_logits", "kv_append_global", "kv_append_global_q8", "kv_append_sliding",
    "kv_quant_q8", "rmsnorm_256", "rmsnorm_512", "rmsnorm_5376", "rope_global_k",
    "rope_global_q", "rope_sliding_k", "rope_sliding_q",
]


def test_every_variant_the_reference_model_loads_resolves():
    import sgq

    L = sgq.lib()
    h = C.c_void_p()
    info = sgq._Info()
    for n in MODEL_VARIANTS:
        rc = L.sgq_kernel_lookup(None, n.encode(), C.byref(h), C.byref(info))
        assert rc == 0, (n, L.sgq_last_error())


def test_f32_suffix_forms_resolve():
    """The reference's names take f16 activations; NAME_f32 is the same
    kernel over fp32 and has the same binding / push layout.  The families
    of this build's own geometry take fp32 only and refuse the suffix."""
    import sgq

    L = sgq.lib()
    h = C.c_void_p()
    for n in ("gemv_q4_0_k5376", "gemv_q4_0_generic", "gemv_q6_k_logits", "rmsnorm_5376_plus1",
              "rope_sliding_q", "rope_global_k", "geglu", "add_scaled", "kv_quant_q8",
              "kv_dequant_q8", "kv_append_global_q8", "kv_append_global_v_q8",
              "gemm_q4_0_i8_swz_m4n1_k5376_n21504", "gemm_q4_0_i8_bb_pfd4"):
        a, b = sgq._Info(), sgq._Info()
        assert L.sgq_kernel_lookup(None, n.encode(), C.byref(h), C.byref(a)) == 0, n
        assert L.sgq_kernel_lookup(None, (n + "_f32").encode(), C.byref(h), C.byref(b)) == 0, n
        assert (a.bindings, a.push_bytes, list(a.workgroup)) == \
            (b.bindings, b.push_bytes, list(b.workgroup)), n
    for n in ("rope_hd128_sliding_q", "kv_append_sliding_q8", "attn_reduce_d128",
              "attn_decode_global_q8_hd128", "gemm_q4_0_i8_splitk4_k21504_n5376",
              "attn_decode_sliding", "kv_append_global"):
        info = sgq._Info()
        assert L.sgq_kernel_lookup(None, n.encode(), C.byref(h), C.byref(info)) == 0, n
        rc = L.sgq_kernel_lookup(None, (n + "_f32").encode(), C.byref(h), C.byref(info))
        assert rc == 4, n
