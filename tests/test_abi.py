"""The C-ABI library loads, exports every function include/frx_ternary.h
declares, and reports errors as statuses (no compute calls: CPU-only)."""
import ctypes
import os
import re

import ferrisres_amd as frx

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "frx_ternary.h")


def _declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(frx_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_expected_entry_points():
    names = _declared()
    for must in ["frx_create", "frx_ternary_linear", "frx_ternary_linear_bias", "frx_sparse24_ternary_linear", "frx_moe_ternary_ffn",
                 "frx_ternary_glu", "frx_ternary_ffn", "frx_set_ffn_mode", "frx_upload_ternary", "frx_upload_stm",
                 "frx_sparse24_cpu_to_gpu_device", "frx_free",
                 "frx_pack_ternary_u8", "frx_repack_u8_to_u32", "frx_pack_sparse24_gpu",
                 "frx_sparse24_cpu_to_gpu", "frx_gpu_ternary_matmul", "frx_gpu_ternary_matmul_vram",
                 "frx_gpu_sparse_ternary_matmul"]:
        assert must in names


def test_library_exports_every_declared_symbol():
    h = ctypes.CDLL(frx.LIB_PATH)
    missing = [n for n in _declared() if not hasattr(h, n)]
    assert not missing, missing
    assert set(_declared()) == set(frx.exported_symbols())


def test_version_and_status_strings():
    lib = frx.lib()
    assert lib.frx_version().decode().startswith("frx_ternary")
    assert lib.frx_status_string(0).decode() == "ok"
    assert lib.frx_status_string(2).decode() == "shape error"
    assert lib.frx_last_error(None).decode() == ""


def test_null_context_is_a_device_error_not_a_crash():
    lib = frx.lib()
    st = lib.frx_ternary_linear(None, None, None, None, 0, None, 0, 1, 16, 1)
    assert st == 3  # FRX_ERR_DEVICE
    assert lib.frx_synchronize(None) == 3


def test_create_without_gpu_fails_cleanly():
    # On a machine without a gfx950 device, context creation must return a
    # status (the caller then falls back, as cpu_block_attn_res.rs:1004-1031).
    import torch
    if torch.cuda.is_available():
        return
    h = ctypes.c_void_p()
    st = frx.lib().frx_create(0, ctypes.byref(h))
    assert st in (3, 6) and not h.value
