"""ctypes binding of libhx_exl3.so (the C ABI declared in include/hx/exl3.h).

The library is the product path: nothing here falls back to another implementation.  When the
shared object is missing the import of this module raises, naming the build command.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

_PKG = Path(__file__).resolve().parent
LIB_PATH = _PKG / "libhx_exl3.so"  # the in-tree build only: no override, so a stale copy cannot load

HX_ERR_INVALID = -1
HX_ERR_WORKSPACE = -2
HX_ERR_HIP = -3
HX_ERR_UNSUPPORTED = -4
HX_ERR_TIMEOUT = -5
HX_GEMM_PATH_MFMA = 1
HX_GEMM_PATH_GEMV = 90


class GroupWordsC(C.Structure):
    _fields_ = [("trellis", C.c_void_p), ("suh", C.c_void_p), ("svh", C.c_void_p), ("mul1", C.c_int)]


class ExpertTablesC(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in (
        "gate_trellis", "gate_suh", "gate_svh", "up_trellis", "up_suh", "up_svh",
        "down_trellis", "down_suh", "down_svh", "gate_bits", "up_bits", "down_bits")] + [("bits_mask", C.c_uint32)]


class ExpertLayoutC(C.Structure):
    _fields_ = [("off", C.c_uint64 * 12), ("piece", C.c_uint64 * 12), ("bits", C.c_int * 3), ("stride", C.c_uint64)]


# name -> (restype, argtypes); the exported symbol set is exactly the declarations of exl3.h
SIGNATURES: dict[str, tuple] = {
    "hx_version": (C.c_char_p, []),
    "hx_last_error": (C.c_char_p, []),
    "hx_workspace_init": (C.c_int, [C.c_void_p, C.c_size_t, C.c_void_p]),
    "hx_profile_enable": (C.c_int, [C.c_int]),
    "hx_profile_read": (C.c_int, [C.POINTER(C.c_double), C.POINTER(C.c_int), C.c_int]),
    "hx_profile_phase_name": (C.c_char_p, [C.c_int]),
    "hx_exl3_gemm_workspace_size": (C.c_size_t, [C.c_int, C.c_int, C.c_int]),
    "hx_exl3_gemm": (C.c_int, [C.c_void_p, C.c_void_p, C.POINTER(GroupWordsC), C.c_int, C.c_int, C.c_int, C.c_int,
                               C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_size_t]),
    "hx_exl3_gemm_noalloc_max_bytes": (C.c_size_t, []),
    "hx_exl3_gemm_noalloc": (C.c_int, [C.c_void_p, C.c_void_p, C.POINTER(GroupWordsC), C.c_int, C.c_int, C.c_int,
                                       C.c_int, C.c_int, C.c_void_p, C.c_int]),
    "hx_exl3_reconstruct_slice": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                            C.c_int, C.c_int64, C.c_void_p]),
    "hx_had_r_128": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64, C.c_int, C.c_int,
                               C.c_float, C.c_void_p]),
    "hx_had_r_128_dual": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                    C.c_void_p, C.c_void_p, C.c_int64, C.c_int, C.c_int, C.c_float, C.c_void_p]),
    "hx_routing_ds3_nogroup": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int,
                                         C.c_float, C.c_int, C.c_int, C.c_void_p]),
    "hx_routing_gemv": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p]),
    "hx_routing_ds3_nogroup_hidden": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                                C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_float, C.c_int,
                                                C.c_void_p]),
    "hx_moe_permute": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p,
                                 C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]),
    "hx_moe_reduce_sorted": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p]),
    "hx_swiglu_clamp": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t, C.c_float, C.c_void_p]),
    "hx_exl3_reconstruct_had_slice": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int,
                                                C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int64, C.c_void_p]),
    "hx_exl3_pack_trellis": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p]),
    "hx_exl3_unpack_trellis": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p]),
    "hx_pack_signs": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_void_p]),
    "hx_count_inf_nan": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64, C.c_int, C.c_void_p]),
    "hx_moe_check_status": (C.c_int, [C.c_void_p, C.c_void_p]),
    "hx_moe_max_concurrency": (C.c_int, [C.c_int]),
    "hx_gemm_nt_f16": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                 C.c_void_p]),
    "hx_gather_rows": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p]),
    "hx_scatter_add_rows": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p]),
    "hx_ckpt_open": (C.c_int, [C.c_char_p, C.POINTER(C.c_void_p)]),
    "hx_ckpt_close": (None, [C.c_void_p]),
    "hx_ckpt_tensor_count": (C.c_int, [C.c_void_p]),
    "hx_ckpt_tensor_info": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_int), C.POINTER(C.c_int64), C.c_int,
                                      C.POINTER(C.c_int), C.POINTER(C.c_uint64)]),
    "hx_ckpt_read": (C.c_int, [C.c_void_p, C.c_char_p, C.c_void_p, C.c_uint64]),
    "hx_ckpt_expert_layout": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(ExpertLayoutC)]),
    "hx_ckpt_load_experts": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.POINTER(ExpertLayoutC), C.c_void_p,
                                       C.c_size_t, C.c_int, C.c_void_p]),
    "hx_ckpt_expert_tables": (C.c_int, [C.POINTER(ExpertLayoutC), C.c_void_p, C.c_int, C.c_void_p,
                                        C.POINTER(ExpertTablesC), C.c_void_p]),
    "hx_moe_workspace_size": (C.c_size_t, [C.c_int] * 5),
    "hx_moe_grouped": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                 C.c_void_p, C.c_void_p, C.POINTER(ExpertTablesC)] + [C.c_int] * 12 +
                       [C.c_float, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t]),
    "hx_moe_layer": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.POINTER(ExpertTablesC),
                               C.POINTER(GroupWordsC), C.POINTER(C.c_int)] + [C.c_int] * 8 +
                     [C.c_float, C.c_float, C.c_int, C.c_int, C.c_void_p, C.c_size_t, C.c_void_p]),
}


def _load() -> C.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is not built; run `python -m helios_glm53flash_amd.build` (hipcc, gfx950)")
    lib = C.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


class HxError(RuntimeError):
    pass


def check(code: int, what: str) -> int:
    if code < 0:
        raise HxError(f"{what} failed ({code}): {lib.hx_last_error().decode()}")
    return code
