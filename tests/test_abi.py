"""The C-ABI library loads on a host without a GPU and exports every entry point that
include/hx/exl3.h declares (no compute calls here)."""
import ctypes
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def declared_symbols():
    text = (ROOT / "include" / "hx" / "exl3.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hx_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    for need in ("hx_exl3_gemm", "hx_exl3_reconstruct_slice", "hx_routing_ds3_nogroup", "hx_moe_permute",
                 "hx_moe_reduce_sorted", "hx_swiglu_clamp", "hx_had_r_128"):
        assert need in syms


def test_library_exports_every_declared_symbol():
    from helios_glm53flash_amd import _lib
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_python_binding_covers_header():
    from helios_glm53flash_amd import _lib
    assert set(declared_symbols()) <= set(_lib.SIGNATURES)


def test_host_side_validation_without_gpu():
    """Argument checks run on the host and report through hx_last_error (nothing is launched)."""
    from helios_glm53flash_amd import _lib
    gw = _lib.GroupWordsC(1, 1, 1, 0)
    r = _lib.lib.hx_exl3_gemm(1, 1, ctypes.byref(gw), 1, 100, 128, 2, 1, None, None, 0, None, 0)
    assert r == _lib.HX_ERR_INVALID and b"multiples of 128" in _lib.lib.hx_last_error()
    r = _lib.lib.hx_exl3_gemm(1, 1, ctypes.byref(gw), 1, 128, 128, 2, 1, None, None, 0, None, 0)
    assert r == _lib.HX_ERR_WORKSPACE
    r = _lib.lib.hx_routing_ds3_nogroup(1, None, 1, 1, 1, 288, 8, 2.5, 1, 2, None)
    assert r == _lib.HX_ERR_UNSUPPORTED
    assert _lib.lib.hx_exl3_gemm_workspace_size(1, 2048, 4096) > 0
    # a shared expert whose codebook differs from the layer's (mul1 layer, mul1 = 0 shared words)
    tabs = _lib.ExpertTablesC(*([1] * 9), None, None, None, 0)
    sh = (_lib.GroupWordsC * 3)(*[_lib.GroupWordsC(1, 1, 1, 0) for _ in range(3)])
    shb = (ctypes.c_int * 3)(2, 2, 2)
    r = _lib.lib.hx_moe_layer(1, None, 1, 1, None, ctypes.byref(tabs), sh, shb, 1, 4096, 2048, 288, 8, 2, 2, 2,
                              2.5, 10.0, 0, 1, None, 0, None)
    assert r == _lib.HX_ERR_INVALID and b"codebook" in _lib.lib.hx_last_error()


def test_cpp_compat_header_compiles_and_links(tmp_path):
    """include/helios/exl3_compat.hpp (reference-signature C++ layer) compiles with hipcc and
    links against the library; nothing is executed."""
    import shutil
    import subprocess
    from helios_glm53flash_amd import _lib
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    src = tmp_path / "t.cpp"
    src.write_text('#include "helios/exl3_compat.hpp"\n#include <hip/hip_fp16.h>\n'
                   "int main(int argc, char**) {\n"
                   "  if (argc > 5) {\n"
                   "    // the dense-MoE fallback's call sites (runner.cpp:902-907) with the engine's half types\n"
                   "    const half* x = nullptr; half* dense_x = nullptr; const half* wsorted = nullptr;\n"
                   "    const int64_t* idx = nullptr; float* y = nullptr; const float* dense_d = nullptr;\n"
                   "    helios::glue::gather_rows(x, idx, dense_x, 4, 4096, nullptr);\n"
                   "    helios::glue::scatter_add_rows(y, dense_d, idx, wsorted, 4, 4096, nullptr);\n"
                   "    helios::exl3::ExpertTables t{};\n"
                   "    helios::exl3::moe_layer(nullptr, nullptr, nullptr, nullptr, nullptr, t, nullptr, nullptr, 1, 4096,"
                   " 2048, 288, 8, 2, 2, 2, 2.5f);\n"
                   "    helios::exl3::GroupWords w{nullptr, nullptr, nullptr, 0};\n"
                   "    helios::exl3::gemm(nullptr, nullptr, w, 1, 128, 128, 2);\n"
                   "    helios::glue::moe_permute(nullptr, nullptr, 1, 8, 288, nullptr, nullptr, nullptr, nullptr);\n"
                   "    helios::glue::gemm_nt_f16(nullptr, nullptr, nullptr, 1, 288, 4096, false, false);\n"
                   "    helios::exl3::pack_trellis(nullptr, nullptr, 1, 1, 2);\n"
                   "    (void)helios::exl3::moe_max_concurrency(0);\n"
                   "    helios::aux::routing_ds3_nogroup_hidden(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 4096, 288, 8, 2.5f,"
                   " helios::aux::ROUTING_ACT_SIGMOID);\n"
                   "    helios::exl3::had_r_128(nullptr, nullptr, nullptr, nullptr, 1, 128, helios::exl3::DType::Half, 1.0f);\n"
                   "    helios::exl3::had_r_128_dual(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 1, 128,"
                   " helios::exl3::DType::Float, 1.0f, nullptr);\n"
                   "    helios::exl3::reconstruct_had_slice(nullptr, nullptr, nullptr, nullptr, 8, 8, 128, 128, 2, false, true, 0);\n"
                   "    helios::exl3::pack_signs(nullptr, nullptr, 0);\n"
                   "    unsigned long long* cnt = nullptr;\n"
                   "    helios::exl3::count_inf_nan(nullptr, cnt, 0, helios::exl3::DType::Half);\n"
                   "  }\n  return 0;\n}\n")
    lib = Path(_lib.LIB_PATH)
    r = subprocess.run([hipcc, "-std=c++17", "-Werror", "-I", str(ROOT / "include"), str(src), "-o",
                        str(tmp_path / "t"), "-L", str(lib.parent), "-lhx_exl3", f"-Wl,-rpath,{lib.parent}"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]


def test_moe_layer_codebook_checks_without_gpu():
    """MoeLayer refuses mcg=True over mul1 experts, and a shared expert whose codebook differs from
    the routed experts' (the layer decodes both with one codebook); host checks only."""
    import pytest
    import torch
    from helios_glm53flash_amd import exl3, moe
    E, hidden, inter = 2, 128, 128

    def group(K, N, mul1):
        return exl3.GroupWords(torch.zeros((K // 16, N // 16, 32), dtype=torch.int16),
                               torch.ones(K, dtype=torch.float16), torch.ones(N, dtype=torch.float16), mul1)

    def experts(mul1):
        shapes = [(hidden, inter), (hidden, inter), (inter, hidden)]
        gw = [[group(K, N, 0) for _ in range(E)] for K, N in shapes]
        return moe.ExpertSet(hidden, inter, [[w.trellis for w in p] for p in gw], [[w.suh for w in p] for p in gw],
                             [[w.svh for w in p] for p in gw], [[2] * E for _ in range(3)], mul1)

    sh_mul1 = [group(hidden, inter, exl3.MUL1), group(hidden, inter, exl3.MUL1), group(inter, hidden, exl3.MUL1)]
    sh_mcg = [group(hidden, inter, 0), group(hidden, inter, 0), group(inter, hidden, 0)]
    moe.MoeLayer(experts(True), sh_mul1, topk=2)
    moe.MoeLayer(experts(False), sh_mcg, topk=2, mcg=True)
    with pytest.raises(ValueError):
        moe.MoeLayer(experts(True), None, topk=2, mcg=True)
    with pytest.raises(ValueError):
        moe.MoeLayer(experts(True), sh_mcg, topk=2)
    with pytest.raises(ValueError):
        moe.MoeLayer(experts(False), sh_mul1, topk=2, mcg=True)
