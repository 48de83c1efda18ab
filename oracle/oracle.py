"""ctypes wrapper of liboracle.so (oracle/exl3_oracle.c).

TEST INFRASTRUCTURE ONLY: the CPU checker and the CPU baseline.  Importable by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg; the product package never imports it.
All arrays are numpy arrays; fp16 data is passed as uint16 bit patterns (np.float16 views work).
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def _load() -> C.CDLL:
    if not LIB_PATH.exists():
        build()
    return C.CDLL(str(LIB_PATH))


_lib = _load()
P = C.c_void_p


def _sig(name, res, args):
    f = getattr(_lib, name)
    f.restype = res
    f.argtypes = args
    return f


_h2d = _sig("hx_or_h2d", C.c_double, [C.c_uint16])
_d2h = _sig("hx_or_d2h", C.c_uint16, [C.c_double])
_window = _sig("hx_or_window", C.c_uint32, [P, C.c_int, C.c_int])
_decode = _sig("hx_or_decode", C.c_uint16, [C.c_int, C.c_uint32])
_table = _sig("hx_or_codebook_table", None, [C.c_int, P])
_pack = _sig("hx_or_pack_tile", None, [P, C.c_int, P])
_unpack = _sig("hx_or_unpack_tile", None, [P, C.c_int, P])
_recon = _sig("hx_or_reconstruct", None, [P, P, C.c_int, C.c_int, C.c_int, C.c_int])
_had = _sig("hx_or_had128", None, [P, C.c_long])
_had16 = _sig("hx_or_had_r_128_f16", None, [P, P, C.c_long, C.c_long, P, P, C.c_double])
_linear = _sig("hx_or_linear", None, [P, P, C.c_int, C.c_int, C.c_int, P, P, P, C.c_int, C.c_int, C.c_int])
_routing = _sig("hx_or_routing", None, [P, P, P, P, C.c_int, C.c_int, C.c_int, C.c_double])
_routing2 = _sig("hx_or_routing2", None, [P, P, P, P, C.c_int, C.c_int, C.c_int, C.c_double, C.c_int, C.c_int])
_permute = _sig("hx_or_permute", None, [P, P, C.c_int, C.c_int, C.c_int, P, P, P, P])
_reduce = _sig("hx_or_reduce_sorted", None, [P, P, P, C.c_int, C.c_int, C.c_int])
_swiglu = _sig("hx_or_swiglu_clamp", None, [P, P, P, C.c_long, C.c_float])
_moe = _sig("hx_or_moe_rows", None, [P, P, P, C.c_int, C.c_int, P, P, C.c_int, P, C.c_int, P, P, C.c_float, C.c_int])
_cpu_linear = _sig("hx_cpu_linear_f32", C.c_double, [P, P, C.c_int, C.c_int, C.c_int, P, P, P, C.c_int, C.c_int,
                                                      C.c_int])
_cpu_threads = _sig("hx_cpu_max_threads", C.c_int, [])


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "arrays must be C-contiguous"
    return a.ctypes.data


def _u16(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a)
    if a.dtype in (np.float16, np.int16):
        a = a.view(np.uint16)
    assert a.dtype == np.uint16
    return a


def h2d(h: int) -> float:
    return _h2d(h)


def d2h(v: float) -> int:
    return _d2h(v)


def window(tile: np.ndarray, bits: int, p: int) -> int:
    return _window(_p(_u16(tile)), bits, p)


def decode(cb: int, w: int) -> int:
    return _decode(cb, w)


def codebook_table(cb: int) -> np.ndarray:
    out = np.empty(65536, np.uint16)
    _table(cb, _p(out))
    return out


def pack_tile(sym: np.ndarray, bits: int) -> np.ndarray:
    out = np.empty(16 * bits, np.uint16)
    _pack(_p(_u16(sym.astype(np.uint16))), bits, _p(out))
    return out


def unpack_tile(tile: np.ndarray, bits: int) -> np.ndarray:
    out = np.empty(256, np.uint16)
    _unpack(_p(_u16(tile)), bits, _p(out))
    return out


def reconstruct(trellis: np.ndarray, K: int, N: int, bits: int, cb: int) -> np.ndarray:
    """W_hat fp16 [K][N] as uint16 bit patterns."""
    out = np.empty((K, N), np.uint16)
    _recon(_p(out), _p(_u16(trellis)), K, N, bits, cb)
    return out


def had128(v: np.ndarray) -> np.ndarray:
    v = np.ascontiguousarray(v, dtype=np.float64).copy()
    _had(_p(v), v.size)
    return v


def had_r_128_f16(x: np.ndarray, pre=None, post=None, r_scale: float = 0.088388347648) -> np.ndarray:
    x = _u16(x)
    out = np.empty_like(x)
    rows, cols = x.shape
    _had16(_p(out), _p(x), rows, cols, _p(None if pre is None else _u16(pre)),
           _p(None if post is None else _u16(post)), r_scale)
    return out


def linear(x: np.ndarray, trellis: np.ndarray, suh: np.ndarray, svh: np.ndarray, K: int, N: int, bits: int, cb: int,
           out_f16: bool = False) -> np.ndarray:
    """fp64 y [M][N] (out_f16: values already rounded to fp16)."""
    x = _u16(x)
    M = x.size // K
    y = np.empty((M, N), np.float64)
    _linear(_p(y), _p(x), M, K, N, _p(_u16(trellis)), _p(_u16(suh)), _p(_u16(svh)), bits, cb, int(out_f16))
    return y


def routing(scores: np.ndarray, K: int, scale: float, bias: np.ndarray | None = None, use_topk: bool = True,
            act_fn: int = 0):
    """act_fn 0 = sigmoid, 1 = sqrt(softplus); use_topk False = the sorting variant (routing.cu:333-443)."""
    s = _u16(scores)
    bsz, E = s.shape
    idx = np.empty((bsz, K), np.int64)
    w = np.empty((bsz, K), np.uint16)
    b = None if bias is None else _u16(bias)
    if use_topk and act_fn == 0:
        _routing(_p(s), _p(b), _p(idx), _p(w), bsz, E, K, scale)
    else:
        _routing2(_p(s), _p(b), _p(idx), _p(w), bsz, E, K, scale, int(use_topk), act_fn)
    return idx, w


def permute(ids: np.ndarray, w: np.ndarray, E: int):
    ids = np.ascontiguousarray(ids, np.int64)
    M, topk = ids.shape
    cnt = np.empty(E + 1, np.int64)
    ts = np.empty(M * topk, np.int64)
    ws = np.empty(M * topk, np.uint16)
    r2s = np.empty(M * topk, np.int64)
    _permute(_p(ids), _p(_u16(w)), M, topk, E, _p(cnt), _p(ts), _p(ws), _p(r2s))
    return cnt, ts, ws, r2s


def reduce_sorted(contrib: np.ndarray, r2s: np.ndarray, M: int, topk: int) -> np.ndarray:
    contrib = np.ascontiguousarray(contrib, np.float32)
    hidden = contrib.shape[-1]
    y = np.empty((M, hidden), np.float32)
    _reduce(_p(y), _p(contrib), _p(np.ascontiguousarray(r2s, np.int64)), M, topk, hidden)
    return y


def swiglu_clamp(g: np.ndarray, u: np.ndarray, limit: float) -> np.ndarray:
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    out = np.empty(g.size, np.uint16)
    _swiglu(_p(g), _p(u), _p(out), g.size, limit)
    return out


class _Experts(C.Structure):
    _fields_ = [("trellis", P * 3), ("suh", P * 3), ("svh", P * 3), ("bits", P * 3), ("cb", C.c_int)]


class _Dense(C.Structure):
    _fields_ = [("trellis", P * 3), ("suh", P * 3), ("svh", P * 3), ("bits", C.c_int * 3), ("cb", C.c_int)]


def moe_rows(x: np.ndarray, hidden: int, inter: int, topk_idx: np.ndarray, topk_w: np.ndarray, rows,
             experts: dict, shared: dict | None, act_limit: float, cb: int = 2, act: int = 0):
    """experts: {"trellis": [gate_list, up_list, down_list], "suh": [...], "svh": [...], "bits": [arr_g, arr_u, arr_d]}
    (host numpy arrays per expert); shared: {"trellis": [g, u, d], "suh": [...], "svh": [...], "bits": [bg, bu, bd]}.
    act: routed activation, 0 SiLU, 1 GELU (tanh form), 2 non-gated relu2 (the gate lists are then
    not read and may hold any arrays).
    Returns (y_routed fp64 [n_rows][hidden], y_out fp16 bits [n_rows][hidden] or None)."""
    keep = []
    ex = _Experts()
    ex.cb = cb
    for pi in range(3):
        for key in ("trellis", "suh", "svh"):
            arrs = [_u16(a) for a in experts[key][pi]]
            keep.append(arrs)
            tab = (P * len(arrs))(*[a.ctypes.data for a in arrs])
            keep.append(tab)
            getattr(ex, key)[pi] = C.cast(tab, P)
        b = np.ascontiguousarray(experts["bits"][pi], np.int32)
        keep.append(b)
        ex.bits[pi] = b.ctypes.data
    sh = None
    if shared is not None:
        sh = _Dense()
        sh.cb = cb
        for pi in range(3):
            for key in ("trellis", "suh", "svh"):
                a = _u16(shared[key][pi])
                keep.append(a)
                getattr(sh, key)[pi] = a.ctypes.data
            sh.bits[pi] = int(shared["bits"][pi])
    rows = np.ascontiguousarray(rows, np.int32)
    yr = np.empty((rows.size, hidden), np.float64)
    yo = np.empty((rows.size, hidden), np.uint16) if shared is not None else None
    _moe(_p(yr), _p(yo), _p(_u16(x)), hidden, inter, _p(np.ascontiguousarray(topk_idx, np.int64)),
         _p(_u16(topk_w)), topk_idx.shape[1], _p(rows), rows.size, C.byref(ex),
         C.byref(sh) if sh is not None else None, act_limit, act)
    return yr, yo


def pack_signs(unpacked: np.ndarray, cols: int) -> np.ndarray:
    """uint16 [cols] from fp16 bit patterns [cols * 16]: the reference kernel's loop
    (src/cuda/quant/pack.cu:180-204): for each of the column's 16 values in order, shift the word
    right by one and put the value's sign bit in bit 15, so value i ends in bit i."""
    u = _u16(np.asarray(unpacked).reshape(-1))[:16 * cols].reshape(cols, 16)
    out = np.zeros(cols, np.uint16)
    for i in range(16):
        out = (out >> np.uint16(1)) | (u[:, i] & np.uint16(0x8000))
    return out


def count_inf_nan(x: np.ndarray) -> tuple[int, int]:
    """(infinities, NaNs) of an fp16 (uint16 bit patterns / float16) or fp32 array, by bit pattern: all
    exponent bits set and a zero (inf) or non-zero (NaN) mantissa (src/cuda/quant/util.cu:54-80)."""
    x = np.asarray(x)
    if x.dtype in (np.float32, np.uint32):
        v = x.view(np.uint32).reshape(-1) & np.uint32(0x7fffffff)
        e = np.uint32(0x7f800000)
    else:
        v = _u16(x.reshape(-1)) & np.uint16(0x7fff)
        e = np.uint16(0x7c00)
    return int(np.count_nonzero(v == e)), int(np.count_nonzero(v > e))


def cpu_linear_f32(x: np.ndarray, trellis, suh, svh, K: int, N: int, bits: int, cb: int, threads: int = 0):
    """CPU baseline: returns (y fp32 [M][N], seconds)."""
    x = _u16(x)
    M = x.size // K
    y = np.empty((M, N), np.float32)
    secs = _cpu_linear(_p(y), _p(x), M, K, N, _p(_u16(trellis)), _p(_u16(suh)), _p(_u16(svh)), bits, cb, threads)
    return y, secs


def cpu_max_threads() -> int:
    return _cpu_threads()
