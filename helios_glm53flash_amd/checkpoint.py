"""EXL3 checkpoint loader: safetensors shards -> HBM-resident expert slabs and dense GroupWords.

Reference behaviour followed:
  * shard container (src/core/safetensors.hpp:1-53): every ``*.safetensors`` file of a directory;
    8-byte little-endian header length, JSON tensor map {name: {dtype, shape, data_offsets}}, data
    region after the header; tensors are found by name across shards.
  * one EXL3 group (src/core/model.cpp:74-90): ``<base>.trellis`` I16 (K/16, N/16, 16*bits),
    ``<base>.suh`` F16 [K], ``<base>.svh`` F16 [N], ``<base>.mul1`` I32 scalar.
  * expert validation (src/core/expert_layout.cpp:6-55): names
    ``model.language_model.layers.<l>.mlp.experts.<e>.{gate,up,down}_proj``, trellis shape
    (in/16, out/16, S) with S % 16 == 0, suh [in], svh [out], mul1 scalar equal to 0x83DCD12D, exact
    byte sizes and dtypes; a violation raises with the tensor's name.

MI355X layout (not the reference's): every expert of a layer lives in ONE device allocation (288 GB of
HBM holds all 42 layers, so there is no host arena and no slot pool to stream into). Each piece
starts on a 256-byte boundary, so the decode kernels' 16-byte loads stay aligned. Per-expert bit
widths may differ within a layer: the decode and prefill kernels dispatch on per-expert bit tables.
The reference rejects mixed widths because its fused kernels are compiled per layer width.
"""
from __future__ import annotations

import json
import os
import struct
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass
from pathlib import Path
from typing import Optional

import numpy as np
import torch

from .exl3 import MUL1, GroupWords
from .moe import ExpertSet

# safetensors dtype name -> (numpy dtype used to read it, element bytes)
_DTYPES = {
    "F16": (np.float16, 2), "BF16": (np.uint16, 2), "F32": (np.float32, 4), "F64": (np.float64, 8),
    "I32": (np.int32, 4), "I16": (np.int16, 2), "I8": (np.int8, 1), "U8": (np.uint8, 1),
    "BOOL": (np.uint8, 1), "I64": (np.int64, 8),
}
PROJ_NAMES = ("gate_proj", "up_proj", "down_proj")
PIECE_ALIGN = 256


class CheckpointError(RuntimeError):
    """A missing, mis-shaped or mis-typed tensor (the message names it)."""


@dataclass
class TensorInfo:
    name: str
    dtype: str
    shape: tuple
    shard: int
    offset: int  # absolute byte offset in the shard file
    nbytes: int

    @property
    def elems(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64)) if self.shape else 1


class ShardSet:
    """Headers of every ``*.safetensors`` shard in a directory (data is read on demand)."""

    def __init__(self, directory) -> None:
        self.paths = sorted(str(p) for p in Path(directory).glob("*.safetensors"))
        if not self.paths:
            raise CheckpointError(f"no *.safetensors shard in {directory}")
        self.tensors: dict[str, TensorInfo] = {}
        for si, path in enumerate(self.paths):
            with open(path, "rb") as f:
                head = f.read(8)
                if len(head) != 8:
                    raise CheckpointError(f"{path}: truncated header")
                (n,) = struct.unpack("<Q", head)
                size = os.fstat(f.fileno()).st_size
                if n > size - 8:
                    raise CheckpointError(f"{path}: header length {n} past the end of the file")
                meta = json.loads(f.read(n))
            start = 8 + n
            for name, t in meta.items():
                if name == "__metadata__":
                    continue
                dt = t.get("dtype")
                if dt not in _DTYPES:
                    raise CheckpointError(f"{name}: unsupported dtype {dt}")
                b, e = t["data_offsets"]
                shape = tuple(int(s) for s in t["shape"])
                info = TensorInfo(name, dt, shape, si, start + int(b), int(e) - int(b))
                if info.nbytes != info.elems * _DTYPES[dt][1] or start + int(e) > size:
                    raise CheckpointError(f"{name}: data range does not match its shape and dtype")
                if name in self.tensors:
                    raise CheckpointError(f"{name}: present in two shards")
                self.tensors[name] = info

    def find(self, name: str) -> Optional[TensorInfo]:
        return self.tensors.get(name)

    def read_into(self, t: TensorInfo, dst: np.ndarray) -> None:
        """The tensor's raw bytes into dst (uint8, t.nbytes long)."""
        with open(self.paths[t.shard], "rb") as f:
            f.seek(t.offset)
            if f.readinto(memoryview(dst)) != t.nbytes:
                raise CheckpointError(f"{t.name}: short read")

    def read(self, t: TensorInfo) -> np.ndarray:
        buf = np.empty(t.nbytes, np.uint8)
        self.read_into(t, buf)
        return buf.view(_DTYPES[t.dtype][0]).reshape(t.shape)


def _align(n: int) -> int:
    return (n + PIECE_ALIGN - 1) // PIECE_ALIGN * PIECE_ALIGN


def _group_tensors(shards: ShardSet, base: str, K: int, N: int) -> tuple:
    """Validated (trellis, suh, svh, mul1) infos of one group and its bit width."""
    ts = []
    for suffix in (".trellis", ".suh", ".svh", ".mul1"):
        t = shards.find(base + suffix)
        if t is None:
            raise CheckpointError(f"missing tensor {base}{suffix}")
        ts.append(t)
    tr, su, sv, mu = ts
    if len(tr.shape) != 3 or tr.shape[0] != K // 16 or tr.shape[1] != N // 16 or tr.shape[2] % 16 or \
            not 16 <= tr.shape[2] <= 128:
        raise CheckpointError(f"unsupported trellis shape {tr.shape} for {base} ({K} -> {N})")
    bits = tr.shape[2] // 16
    if su.shape != (K,) or sv.shape != (N,) or mu.shape != ():
        raise CheckpointError(f"invalid scales/multiplier shape: {base}")
    want = (("I16", K * N * bits // 8), ("F16", 2 * K), ("F16", 2 * N), ("I32", 4))
    for t, (dt, nb) in zip(ts, want):
        if t.dtype != dt or t.nbytes != nb:
            raise CheckpointError(f"invalid tensor size/dtype: {t.name}")
    return tr, su, sv, mu, bits


@dataclass
class ExpertLayout:
    """Byte offsets of every expert's pieces in the layer slab: off[e][p] = (trellis, suh, svh)."""
    off: list
    bits: list  # [e][p]
    total: int


def expert_layout(shards: ShardSet, layer: int, experts: int, hidden: int, inter: int,
                  prefix: str = "model.language_model.layers") -> tuple[ExpertLayout, list]:
    """Validate every expert tensor of a layer (expert_layout.cpp:6-55) and place the pieces."""
    off, bits, infos = [], [], []
    pos = 0
    for e in range(experts):
        eo, eb, ei = [], [], []
        for p, pn in enumerate(PROJ_NAMES):
            base = f"{prefix}.{layer}.mlp.experts.{e}.{pn}"
            K, N = (inter, hidden) if p == 2 else (hidden, inter)
            tr, su, sv, mu, b = _group_tensors(shards, base, K, N)
            mul = int(shards.read(mu)) & 0xFFFFFFFF
            if mul != MUL1:
                raise CheckpointError(f"unsupported expert mul1 codebook {mul:#x}: {base}")
            o = []
            for t in (tr, su, sv):
                o.append(pos)
                pos = _align(pos + t.nbytes)
            eo.append(tuple(o))
            eb.append(b)
            ei.append((tr, su, sv))
        off.append(eo)
        bits.append(eb)
        infos.append(ei)
    return ExpertLayout(off, bits, pos), infos


def load_experts(shards: ShardSet, layer: int, experts: int, hidden: int, inter: int, device="cuda",
                 prefix: str = "model.language_model.layers", readers: int = 8) -> ExpertSet:
    """Every routed expert of a layer in one device slab; the ExpertSet's tensors are views of it."""
    lay, infos = expert_layout(shards, layer, experts, hidden, inter, prefix)
    host = torch.empty(lay.total, dtype=torch.uint8, pin_memory=torch.device(device).type == "cuda")
    hv = host.numpy()
    jobs = [(t, o) for e in range(experts) for p in range(3) for t, o in zip(infos[e][p], lay.off[e][p])]
    # file reads release the interpreter lock: a few readers keep the page cache / disk busy
    # (measured on the MI355X box, one 1.8 GB layer from page cache: 0.72 s serial, 0.15 s with 8)
    with ThreadPoolExecutor(max(1, min(readers, len(jobs)))) as pool:
        list(pool.map(lambda j: shards.read_into(j[0], hv[j[1]:j[1] + j[0].nbytes]), jobs))
    slab = host.to(device, non_blocking=True)
    if slab.is_cuda:
        torch.cuda.current_stream(slab.device).synchronize()  # the pinned host buffer is freed on return
    tr, su, sv, bt = [[], [], []], [[], [], []], [[], [], []], [[], [], []]
    for e in range(experts):
        for p in range(3):
            K, N = (inter, hidden) if p == 2 else (hidden, inter)
            b = lay.bits[e][p]
            (ot, os_, ov) = lay.off[e][p]
            tr[p].append(slab[ot:ot + K * N * b // 8].view(torch.int16).view(K // 16, N // 16, 16 * b))
            su[p].append(slab[os_:os_ + 2 * K].view(torch.float16))
            sv[p].append(slab[ov:ov + 2 * N].view(torch.float16))
            bt[p].append(b)
    # the views hold the slab's storage alive
    return ExpertSet(hidden, inter, tr, su, sv, bt, True)


def load_group(shards: ShardSet, base: str, in_features: int, out_features: int, device="cuda") -> GroupWords:
    """One dense EXL3 linear (model.cpp:74-90), e.g. ``lm_head`` or a shared expert's projection."""
    tr, su, sv, mu, bits = _group_tensors(shards, base, in_features, out_features)
    mul = int(shards.read(mu)) & 0xFFFFFFFF
    t = torch.from_numpy(shards.read(tr).copy()).to(device)
    s_in = torch.from_numpy(shards.read(su).copy()).to(device)
    s_out = torch.from_numpy(shards.read(sv).copy()).to(device)
    return GroupWords(t, s_in, s_out, mul)


def load_shared_mlp(shards: ShardSet, layer: int, hidden: int, inter: int, device="cuda",
                    prefix: str = "model.language_model.layers") -> Optional[list]:
    """gate, up, down of a layer's shared expert (model.cpp:185-200), or None when absent."""
    base = f"{prefix}.{layer}.mlp.shared_experts"
    if shards.find(base + ".gate_proj.trellis") is None:
        return None
    return [load_group(shards, f"{base}.{pn}", K, N, device)
            for pn, (K, N) in zip(PROJ_NAMES, ((hidden, inter), (hidden, inter), (inter, hidden)))]


def _to_f16(shards: ShardSet, t: TensorInfo) -> np.ndarray:
    a = shards.read(t)
    if t.dtype == "F16":
        return a
    if t.dtype == "BF16":  # bf16 bits -> fp32 (exact) -> fp16 (round to nearest even)
        return (a.astype(np.uint32) << 16).view(np.float32).astype(np.float16)
    if t.dtype in ("F32", "F64"):
        return a.astype(np.float16)
    raise CheckpointError(f"{t.name}: expected a floating-point tensor, got {t.dtype}")


def load_router(shards: ShardSet, layer: int, experts: int, hidden: int, device="cuda",
                prefix: str = "model.language_model.layers") -> tuple:
    """Router gate fp16 [E][hidden] and score-correction bias (model.cpp:185-196), or (None, None).

    The bias is stored centred, as the reference's loader does (model.cpp:524-535): read as fp32, minus
    its mean (fp64 sum, rounded to fp32), then rounded to fp16; top-k selection is unchanged by the
    shift and the fp16 values keep more precision."""
    base = f"{prefix}.{layer}.mlp.gate"
    tw = shards.find(base + ".weight")
    if tw is None:
        return None, None
    if tw.shape != (experts, hidden):
        raise CheckpointError(f"invalid router gate shape {tw.shape}: {base}.weight")
    w = torch.from_numpy(_to_f16(shards, tw).copy()).to(device)
    tb = shards.find(base + ".e_score_correction_bias")
    if tb is None:
        return w, None
    if tb.shape != (experts,):
        raise CheckpointError(f"invalid router bias shape {tb.shape}: {base}.e_score_correction_bias")
    f = shards.read(tb).astype(np.float32) if tb.dtype != "BF16" else \
        (shards.read(tb).astype(np.uint32) << 16).view(np.float32)
    mean = np.float32(f.astype(np.float64).sum() / f.size)
    b = (f - mean).astype(np.float16)
    return w, torch.from_numpy(b).to(device)


# ---------------------------------------------------------------- native loader (C ABI, C++ host code)

class NativeCheckpoint:
    """The library's C++ loader (hx_ckpt_*: safetensors.hpp / expert_layout.cpp / model.cpp:254-340
    restated): the path a C++ engine binds.  Same validation as the Python loader above, the
    reference's one-width-per-projection rule and its 64-byte-aligned slab layout."""

    def __init__(self, directory) -> None:
        import ctypes as C
        from ._lib import check, lib
        self._lib = lib
        h = C.c_void_p()
        check(lib.hx_ckpt_open(str(directory).encode(), C.byref(h)), "hx_ckpt_open")
        self._h = h

    def close(self) -> None:
        if self._h:
            self._lib.hx_ckpt_close(self._h)
            self._h = None

    def __del__(self) -> None:
        self.close()

    def tensor_count(self) -> int:
        return self._lib.hx_ckpt_tensor_count(self._h)

    def expert_layout(self, layer: int, experts: int, hidden: int, inter: int):
        from ._lib import ExpertLayoutC, check
        import ctypes as C
        lay = ExpertLayoutC()
        check(self._lib.hx_ckpt_expert_layout(self._h, layer, experts, hidden, inter, C.byref(lay)),
              "hx_ckpt_expert_layout")
        return lay

    def load_experts(self, layer: int, experts: int, hidden: int, inter: int, device="cuda",
                     readers: int = 8) -> ExpertSet:
        """Every routed expert of a layer in one device slab (layout of hx_ckpt_expert_layout); the
        ExpertSet's tensors are views of the slab and its pointer tables come from hx_ckpt_expert_tables."""
        import ctypes as C
        from ._lib import ExpertTablesC, check
        from .exl3 import _stream
        lay = self.expert_layout(layer, experts, hidden, inter)
        slab = torch.empty(experts * lay.stride, dtype=torch.uint8, device=device)
        st = _stream(None)
        check(self._lib.hx_ckpt_load_experts(self._h, layer, experts, C.byref(lay), slab.data_ptr(), slab.numel(),
                                             readers, st), "hx_ckpt_load_experts")
        tables = torch.empty(9 * experts, dtype=torch.int64, device=device)
        tc = ExpertTablesC()
        check(self._lib.hx_ckpt_expert_tables(C.byref(lay), slab.data_ptr(), experts, tables.data_ptr(),
                                              C.byref(tc), st), "hx_ckpt_expert_tables")
        tr, su, sv, bt = [[], [], []], [[], [], []], [[], [], []], [[], [], []]
        for e in range(experts):
            base = e * lay.stride
            for p in range(3):
                K, N = (inter, hidden) if p == 2 else (hidden, inter)
                b = lay.bits[p]
                ot, os_, ov = (base + lay.off[4 * p + q] for q in range(3))
                tr[p].append(slab[ot:ot + K * N * b // 8].view(torch.int16).view(K // 16, N // 16, 16 * b))
                su[p].append(slab[os_:os_ + 2 * K].view(torch.float16))
                sv[p].append(slab[ov:ov + 2 * N].view(torch.float16))
                bt[p].append(b)
        ex = ExpertSet(hidden, inter, tr, su, sv, bt, True)
        ex._keep = [tables]
        ex._tables = tc
        return ex
