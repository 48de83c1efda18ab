"""MoE-layer entry points over libhx_exl3.so: expert tables resident in HBM, the reference's
moe_grouped (src/cuda/quant/exl3_moe.cuh:74-105) and the whole single-GPU moe_ffn flow
(src/engine/runner.cpp:711-959) as one host-sync-free call.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field
from typing import Optional, Sequence

import torch

from ._lib import ExpertTablesC, GroupWordsC, check, lib
from .exl3 import MUL1, GroupWords, _need, _ptr, _stream, gemm_nt_f16, workspace

PROJ = ("gate", "up", "down")


@dataclass
class ExpertSet:
    """Routed experts of one layer.  Per projection p: trellis[p][e] (K/16, N/16, 16*bits) int16,
    suh[p][e] fp16 [K], svh[p][e] fp16 [N]; bits[p][e].  Device pointer tables are built once."""
    hidden: int
    inter: int
    trellis: list  # [3][E] tensors
    suh: list
    svh: list
    bits: list  # [3][E] ints
    mul1: bool = True
    _keep: list = field(default_factory=list, repr=False)
    _tables: Optional[ExpertTablesC] = field(default=None, repr=False)

    @property
    def num_experts(self) -> int:
        return len(self.trellis[0])

    def uniform_bits(self) -> Optional[tuple]:
        u = tuple(b[0] for b in self.bits)
        return u if all(all(x == u[p] for x in self.bits[p]) for p in range(3)) else None

    def tables(self) -> ExpertTablesC:
        if self._tables is not None:
            return self._tables
        dev = self.trellis[0][0].device
        ptrs = []
        for p in range(3):
            for arr in (self.trellis[p], self.suh[p], self.svh[p]):
                t = torch.tensor([a.data_ptr() for a in arr], dtype=torch.int64, device=dev)
                ptrs.append(t)
        fields = [t.data_ptr() for t in ptrs]
        mask = 0
        bit_ptrs = [None, None, None]
        if self.uniform_bits() is None:
            for p in range(3):
                bt = torch.tensor(self.bits[p], dtype=torch.int32, device=dev)
                ptrs.append(bt)
                bit_ptrs[p] = bt.data_ptr()
                for b in self.bits[p]:
                    mask |= 1 << int(b)
        self._keep = ptrs
        self._tables = ExpertTablesC(*fields, *bit_ptrs, mask)
        return self._tables

    @classmethod
    def synthetic(cls, num_experts: int, hidden: int, inter: int, bits, seed: int, device="cuda",
                  mul1: bool = True) -> "ExpertSet":
        """Seeded synthetic experts: uniform trellis words, suh = +-1, svh = +-U(0.5, 1.5) in fp16.
        bits: int, (g, u, d), or a per-expert list of ints/(g, u, d)."""
        if isinstance(bits, int):
            per = [(bits, bits, bits)] * num_experts
        elif isinstance(bits, tuple):
            per = [bits] * num_experts
        else:
            per = [(b, b, b) if isinstance(b, int) else tuple(b) for b in bits]
        g = torch.Generator(device=device)
        g.manual_seed(seed)
        shapes = [(hidden, inter), (hidden, inter), (inter, hidden)]
        tr, su, sv, bt = [[], [], []], [[], [], []], [[], [], []], [[], [], []]
        for e in range(num_experts):
            for p, (K, N) in enumerate(shapes):
                b = per[e][p]
                t, s_in, s_out = synthetic_linear(K, N, b, g, device)
                tr[p].append(t)
                su[p].append(s_in)
                sv[p].append(s_out)
                bt[p].append(b)
        return cls(hidden, inter, tr, su, sv, bt, mul1)

    def weight_bytes(self, experts: Sequence[int]) -> int:
        """Compressed EXL3 bytes (trellis + suh + svh) of the given experts."""
        n = 0
        for e in experts:
            for p in range(3):
                n += self.trellis[p][e].numel() * 2 + self.suh[p][e].numel() * 2 + self.svh[p][e].numel() * 2
        return n


def synthetic_linear(K: int, N: int, bits: int, g: torch.Generator, device="cuda"):
    tr = torch.randint(-32768, 32768, (K // 16, N // 16, 16 * bits), dtype=torch.int16, generator=g, device=device)
    suh = (torch.randint(0, 2, (K,), generator=g, device=device) * 2 - 1).to(torch.float16)
    sign = torch.randint(0, 2, (N,), generator=g, device=device) * 2 - 1
    svh = (sign * (0.5 + torch.rand(N, generator=g, device=device))).to(torch.float16)
    return tr, suh, svh


def synthetic_dense_mlp(hidden: int, inter: int, bits, seed: int, device="cuda") -> list[GroupWords]:
    """gate, up, down GroupWords of a dense (shared-expert) MLP."""
    if isinstance(bits, int):
        bits = (bits, bits, bits)
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    out = []
    for (K, N), b in zip([(hidden, inter), (hidden, inter), (inter, hidden)], bits):
        t, s_in, s_out = synthetic_linear(K, N, b, g, device)
        out.append(GroupWords(t, s_in, s_out, MUL1))
    return out


def moe_workspace_bytes(tokens: int, hidden: int, inter: int, num_experts: int, topk: int) -> int:
    return lib.hx_moe_workspace_size(tokens, hidden, inter, num_experts, topk)


def moe_grouped(x: torch.Tensor, y: Optional[torch.Tensor], expert_count: torch.Tensor, token_sorted: torch.Tensor,
                weight_sorted: torch.Tensor, experts: ExpertSet, tokens: int, topk: int, act_limit: float = 10.0,
                stream=None, sorted_contributions: Optional[torch.Tensor] = None,
                route_to_sorted: Optional[torch.Tensor] = None, mcg: bool = False, act_function: int = 0) -> None:
    """Reference moe_grouped: y (fp32) += routed sum, or sorted_contributions (fp32 rows).
    act_function: 0 SiLU, 1 GELU (tanh form), 2 non-gated relu2 (exl3_moe_common.cuh:6-8)."""
    _need(x, "x", (torch.float16,))
    ub = experts.uniform_bits() or (0, 0, 0)
    E = experts.num_experts
    nbytes = moe_workspace_bytes(tokens, experts.hidden, experts.inter, E, topk)
    ws = workspace(nbytes, x.device, stream)
    mul1 = experts.mul1 and not mcg
    check(lib.hx_moe_grouped(x.data_ptr(), _ptr(y), expert_count.data_ptr(), token_sorted.data_ptr(),
                             weight_sorted.data_ptr(), None, None, None, None, C.byref(experts.tables()), tokens,
                             experts.hidden, experts.inter, E, topk, tokens, 0, ub[0], ub[1], ub[2], int(mcg),
                             int(mul1), act_limit, act_function, -1, _stream(stream), _ptr(sorted_contributions),
                             _ptr(route_to_sorted), ws.data_ptr(), ws.numel()), "hx_moe_grouped")


class MoeLayer:
    """One MoE FFN layer (routed experts + optional shared expert), resident in HBM."""

    def __init__(self, experts: ExpertSet, shared: Optional[list] = None, topk: int = 8,
                 routed_scale: float = 2.5, act_limit: float = 10.0, router_weight: Optional[torch.Tensor] = None,
                 mcg: bool = False):
        """router_weight: optional router gate fp16 [E][hidden]; with it the layer may be called with
        scores=None and computes the logits itself (gemm_nt_f16, stream-ordered, no host sync).
        mcg: the experts (routed and shared) use the MCG codebook (the reference layer's mcg flag;
        experts.mul1 must then be False).  A layer is MCG or mul1, never the 3INST codebook."""
        if mcg and experts.mul1:
            raise ValueError("MoeLayer: mcg=True needs experts built with mul1=False")
        # the layer decodes the shared expert with the routed experts' codebook
        layer_mul1 = bool(experts.mul1) and not mcg
        if shared is not None and any(bool(w.mul1) != layer_mul1 for w in shared):
            raise ValueError("MoeLayer: the shared expert's codebook (GroupWords.mul1) must match the routed "
                             "experts'")
        self.mcg = mcg
        self.router_weight = router_weight
        self.experts = experts
        self.shared = shared
        self.topk = topk
        self.routed_scale = routed_scale
        self.act_limit = act_limit
        self._shared_c = None
        self._shared_bits = None
        if shared is not None:
            self._shared_c = (GroupWordsC * 3)(*[w.c() for w in shared])
            self._shared_bits = (C.c_int * 3)(*[w.bits for w in shared])

    def workspace_bytes(self, tokens: int) -> int:
        return moe_workspace_bytes(tokens, self.experts.hidden, self.experts.inter, self.experts.num_experts, self.topk)

    def __call__(self, x: torch.Tensor, scores: Optional[torch.Tensor] = None, y: Optional[torch.Tensor] = None,
                 y_routed: Optional[torch.Tensor] = None, bias: Optional[torch.Tensor] = None, stream=None,
                 ws: Optional[torch.Tensor] = None) -> torch.Tensor:
        _need(x, "x", (torch.float16,))
        T = x.shape[0]
        ex = self.experts
        if scores is None:
            if self.router_weight is None:
                raise ValueError("MoeLayer: scores=None needs router_weight")
            scores = torch.empty((T, ex.num_experts), dtype=torch.float16, device=x.device)
            gemm_nt_f16(scores, x, self.router_weight, T, ex.num_experts, ex.hidden, stream=stream)
        _need(scores, "scores", (torch.float16,))
        if y is None:
            y = torch.empty((T, ex.hidden), dtype=torch.float16, device=x.device)
        if ws is None:
            ws = workspace(self.workspace_bytes(T), x.device, stream)
        ub = ex.uniform_bits() or (0, 0, 0)
        check(lib.hx_moe_layer(y.data_ptr(), _ptr(y_routed), x.data_ptr(), scores.data_ptr(), _ptr(bias),
                               C.byref(ex.tables()),
                               self._shared_c if self._shared_c is not None else None,
                               self._shared_bits if self._shared_bits is not None else None,
                               T, ex.hidden, ex.inter, ex.num_experts, self.topk, ub[0], ub[1], ub[2],
                               self.routed_scale, self.act_limit, int(self.mcg), int(ex.mul1 and not self.mcg),
                               ws.data_ptr(), ws.numel(),
                               _stream(stream)), "hx_moe_layer")
        return y


def check_status(ws: torch.Tensor, stream=None) -> None:
    """Raise if a bounded in-kernel wait of the few-token layer gave up since the last check (the
    flag is cleared); synchronizes the stream."""
    check(lib.hx_moe_check_status(ws.data_ptr(), _stream(stream)), "hx_moe_check_status")


__all__ = ["ExpertSet", "MoeLayer", "check_status", "moe_grouped", "moe_workspace_bytes", "synthetic_dense_mlp", "synthetic_linear"]
