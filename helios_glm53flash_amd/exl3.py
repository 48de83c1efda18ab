"""Python mirror of the reference's EXL3 / router / MoE-glue entry points over libhx_exl3.so.

Same names, argument meaning and order as the reference C++ interfaces
(src/cuda/quant/exl3_gemm.cuh:51-83, reconstruct.cuh:15-63, hadamard.cuh:14-43,
src/cuda/aux/routing.cuh:36-49, src/engine/glue2.cuh:44-64, src/cuda/quant/exl3_moe.cuh:74-105).
Buffers are torch tensors on the current HIP device (torch only provides device memory and the
stream; all compute runs in the HIP kernels).  Where the reference aborts, these raise.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional

import torch

from ._lib import GroupWordsC, HX_GEMM_PATH_GEMV, HX_GEMM_PATH_MFMA, HxError, check, lib

MUL1 = 0x83DCD12D
GEMV_MAX_M = 16  # largest M served by the fused decode-GEMV (one MFMA row block)
MUL1_I32 = MUL1 - (1 << 32)  # the int32 value stored in checkpoints


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(stream) -> int:
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def _need(t: torch.Tensor, name: str, dtypes: tuple) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a device tensor (got {t.device})")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.dtype not in dtypes:
        raise ValueError(f"{name} has dtype {t.dtype}, expected one of {dtypes}")


_workspaces: dict[tuple, torch.Tensor] = {}


def workspace(nbytes: int, device: Optional[torch.device] = None, stream=None) -> torch.Tensor:
    """Zero-initialised workspace of one (device, stream), grown on demand (the counters inside stay
    zero between calls because every kernel resets what it uses).  A workspace serves one stream at
    a time: calls on different streams get different workspaces, so their arrival counters and
    ready flags never meet.  Growing synchronizes the device twice: before the old buffer is
    released (kernels still queued on any stream may use it) and after the zero fill (issued on
    torch's current stream, the kernels run on `stream`).  Grow outside graph capture."""
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    key = (idx, _stream(stream))
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("the workspace of this stream must be allocated before graph capture: run the call "
                               "once on the capturing stream first, or pass a workspace")
        torch.cuda.synchronize(idx)
        ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=dev)
        torch.cuda.synchronize(idx)
        _workspaces[key] = ws
    return ws


@dataclass
class GroupWords:
    """One EXL3 linear (reference GroupWords, exl3_gemm.cuh:30-36): trellis (K/16, N/16, 16*bits)
    int16/uint16, suh fp16 [K], svh fp16 [N], mul1 (nonzero selects codebook 2)."""
    trellis: torch.Tensor
    suh: torch.Tensor
    svh: torch.Tensor
    mul1: int = 0

    @property
    def bits(self) -> int:
        return self.trellis.shape[-1] // 16

    @property
    def in_features(self) -> int:
        return self.suh.numel()

    @property
    def out_features(self) -> int:
        return self.svh.numel()

    def c(self) -> GroupWordsC:
        m = self.mul1
        if m and m > 0x7FFFFFFF:
            m -= 1 << 32
        return GroupWordsC(self.trellis.data_ptr(), self.suh.data_ptr(), self.svh.data_ptr(), m)


def gemm(y: torch.Tensor, x: torch.Tensor, w: GroupWords, M: int, N: int, K: int, bits: int, y_fp32: bool = False,
         stream=None, a_had: Optional[torch.Tensor] = None, mcg: bool = False) -> int:
    """y = svh . H_N(H_K(x . suh) . W_hat).  Returns 90 when the small-M GEMV ran, 1 for MFMA."""
    _need(x, "x", (torch.float16,))
    _need(y, "y", (torch.float32,) if y_fp32 else (torch.float16,))
    for t, n in ((w.trellis, "trellis"), (w.suh, "suh"), (w.svh, "svh")):
        _need(t, n, (torch.int16, torch.uint16, torch.float16))
    if x.numel() < M * K or y.numel() < M * N:
        raise ValueError("x / y smaller than M*K / M*N")
    if w.trellis.numel() != (K // 16) * (N // 16) * 16 * bits or w.suh.numel() < K or w.svh.numel() < N:
        raise ValueError("GroupWords shapes do not match K, N, bits")
    if a_had is not None:
        _need(a_had, "a_had", (torch.float16,))
    nbytes = lib.hx_exl3_gemm_workspace_size(M, N, K)
    ws = workspace(nbytes, x.device, stream) if (M <= GEMV_MAX_M or a_had is None) else None
    gw = w.c()
    return check(lib.hx_exl3_gemm(y.data_ptr(), x.data_ptr(), C.byref(gw), M, N, K, bits, int(y_fp32),
                                  _stream(stream), _ptr(a_had), int(mcg), _ptr(ws), ws.numel() if ws is not None else 0),
                 "hx_exl3_gemm")


def gemm_noalloc(y: torch.Tensor, x: torch.Tensor, w: GroupWords, M: int, N: int, K: int, bits: int,
                 y_fp32: bool = False, stream=None, mcg: bool = False) -> int:
    """gemm without a workspace and without allocation (the library's fixed per-GPU scratch array of
    hx_exl3_gemm_noalloc_max_bytes()); calls overlapping on one GPU race."""
    _need(x, "x", (torch.float16,))
    _need(y, "y", (torch.float32,) if y_fp32 else (torch.float16,))
    if x.numel() < M * K or y.numel() < M * N:
        raise ValueError("x / y smaller than M*K / M*N")
    gw = w.c()
    return check(lib.hx_exl3_gemm_noalloc(y.data_ptr(), x.data_ptr(), C.byref(gw), M, N, K, bits, int(y_fp32),
                                          _stream(stream), int(mcg)), "hx_exl3_gemm_noalloc")


def gemv(y, x, w: GroupWords, M, N, K, bits, y_fp32=False, stream=None, a_had=None, mcg=False) -> None:
    """Forced small-M path (reference gemv, exl3_gemm.cuh:70-83); M must be <= 16."""
    if M > GEMV_MAX_M:
        raise ValueError(f"gemv requires M <= {GEMV_MAX_M}")
    gemm(y, x, w, M, N, K, bits, y_fp32, stream, a_had, mcg)


def reconstruct_slice(unpacked: torch.Tensor, packed: torch.Tensor, packed_rows: int, packed_cols: int,
                      unpacked_cols: int, K: int, mcg: bool, mul1: bool, n_offset: int, stream=None) -> None:
    """Bit-exact trellis -> W_hat fp16 (reference reconstruct_slice, reconstruct.cuh:15-35)."""
    _need(unpacked, "unpacked", (torch.float16, torch.int16, torch.uint16))
    _need(packed, "packed", (torch.int16, torch.uint16))
    check(lib.hx_exl3_reconstruct_slice(unpacked.data_ptr(), packed.data_ptr(), packed_rows, packed_cols,
                                        unpacked_cols, K, int(mcg), int(bool(mul1)), n_offset, _stream(stream)),
          "hx_exl3_reconstruct_slice")


def reconstruct(unpacked, packed, packed_rows, packed_cols, unpacked_cols, K, mcg, mul1, stream=None) -> None:
    """Full-width reconstruct (reference reconstruct.cuh:38-48)."""
    reconstruct_slice(unpacked, packed, packed_rows, packed_cols, unpacked_cols, K, mcg, mul1, 0, stream)


def reconstruct_had_slice(unpacked: torch.Tensor, packed: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor,
                          packed_rows: int, packed_cols: int, unpacked_rows: int, unpacked_cols: int, K: int,
                          mcg: bool, mul1: bool, n_offset: int, stream=None) -> None:
    """Original-basis weights diag(suh) H W_hat H diag(svh) / 128 per 128 x 128 tile (reference
    reconstruct_had_slice, reconstruct.cuh:37-63); svh already offset by n_offset."""
    _need(unpacked, "unpacked", (torch.float16,))
    _need(packed, "packed", (torch.int16, torch.uint16))
    _need(suh, "suh", (torch.float16,))
    _need(svh, "svh", (torch.float16,))
    check(lib.hx_exl3_reconstruct_had_slice(unpacked.data_ptr(), packed.data_ptr(), suh.data_ptr(), svh.data_ptr(),
                                            packed_rows, packed_cols, unpacked_rows, unpacked_cols, K, int(mcg),
                                            int(bool(mul1)), n_offset, _stream(stream)),
          "hx_exl3_reconstruct_had_slice")


def pack_trellis(packed: torch.Tensor, unpacked: torch.Tensor, rows: int, cols: int, K: int, stream=None) -> None:
    """rows*cols blocks of 256 K-bit symbols -> 16*K trellis words each (reference pack.cuh:9-20)."""
    _need(packed, "packed", (torch.int16, torch.uint16))
    _need(unpacked, "unpacked", (torch.int16, torch.uint16))
    check(lib.hx_exl3_pack_trellis(packed.data_ptr(), unpacked.data_ptr(), rows, cols, K, _stream(stream)),
          "hx_exl3_pack_trellis")


def unpack_trellis(unpacked: torch.Tensor, packed: torch.Tensor, rows: int, cols: int, K: int, stream=None) -> None:
    """Inverse of pack_trellis: symbols with the bits above K zero (reference pack.cuh:22-33)."""
    _need(packed, "packed", (torch.int16, torch.uint16))
    _need(unpacked, "unpacked", (torch.int16, torch.uint16))
    check(lib.hx_exl3_unpack_trellis(unpacked.data_ptr(), packed.data_ptr(), rows, cols, K, _stream(stream)),
          "hx_exl3_unpack_trellis")


def pack_signs(packed: torch.Tensor, unpacked: torch.Tensor, cols: int, stream=None) -> None:
    """packed[c] bit i = sign bit of unpacked[16 c + i]: uint16 [cols] from fp16 [cols * 16]
    (reference pack.cuh:36-44)."""
    _need(unpacked, "unpacked", (torch.float16,))
    _need(packed, "packed", (torch.int16, torch.uint16))
    if unpacked.numel() < 16 * cols or packed.numel() < cols:
        raise ValueError("pack_signs: unpacked needs 16 * cols values and packed cols")
    check(lib.hx_pack_signs(packed.data_ptr(), unpacked.data_ptr(), cols, _stream(stream)), "hx_pack_signs")


def count_inf_nan(x: torch.Tensor, counts: torch.Tensor, stream=None) -> None:
    """counts[0] += infinities, counts[1] += NaNs in x (fp16 or fp32); counts is an int64 [2] tensor
    that the caller zeroes first (reference util.cuh:9-19)."""
    if x.dtype not in (torch.float16, torch.float32):
        raise TypeError("count_inf_nan: x must be float16 or float32")
    _need(x, "x", (x.dtype,))
    _need(counts, "counts", (torch.int64,))
    if counts.numel() < 2:
        raise ValueError("count_inf_nan: counts needs 2 elements")
    check(lib.hx_count_inf_nan(x.data_ptr(), counts.data_ptr(), x.numel(), 0 if x.dtype == torch.float16 else 1,
                               _stream(stream)), "hx_count_inf_nan")


_HAD_DTYPES = {torch.float16: 0, torch.float32: 1}


def _had_dtype(*ts: torch.Tensor) -> int:
    if ts[0].dtype not in _HAD_DTYPES or any(t.dtype != ts[0].dtype for t in ts):
        raise TypeError("had_r_128: inputs and outputs must all be float16 or all float32")
    return _HAD_DTYPES[ts[0].dtype]


def had_r_128(input: torch.Tensor, output: torch.Tensor, pre_scale: Optional[torch.Tensor],
              post_scale: Optional[torch.Tensor], rows: int, cols: int, scale: float = 1.0, stream=None) -> None:
    """y = H128(x) * scale / sqrt(128) per 128-element group, fp16 or fp32 data (the dtype of `input`),
    optional fp16 per-column scale before or after the transform (reference hadamard.cuh:14-25)."""
    dt = _had_dtype(input, output)
    check(lib.hx_had_r_128(input.data_ptr(), output.data_ptr(), _ptr(pre_scale), _ptr(post_scale), rows, cols, dt,
                           scale, _stream(stream)), "hx_had_r_128")


def had_r_128_dual(input1: torch.Tensor, output1: torch.Tensor, pre_scale1, post_scale1, input2: torch.Tensor,
                   output2: torch.Tensor, pre_scale2, post_scale2, rows: int, cols: int, scale: float = 1.0,
                   stream=None) -> None:
    """had_r_128 on two tensors of one shape in one launch (reference hadamard.cuh:27-43)."""
    dt = _had_dtype(input1, output1, input2, output2)
    check(lib.hx_had_r_128_dual(input1.data_ptr(), output1.data_ptr(), _ptr(pre_scale1), _ptr(post_scale1),
                                input2.data_ptr(), output2.data_ptr(), _ptr(pre_scale2), _ptr(post_scale2), rows,
                                cols, dt, scale, _stream(stream)), "hx_had_r_128_dual")


def routing_gemv(x: torch.Tensor, gate_t: torch.Tensor, scores: torch.Tensor, k: int, num_experts: int,
                 stream=None) -> None:
    """Single-token router GEMV scores = x @ gate_t.T (reference routing.cuh:19-29)."""
    _need(x, "x", (torch.float16,))
    _need(gate_t, "gate_t", (torch.float16,))
    _need(scores, "scores", (torch.float16,))
    check(lib.hx_routing_gemv(x.data_ptr(), gate_t.data_ptr(), scores.data_ptr(), k, num_experts, _stream(stream)),
          "hx_routing_gemv")


def routing_ds3_nogroup_hidden(hidden: torch.Tensor, gate_t: torch.Tensor, scores: torch.Tensor,
                               bias: Optional[torch.Tensor], topk_indices: torch.Tensor, topk_weights: torch.Tensor,
                               k: int, num_experts: int, K: int, scaling_factor: float, act_fn: int = 0,
                               stream=None) -> None:
    """Decode fast path: router GEMV into the scratch `scores`, then top-k (reference routing.cuh:51-66)."""
    _need(hidden, "hidden", (torch.float16,))
    _need(topk_indices, "topk_indices", (torch.int64,))
    _need(topk_weights, "topk_weights", (torch.float16,))
    check(lib.hx_routing_ds3_nogroup_hidden(hidden.data_ptr(), gate_t.data_ptr(), scores.data_ptr(), _ptr(bias),
                                            topk_indices.data_ptr(), topk_weights.data_ptr(), k, num_experts, K,
                                            scaling_factor, act_fn, _stream(stream)),
          "hx_routing_ds3_nogroup_hidden")


def routing_ds3_nogroup(scores: torch.Tensor, bias: Optional[torch.Tensor], topk_indices: torch.Tensor,
                        topk_weights: torch.Tensor, bsz: int, num_experts: int, K: int, scaling_factor: float,
                        use_topk: bool = True, act_fn: int = 0, stream=None) -> None:
    _need(scores, "scores", (torch.float16,))
    _need(topk_indices, "topk_indices", (torch.int64,))
    _need(topk_weights, "topk_weights", (torch.float16,))
    check(lib.hx_routing_ds3_nogroup(scores.data_ptr(), _ptr(bias), topk_indices.data_ptr(), topk_weights.data_ptr(),
                                     bsz, num_experts, K, scaling_factor, int(use_topk), act_fn, _stream(stream)),
          "hx_routing_ds3_nogroup")


def moe_permute(ids: torch.Tensor, weights: torch.Tensor, M: int, topk: int, E: int, expert_count: torch.Tensor,
                token_sorted: torch.Tensor, weight_sorted: torch.Tensor, workspace: Optional[torch.Tensor] = None,
                stream=None, route_to_sorted: Optional[torch.Tensor] = None) -> None:
    _need(ids, "ids", (torch.int64,))
    _need(weights, "weights", (torch.float16,))
    _need(expert_count, "expert_count", (torch.int64,))
    _need(token_sorted, "token_sorted", (torch.int64,))
    _need(weight_sorted, "weight_sorted", (torch.float16,))
    if expert_count.numel() < E + 1 or token_sorted.numel() < M * topk or weight_sorted.numel() < M * topk:
        raise ValueError("moe_permute output buffers too small")
    check(lib.hx_moe_permute(ids.data_ptr(), weights.data_ptr(), M, topk, E, expert_count.data_ptr(),
                             token_sorted.data_ptr(), weight_sorted.data_ptr(), _ptr(workspace), _stream(stream),
                             _ptr(route_to_sorted)), "hx_moe_permute")


def moe_reduce_sorted(y: torch.Tensor, contributions: torch.Tensor, route_to_sorted: torch.Tensor, M: int, topk: int,
                      hidden: int, stream=None) -> None:
    _need(y, "y", (torch.float32,))
    _need(contributions, "contributions", (torch.float32,))
    _need(route_to_sorted, "route_to_sorted", (torch.int64,))
    check(lib.hx_moe_reduce_sorted(y.data_ptr(), contributions.data_ptr(), route_to_sorted.data_ptr(), M, topk, hidden,
                                   _stream(stream)), "hx_moe_reduce_sorted")


def swiglu_clamp(gate: torch.Tensor, up: torch.Tensor, out: torch.Tensor, n: int, limit: float, stream=None) -> None:
    _need(gate, "gate", (torch.float32,))
    _need(up, "up", (torch.float32,))
    _need(out, "out", (torch.float16,))
    check(lib.hx_swiglu_clamp(gate.data_ptr(), up.data_ptr(), out.data_ptr(), n, limit, _stream(stream)),
          "hx_swiglu_clamp")


def gather_rows(src: torch.Tensor, idx: torch.Tensor, dst: torch.Tensor, n: int, h: int, stream=None) -> None:
    """dst[r] = src[idx[r]] for r < n, fp16 rows of h (glue.cu:48-60, the dense-MoE row gather)."""
    _need(src, "src", (torch.float16,))
    _need(idx, "idx", (torch.int64,))
    _need(dst, "dst", (torch.float16,))
    if idx.numel() < n or dst.numel() < n * h:
        raise ValueError("gather_rows: idx / dst smaller than n / n*h")
    check(lib.hx_gather_rows(src.data_ptr(), idx.data_ptr(), dst.data_ptr(), n, h, _stream(stream)), "hx_gather_rows")


def scatter_add_rows(y: torch.Tensor, src: torch.Tensor, idx: torch.Tensor, w: torch.Tensor, n: int, h: int,
                     stream=None) -> None:
    """y[idx[r]] += float(w[r]) * src[r] for r < n (glue.cu:62-82); idx distinct within a call."""
    _need(y, "y", (torch.float32,))
    _need(src, "src", (torch.float32,))
    _need(idx, "idx", (torch.int64,))
    _need(w, "w", (torch.float16,))
    if idx.numel() < n or w.numel() < n or src.numel() < n * h:
        raise ValueError("scatter_add_rows: idx / w / src smaller than n / n / n*h")
    check(lib.hx_scatter_add_rows(y.data_ptr(), src.data_ptr(), idx.data_ptr(), w.data_ptr(), n, h, _stream(stream)),
          "hx_scatter_add_rows")


def gemm_nt_f16(y: torch.Tensor, x: torch.Tensor, w: torch.Tensor, M: int, N: int, K: int, y_fp32: bool = False,
                add: bool = False, stream=None) -> None:
    """y[m][n] = sum_k x[m][k] * w[n][k] (glue2.cu:9-65,165-182): the MoE router logits with w the
    router gate [E][hidden]; fp16 y rounded once from the fp32 sum, or fp32 y (added to when add)."""
    _need(x, "x", (torch.float16,))
    _need(w, "w", (torch.float16,))
    _need(y, "y", (torch.float32,) if y_fp32 else (torch.float16,))
    check(lib.hx_gemm_nt_f16(y.data_ptr(), x.data_ptr(), w.data_ptr(), M, N, K, int(y_fp32), int(add),
                             _stream(stream)), "hx_gemm_nt_f16")


__all__ = ["GroupWords", "gemm", "gemm_nt_f16", "reconstruct_had_slice", "pack_trellis", "unpack_trellis", "gemv", "reconstruct", "reconstruct_slice", "had_r_128", "had_r_128_dual", "routing_gemv", "routing_ds3_nogroup_hidden", "routing_ds3_nogroup",
           "moe_permute", "moe_reduce_sorted", "swiglu_clamp", "workspace", "MUL1", "HxError",
           "HX_GEMM_PATH_GEMV", "HX_GEMM_PATH_MFMA"]
