"""Python mirror of the reference's quant op interface (cpp/src/quant.hpp:32-141)
over libnq_hip.so, on device tensors.

Same names, argument meaning and error behaviour as the reference free functions
and the Weight factory; shapes follow quant.hpp (weights [out, in], x [m, in],
y [m, out]). Errors the reference raises as std::invalid_argument surface as
ValueError (NqShapeError). torch is only the device-memory/stream plumbing: every
computation below is a libnq_hip.so kernel, and importing this module fails when
the library is not built.
"""
from __future__ import annotations

import enum
import os
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import NQ_F16, NQ_F32, NQ_PATH_AUTO, check

_lib.load()  # fail loudly at import when the HIP library is missing

_DT = {torch.float32: NQ_F32, torch.float16: NQ_F16}


def _ptr(t):
    return None if t is None else t.data_ptr()


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _dev(t: torch.Tensor, name: str) -> torch.Tensor:
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    return t.contiguous()


def _dtype_code(t: torch.Tensor, name: str) -> int:
    if t.dtype not in _DT:
        raise ValueError(f"{name} must be float32 or float16, got {t.dtype}")
    return _DT[t.dtype]


def _bias(bias, out):
    if bias is None:
        return None
    b = _dev(bias, "bias").to(torch.float32)
    if b.numel() != out:
        raise ValueError("bias must match out-features")
    return b


class QuantMode(enum.IntEnum):
    """quant.hpp:32"""
    NONE = 0
    Q8 = 1
    Q4 = 2
    Q4G = 3
    W8A8 = 4


class Format(enum.IntEnum):
    """quant.hpp:41"""
    F32 = 0
    F16 = 1
    BF16 = 2
    Q8 = 3
    Q4 = 4
    Q4G = 5
    W8A8 = 6


def format_name(f: Format) -> str:
    """quant.cpp:447-458"""
    return {Format.F32: "f32", Format.F16: "f16", Format.BF16: "bf16", Format.Q8: "q8",
            Format.Q4: "q4", Format.Q4G: "q4g", Format.W8A8: "w8a8"}.get(Format(f), "?")


def quant_mode(name: str) -> QuantMode:
    """nicpp.cpp:51-59"""
    table = {"fp32": QuantMode.NONE, "none": QuantMode.NONE, "q8": QuantMode.Q8, "q4": QuantMode.Q4,
             "q4g": QuantMode.Q4G, "w8a8": QuantMode.W8A8}
    if name not in table:
        raise ValueError(f"unknown quant mode '{name}' (fp32|q8|q4|q4g|w8a8)")
    return table[name]


@dataclass
class QTensor:
    """quant.hpp:49-54 on device: int8 codes [out, in] + fp32 scale [out]."""
    q: torch.Tensor
    scale: torch.Tensor
    out: int
    in_: int

    def check(self):
        if self.q.numel() != self.out * self.in_:
            raise ValueError("QTensor: q size != out*in")
        if self.scale.numel() != self.out:
            raise ValueError("QTensor: scale size != out")


@dataclass
class Q4GTensor:
    """quant.hpp:105-111 on device: packed nibbles [out, ceil(in/2)] + one scale
    per (row, group) [out, ceil(in/group)], fp32 (reference) or fp16."""
    q: torch.Tensor
    scale: torch.Tensor
    out: int
    in_: int
    group: int

    def check(self):
        if self.group <= 0:
            raise ValueError("Q4GTensor: group must be positive")
        if self.q.numel() != self.out * ((self.in_ + 1) // 2):
            raise ValueError("Q4GTensor: q size != out*ceil(in/2)")
        if self.scale.numel() != self.out * ((self.in_ + self.group - 1) // self.group):
            raise ValueError("Q4GTensor: scale size != out*ceil(in/group)")


def _w2d(w, who):
    w = _dev(w, "w")
    if w.dim() != 2:
        raise ValueError(f"{who} expects a 2-D [out, in] weight")
    return w.to(torch.float32).contiguous()


def quantize_q8(w: torch.Tensor) -> QTensor:
    """quant.cpp:88-108 (device side, bit-exact)."""
    w = _w2d(w, "quantize_q8")
    out, k = w.shape
    q = torch.empty((out, k), dtype=torch.int8, device=w.device)
    s = torch.empty(out, dtype=torch.float32, device=w.device)
    check(_lib.load().nq_quantize_q8(_ptr(w), out, k, _ptr(q), _ptr(s), _stream()))
    return QTensor(q, s, out, k)


def quantize_q4g(w: torch.Tensor, group: int = 32, scale_dtype=torch.float32) -> Q4GTensor:
    """quant.cpp:295-321 (device side, bit-exact codes; fp16 scale storage optional)."""
    w = _w2d(w, "quantize_q4g")
    if group <= 0:
        raise ValueError("quantize_q4g: group must be positive")
    out, k = w.shape
    nb = (k + group - 1) // group
    q = torch.empty((out, (k + 1) // 2), dtype=torch.uint8, device=w.device)
    s = torch.empty((out, nb), dtype=scale_dtype, device=w.device)
    check(_lib.load().nq_quantize_q4g(_ptr(w), out, k, group, _ptr(q), _ptr(s),
                                      _dtype_code(s, "scale"), _stream()))
    return Q4GTensor(q, s, out, k, group)


def quantize_q4(w: torch.Tensor) -> Q4GTensor:
    """quant.cpp:212-233: per-row int4 is Q4G with one block per row."""
    w = _w2d(w, "quantize_q4")
    return quantize_q4g(w, max(1, w.shape[1]))


def act_quant(x: torch.Tensor):
    """The activation quant of linear_w8a8 (quant.cpp:179-193): (xq int8, a_scale fp32)."""
    x = _dev(x, "x")
    if x.dim() != 2:
        raise ValueError("act_quant expects 2-D x")
    m, k = x.shape
    xq = torch.empty((m, k), dtype=torch.int8, device=x.device)
    s = torch.empty(m, dtype=torch.float32, device=x.device)
    check(_lib.load().nq_act_quant_i8(_ptr(x), _dtype_code(x, "x"), m, k, _ptr(xq), _ptr(s), _stream()))
    return xq, s


def act_quant_heads(a: torch.Tensor):
    """act_quant of a head-major [heads, s, d] tensor's transpose [s, heads*d]
    (an attention output feeding o_proj) without the transpose copy."""
    a = _dev(a, "a")
    if a.dim() != 3 or not a.is_contiguous():
        raise ValueError("act_quant_heads expects a contiguous [heads, s, d] tensor")
    h, s, d = a.shape
    xq = torch.empty((s, h * d), dtype=torch.int8, device=a.device)
    sc = torch.empty(s, dtype=torch.float32, device=a.device)
    check(_lib.load().nq_act_quant_i8_heads(_ptr(a), _dtype_code(a, "a"), h, s, d, _ptr(xq), _ptr(sc), _stream()))
    return xq, sc


def rmsnorm_quant(x: torch.Tensor, w: torch.Tensor, eps: float):
    """rmsnorm (ops.cpp:272-290) with the act quant of linear_w8a8 fused in:
    (xq int8, a_scale fp32) of x * (1/sqrt(mean(x^2) + eps)) * w."""
    x = _dev(x, "x")
    if x.dim() != 2:
        raise ValueError("rmsnorm_quant expects 2-D x")
    m, k = x.shape
    w = _dev(w, "w").to(torch.float32)
    if w.numel() != k:
        raise ValueError("rmsnorm_quant: weight must match the last dimension")
    xq = torch.empty((m, k), dtype=torch.int8, device=x.device)
    s = torch.empty(m, dtype=torch.float32, device=x.device)
    check(_lib.load().nq_rmsnorm_quant_i8(_ptr(x), _dtype_code(x, "x"), _ptr(w), float(eps), m, k, _ptr(xq), _ptr(s),
                                          _stream()))
    return xq, s


def add_rmsnorm_quant(x: torch.Tensor, r: torch.Tensor, w: torch.Tensor, eps: float, inplace: bool = False):
    """h = x + r (the residual add, model.cpp:175-186) and rmsnorm_quant(h) in one
    launch: returns (h, xq, a_scale); with inplace=True h is written into x."""
    x, r = _dev(x, "x"), _dev(r, "r")
    if x.dim() != 2 or r.shape != x.shape or r.dtype != x.dtype or not x.is_contiguous() or not r.is_contiguous():
        raise ValueError("add_rmsnorm_quant: x and r must be contiguous 2-D tensors of one shape and dtype")
    m, k = x.shape
    w = _dev(w, "w").to(torch.float32)
    if w.numel() != k:
        raise ValueError("add_rmsnorm_quant: weight must match the last dimension")
    h = x if inplace else torch.empty_like(x)
    xq = torch.empty((m, k), dtype=torch.int8, device=x.device)
    s = torch.empty(m, dtype=torch.float32, device=x.device)
    check(_lib.load().nq_add_rmsnorm_quant_i8(_ptr(x), _ptr(r), _dtype_code(x, "x"), _ptr(w), float(eps), m, k,
                                              _ptr(h), _ptr(xq), _ptr(s), _stream()))
    return h, xq, s


def silu_mul_quant(gate: torch.Tensor, up: torch.Tensor):
    """silu(gate) * up (ops.cpp:86-100) with the act quant fused in. gate and up
    are [m, k] views with unit column stride and one common row stride (e.g. the
    two halves of a fused gate|up projection output)."""
    if not (isinstance(gate, torch.Tensor) and gate.is_cuda and isinstance(up, torch.Tensor) and up.is_cuda):
        raise ValueError("gate and up must be device tensors")
    if gate.shape != up.shape or gate.dim() != 2 or gate.dtype != up.dtype:
        raise ValueError("silu_mul_quant: gate and up must be 2-D tensors of one shape and dtype")
    if gate.stride(1) != 1 or up.stride(1) != 1 or gate.stride(0) != up.stride(0):
        raise ValueError("silu_mul_quant: unit column stride and a common row stride required")
    m, k = gate.shape
    xq = torch.empty((m, k), dtype=torch.int8, device=gate.device)
    s = torch.empty(m, dtype=torch.float32, device=gate.device)
    check(_lib.load().nq_silu_mul_quant_i8(_ptr(gate), _ptr(up), _dtype_code(gate, "gate"), m, k, gate.stride(0),
                                           _ptr(xq), _ptr(s), _stream()))
    return xq, s


def _x2d(x, w_in, who):
    x = _dev(x, "x")
    if x.dim() != 2:
        raise ValueError(f"{who} expects 2-D x")
    if x.shape[1] != w_in:
        raise ValueError(f"{who}: x cols must match weight in-features")
    return x


def linear_q8(x: torch.Tensor, w: QTensor, bias=None, out_dtype=None, path: int = NQ_PATH_AUTO) -> torch.Tensor:
    """quant.cpp:136-163 / cuda_quant.cu:300-322. Batched shapes whose weight
    has too few rows to fill the GPU split K over a workspace from torch's
    allocator. path forces a kernel family (the per-call form of the
    reference's CudaPolicy::force_tiled_q8, cuda_backend.hpp:57-59):
    NQ_PATH_GEMV, NQ_PATH_MFMA or NQ_PATH_GENERIC (nq_linear_q8_ex)."""
    w.check()
    x = _x2d(x, w.in_, "linear_q8")
    b = _bias(bias, w.out)
    y = torch.empty((x.shape[0], w.out), dtype=out_dtype or x.dtype, device=x.device)
    lib = _lib.load()
    nbytes = lib.nq_linear_wq_workspace_size(x.shape[0], w.out, w.in_)
    ws = _workspace(nbytes, x.device) if nbytes else None
    check(lib.nq_linear_q8_ex(_ptr(x), _dtype_code(x, "x"), _ptr(w.q), _ptr(w.scale), _ptr(b), _ptr(y),
                              _dtype_code(y, "y"), x.shape[0], w.out, w.in_, _ptr(ws), nbytes, int(path),
                              _stream()))
    return y


def linear_q4g(x: torch.Tensor, w: Q4GTensor, bias=None, out_dtype=None, path: int = NQ_PATH_AUTO) -> torch.Tensor:
    """quant.cpp:337-389 (no GPU counterpart in the reference); split K and
    the per-call path as linear_q8 (nq_linear_q4g_ex)."""
    w.check()
    x = _x2d(x, w.in_, "linear_q4g")
    b = _bias(bias, w.out)
    y = torch.empty((x.shape[0], w.out), dtype=out_dtype or x.dtype, device=x.device)
    lib = _lib.load()
    nbytes = lib.nq_linear_wq_workspace_size(x.shape[0], w.out, w.in_)
    ws = _workspace(nbytes, x.device) if nbytes else None
    check(lib.nq_linear_q4g_ex(_ptr(x), _dtype_code(x, "x"), _ptr(w.q), _ptr(w.scale),
                               _dtype_code(w.scale, "scale"), w.group, _ptr(b), _ptr(y), _dtype_code(y, "y"),
                               x.shape[0], w.out, w.in_, _ptr(ws), nbytes, int(path), _stream()))
    return y


linear_q4 = linear_q4g  # quant.cpp:247-293: Q4 is Q4G with group == in


def nit_info(path: str):
    """(dtype, shape) of a NIT0 / NIT1 weight file (serialize.hpp:1-23); dtype 0
    fp32, 1 bf16. Raises NqError (NQ_IO_ERROR) for load_bin's malformed cases."""
    import ctypes
    dt, nd = ctypes.c_int32(0), ctypes.c_int32(0)
    shape = (ctypes.c_int64 * 8)()
    check(_lib.load().nq_nit_info(os.fsencode(path), ctypes.addressof(dt), ctypes.addressof(nd),
                                  ctypes.addressof(shape), 8))
    return dt.value, tuple(shape[i] for i in range(nd.value))


def load_nit(path: str, device="cuda") -> torch.Tensor:
    """load_bin (serialize.cpp:11-72) onto the device as fp32 (bf16 payloads
    inflated exactly, bits << 16)."""
    _, shape = nit_info(path)
    t = torch.empty(shape, dtype=torch.float32, device=device)
    with torch.cuda.device(t.device):
        check(_lib.load().nq_nit_load_f32(os.fsencode(path), _ptr(t), t.numel(), _stream()))
    return t


def _nit_2d(path, who):
    _, shape = nit_info(path)
    if len(shape) != 2:
        raise ValueError(f"{who}: {path} holds a {len(shape)}-d tensor, expected [out, in]")
    return shape


def load_nit_q8(path: str, device="cuda") -> QTensor:
    """quantize_q8(load_bin(path)) with the payload streamed to the device and
    quantized there (bit-exact codes and scales)."""
    out, k = _nit_2d(path, "load_nit_q8")
    q = torch.empty((out, k), dtype=torch.int8, device=device)
    s = torch.empty(out, dtype=torch.float32, device=device)
    with torch.cuda.device(q.device):
        check(_lib.load().nq_nit_load_q8(os.fsencode(path), _ptr(q), _ptr(s), out, k, _stream()))
    return QTensor(q, s, out, k)


def load_nit_q4g(path: str, group: int = 32, scale_dtype=torch.float32, device="cuda") -> Q4GTensor:
    """quantize_q4g(load_bin(path), group) on the device (bit-exact codes)."""
    out, k = _nit_2d(path, "load_nit_q4g")
    if group <= 0:
        raise ValueError("load_nit_q4g: group must be positive")
    q = torch.empty((out, (k + 1) // 2), dtype=torch.uint8, device=device)
    s = torch.empty((out, (k + group - 1) // group), dtype=scale_dtype, device=device)
    with torch.cuda.device(q.device):
        check(_lib.load().nq_nit_load_q4g(os.fsencode(path), _ptr(q), _ptr(s), _dtype_code(s, "scale"), group,
                                          out, k, _stream()))
    return Q4GTensor(q, s, out, k, group)


def lm_head_argmax(x: torch.Tensor, w: QTensor, bias=None) -> torch.Tensor:
    """Greedy next-token ids (int64 [m]) = argmax of linear_q8(x, w, bias) in
    fp32, with the reference's first-index / NaN rules (sampling.cpp:14-20),
    without materialising the logits (cuda_quant.cu:357-379 -> sampling.cpp:95)."""
    w.check()
    x = _x2d(x, w.in_, "lm_head_argmax")
    b = _bias(bias, w.out)
    m = x.shape[0]
    ids = torch.empty(m, dtype=torch.int64, device=x.device)
    lib = _lib.load()
    ws = _workspace(lib.nq_lm_head_argmax_q8_workspace_size(m, w.out, w.in_), x.device)
    check(lib.nq_lm_head_argmax_q8(_ptr(x), _dtype_code(x, "x"), _ptr(w.q), _ptr(w.scale), _ptr(b), _ptr(ids),
                                   m, w.out, w.in_, _ptr(ws), ws.numel(), _stream()))
    return ids


def _workspace(nbytes: int, device) -> torch.Tensor:
    # 256-byte aligned by the caching allocator; at least one element.
    return torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)


def linear_w8a8(x: torch.Tensor, w: QTensor, bias=None, out_dtype=None, path: int = NQ_PATH_AUTO):
    """quant.cpp:165-210 / cuda_quant.cu:250-284."""
    w.check()
    x = _x2d(x, w.in_, "linear_w8a8")
    b = _bias(bias, w.out)
    lib = _lib.load()
    m = x.shape[0]
    y = torch.empty((m, w.out), dtype=out_dtype or x.dtype, device=x.device)
    nbytes = lib.nq_linear_w8a8_workspace_size(m, w.out, w.in_)
    ws = _workspace(nbytes, x.device)
    check(lib.nq_linear_w8a8(_ptr(x), _dtype_code(x, "x"), _ptr(w.q), _ptr(w.scale), _ptr(b), _ptr(y),
                             _dtype_code(y, "y"), m, w.out, w.in_, _ptr(ws), ws.numel(), path, _stream()))
    return y


def gemm_w8a8(xq, a_scale, w: QTensor, bias=None, out_dtype=torch.float16, path: int = NQ_PATH_AUTO):
    """W8A8 on pre-quantized activations (the GEMM half of cuda_linear_w8a8)."""
    w.check()
    xq = _dev(xq, "xq")
    m = xq.shape[0]
    b = _bias(bias, w.out)
    lib = _lib.load()
    y = torch.empty((m, w.out), dtype=out_dtype, device=xq.device)
    ws = _workspace(lib.nq_gemm_w8a8_workspace_size(m, w.out, w.in_), xq.device)
    check(lib.nq_gemm_w8a8(_ptr(xq), _ptr(a_scale), _ptr(w.q), _ptr(w.scale), _ptr(b), _ptr(y),
                           _dtype_code(y, "y"), m, w.out, w.in_, _ptr(ws), ws.numel(), path, _stream()))
    return y


def w8a8_acc_i32(xq: torch.Tensor, wq: torch.Tensor, path: int = NQ_PATH_AUTO) -> torch.Tensor:
    """Exact int32 accumulators sum_j xq[i,j]*wq[o,j] of the chosen kernel path."""
    xq = _dev(xq, "xq")
    wq = _dev(wq, "wq")
    if xq.shape[1] != wq.shape[1]:
        raise ValueError("w8a8_acc_i32: k mismatch")
    m, k = xq.shape
    n = wq.shape[0]
    lib = _lib.load()
    acc = torch.empty((m, n), dtype=torch.int32, device=xq.device)
    ws = _workspace(lib.nq_gemm_w8a8_workspace_size(m, n, k), xq.device)
    check(lib.nq_w8a8_acc_i32(_ptr(xq), _ptr(wq), _ptr(acc), m, n, k, _ptr(ws), ws.numel(), path, _stream()))
    return acc


def embedding_q8(table: QTensor, ids, out_dtype=torch.float32) -> torch.Tensor:
    """quant.cpp:121-134 / cuda_quant.cu:286-298: ids is a host sequence."""
    import ctypes

    import numpy as np

    table.check()
    ids_np = np.ascontiguousarray(np.asarray(ids, dtype=np.int64).reshape(-1))
    out = torch.empty((ids_np.size, table.in_), dtype=out_dtype, device=table.q.device)
    check(_lib.load().nq_embedding_q8(_ptr(table.q), _ptr(table.scale), table.out, table.in_,
                                      ids_np.ctypes.data_as(ctypes.c_void_p), ids_np.size, _ptr(out),
                                      _dtype_code(out, "out"), _stream()))
    return out


def dequantize_q8(w: QTensor, out_dtype=torch.float32) -> torch.Tensor:
    """quant.cpp:110-119: w[o, j] = float(q[o, j]) * scale[o] (nq_dequantize_q8)."""
    w.check()
    y = torch.empty((w.out, w.in_), dtype=out_dtype, device=w.q.device)
    check(_lib.load().nq_dequantize_q8(_ptr(w.q), _ptr(w.scale), w.out, w.in_, _ptr(y),
                                       _dtype_code(y, "out"), _stream()))
    return y


def dequantize_q4g(w: Q4GTensor, out_dtype=torch.float32) -> torch.Tensor:
    """quant.cpp:323-335: w[o, j] = float(nib - 8) * scale[o, j / group] (nq_dequantize_q4g)."""
    w.check()
    y = torch.empty((w.out, w.in_), dtype=out_dtype, device=w.q.device)
    check(_lib.load().nq_dequantize_q4g(_ptr(w.q), _ptr(w.scale), _dtype_code(w.scale, "scale"), w.group,
                                        w.out, w.in_, _ptr(y), _dtype_code(y, "out"), _stream()))
    return y


# ---- Weight / factory (quant.hpp:120-141, backend.hpp:109-114) -------------------------
class Weight:
    """Polymorphic device weight (quant.hpp:120-133)."""

    def linear(self, x, bias=None):
        raise NotImplementedError

    def gather(self, ids):
        """quant.cpp:473-475: only the embedding weight gathers."""
        raise RuntimeError("Weight::gather: this weight is not an embedding table")

    def format(self) -> Format:
        raise NotImplementedError

    def bytes(self) -> int:
        raise NotImplementedError

    def fp32_bytes(self) -> int:
        raise NotImplementedError


class _Q8Weight(Weight):
    fmt = Format.Q8

    def __init__(self, t: QTensor):
        self.t = t

    def linear(self, x, bias=None):
        return linear_q8(x, self.t, bias)

    def format(self):
        return self.fmt

    def bytes(self):
        return self.t.q.numel() + self.t.scale.numel() * 4

    def fp32_bytes(self):
        return self.t.out * self.t.in_ * 4


class _W8A8Weight(_Q8Weight):
    fmt = Format.W8A8

    def linear(self, x, bias=None):
        return linear_w8a8(x, self.t, bias)


@dataclass
class Policy:
    """Kernel-selection knobs of the int8 embedding / LM-head weight, the two
    CudaPolicy fields (cuda_backend.hpp:43-89) that reach the quantized path:
    use_w8a8_lmhead runs the LM head's prefill linear (m > 8, the decode GEMV's
    batch) as W8A8 on the same int8 codes (cuda_quant.cu:362-372; opt-in: the
    activation quant can flip a close greedy token); force_tiled_q8 runs its
    weight-only linear on the MFMA GEMM at any m (cuda_quant.cu:308, A/B only)."""
    use_w8a8_lmhead: bool = False
    force_tiled_q8: bool = False


_POLICY = Policy()


def policy() -> Policy:
    """The process-wide policy (mutable, as the reference's cuda_policy())."""
    return _POLICY


GEMV_MAX_M = 8  # decode GEMV batch: rows beyond it are prefill (the reference's kGemvMaxM)


def lm_head_linear(x: torch.Tensor, t: QTensor, bias=None, out_dtype=None) -> torch.Tensor:
    """The int8 embedding's linear under policy() (CudaEmbedQ8Weight::linear,
    cuda_quant.cu:362-372)."""
    pol = policy()
    if pol.use_w8a8_lmhead and x.shape[0] > GEMV_MAX_M:
        return linear_w8a8(x, t, bias, out_dtype)
    return linear_q8(x, t, bias, out_dtype, _lib.NQ_PATH_MFMA if pol.force_tiled_q8 else NQ_PATH_AUTO)


class _EmbedQ8Weight(_Q8Weight):
    def linear(self, x, bias=None):
        return lm_head_linear(x, self.t, bias)

    def gather(self, ids):
        return embedding_q8(self.t, ids)


class _Q4GWeight(Weight):
    def __init__(self, t: Q4GTensor, fmt: Format):
        self.t = t
        self.fmt = fmt

    def linear(self, x, bias=None):
        return linear_q4g(x, self.t, bias)

    def format(self):
        return self.fmt

    def bytes(self):
        return self.t.q.numel() + self.t.scale.numel() * self.t.scale.element_size()

    def fp32_bytes(self):
        return self.t.out * self.t.in_ * 4


def make_quantized(w: torch.Tensor, mode: QuantMode):
    """quant.cpp:460-469 / the device factory CudaBackend::make_quant_weight
    (cuda_quant.cu:390-395) — here every mode is device-resident."""
    mode = QuantMode(mode)
    if mode == QuantMode.Q8:
        return _Q8Weight(quantize_q8(w))
    if mode == QuantMode.Q4:
        return _Q4GWeight(quantize_q4(w), Format.Q4)
    if mode == QuantMode.Q4G:
        return _Q4GWeight(quantize_q4g(w, 32), Format.Q4G)
    if mode == QuantMode.W8A8:
        return _W8A8Weight(quantize_q8(w))
    return None


def make_q8_embed(w: torch.Tensor) -> Weight:
    """quant.cpp:477-479 / make_cuda_q8_embed (cuda_quant.cu:382-388)."""
    return _EmbedQ8Weight(quantize_q8(w))
