"""CPU oracle for the quantized-weight matrix path — TEST INFRASTRUCTURE ONLY.

numpy front-end over two C libraries with one function table:

* ``liboracle.so``  — the plain-C restatement in ``nq_oracle.c`` (always built);
* ``_ref/libnqref.so`` — the reference's own ``cpp/src/quant.cpp`` compiled from
  its sources (``Makefile`` target ``ref``; present only where it was built).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker or the timed CPU baseline.
The product (``nanoinfer_amd``) never imports it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libnqref.so")
REF_SRC = "/root/reference/cpp/src"

_P = ctypes.c_void_p
_I = ctypes.c_int64

_SIGS = {
    "quantize_q8": [_P, _I, _I, _P, _P],
    "dequantize_q8": [_P, _P, _I, _I, _P],
    "embedding_q8": [_P, _P, _I, _I, _P, _I, _P],
    "linear_q8": [_P, _I, _P, _P, _I, _I, _P, _P],
    "linear_w8a8": [_P, _I, _P, _P, _I, _I, _P, _P],
    "w8a8_acc": [_P, _I, _P, _I, _I, _P],
    "quantize_q4g": [_P, _I, _I, _I, _P, _P],
    "dequantize_q4g": [_P, _P, _I, _I, _I, _P],
    "linear_q4g": [_P, _I, _P, _P, _I, _I, _I, _P, _P],
    "quantize_q4": [_P, _I, _I, _P, _P],
    "linear_q4": [_P, _I, _P, _P, _I, _I, _P, _P],
    "linear_f32": [_P, _I, _P, _I, _I, _P, _P],
}


def build(ref: bool | None = None) -> None:
    """Compile liboracle.so (and the reference build when its sources exist)."""
    targets = ["all"]
    if ref or (ref is None and os.path.isdir(REF_SRC)):
        targets.append("ref")
    subprocess.run(["make", "-s", "-C", HERE, *targets], check=True)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


class OracleError(ValueError):
    """Raised where the reference throws std::invalid_argument."""


class CpuQuant:
    """One CPU implementation of the quant path (restatement or reference build)."""

    def __init__(self, path: str, prefix: str, kind: str):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} not built (run `make -C {HERE}`)")
        self.kind = kind
        self.path = path
        self._lib = ctypes.CDLL(path)
        self._fn = {}
        for name, args in _SIGS.items():
            f = getattr(self._lib, prefix + name)
            f.argtypes = args
            f.restype = ctypes.c_int
            self._fn[name] = f
        self._unpack = getattr(self._lib, prefix + "unpack_q4")
        self._unpack.argtypes = [_P, _P, _I]
        self._unpack.restype = None
        self._maxt = getattr(self._lib, prefix + "max_threads")
        self._maxt.restype = ctypes.c_int
        self._sett = getattr(self._lib, prefix + "set_threads")
        self._sett.argtypes = [ctypes.c_int]
        self._sett.restype = None

    def _call(self, name, *args):
        rc = self._fn[name](*args)
        if rc != 0:
            raise OracleError(f"{self.kind}.{name}: invalid argument")

    # threads -------------------------------------------------------------
    def max_threads(self) -> int:
        return int(self._maxt())

    def set_threads(self, n: int) -> None:
        self._sett(int(n))

    # Q8 ------------------------------------------------------------------
    def quantize_q8(self, w):
        w = _f32(w)
        out, k = w.shape
        q = np.empty((out, k), np.int8)
        s = np.empty(out, np.float32)
        self._call("quantize_q8", _ptr(w), out, k, _ptr(q), _ptr(s))
        return q, s

    def dequantize_q8(self, q, s):
        q = np.ascontiguousarray(q, np.int8)
        s = _f32(s)
        w = np.empty(q.shape, np.float32)
        self._call("dequantize_q8", _ptr(q), _ptr(s), q.shape[0], q.shape[1], _ptr(w))
        return w

    def embedding_q8(self, q, s, ids):
        q = np.ascontiguousarray(q, np.int8)
        s = _f32(s)
        ids = np.ascontiguousarray(ids, np.int64)
        out = np.empty((ids.size, q.shape[1]), np.float32)
        self._call("embedding_q8", _ptr(q), _ptr(s), q.shape[0], q.shape[1], _ptr(ids), ids.size, _ptr(out))
        return out

    def linear_q8(self, x, q, s, bias=None):
        x = _f32(x)
        q = np.ascontiguousarray(q, np.int8)
        s = _f32(s)
        b = None if bias is None else _f32(bias)
        m, k = x.shape
        n = q.shape[0]
        y = np.empty((m, n), np.float32)
        self._call("linear_q8", _ptr(x), m, _ptr(q), _ptr(s), n, k, _ptr(b), _ptr(y))
        return y

    def act_quant(self, x):
        return self.quantize_q8(x)

    def w8a8_acc(self, xq, wq):
        xq = np.ascontiguousarray(xq, np.int8)
        wq = np.ascontiguousarray(wq, np.int8)
        m, k = xq.shape
        n = wq.shape[0]
        acc = np.empty((m, n), np.int32)
        self._call("w8a8_acc", _ptr(xq), m, _ptr(wq), n, k, _ptr(acc))
        return acc

    def linear_w8a8(self, x, wq, ws, bias=None):
        x = _f32(x)
        wq = np.ascontiguousarray(wq, np.int8)
        ws = _f32(ws)
        b = None if bias is None else _f32(bias)
        m, k = x.shape
        n = wq.shape[0]
        y = np.empty((m, n), np.float32)
        self._call("linear_w8a8", _ptr(x), m, _ptr(wq), _ptr(ws), n, k, _ptr(b), _ptr(y))
        return y

    # Q4 / Q4G ------------------------------------------------------------
    def quantize_q4g(self, w, group=32):
        w = _f32(w)
        out, k = w.shape
        nb = (k + group - 1) // group if group > 0 else 0
        q = np.zeros((out, (k + 1) // 2), np.uint8)
        s = np.empty((out, max(nb, 0)), np.float32)
        self._call("quantize_q4g", _ptr(w), out, k, group, _ptr(q), _ptr(s))
        return q, s

    def dequantize_q4g(self, q, s, k, group):
        q = np.ascontiguousarray(q, np.uint8)
        s = _f32(s)
        w = np.empty((q.shape[0], k), np.float32)
        self._call("dequantize_q4g", _ptr(q), _ptr(s), q.shape[0], k, group, _ptr(w))
        return w

    def linear_q4g(self, x, q, s, group, bias=None):
        x = _f32(x)
        q = np.ascontiguousarray(q, np.uint8)
        s = _f32(s)
        b = None if bias is None else _f32(bias)
        m, k = x.shape
        n = q.shape[0]
        y = np.empty((m, n), np.float32)
        self._call("linear_q4g", _ptr(x), m, _ptr(q), _ptr(s), n, k, group, _ptr(b), _ptr(y))
        return y

    def quantize_q4(self, w):
        w = _f32(w)
        out, k = w.shape
        q = np.zeros((out, (k + 1) // 2), np.uint8)
        s = np.empty(out, np.float32)
        self._call("quantize_q4", _ptr(w), out, k, _ptr(q), _ptr(s))
        return q, s

    def linear_q4(self, x, q, s, bias=None):
        x = _f32(x)
        q = np.ascontiguousarray(q, np.uint8)
        s = _f32(s)
        b = None if bias is None else _f32(bias)
        m, k = x.shape
        n = q.shape[0]
        y = np.empty((m, n), np.float32)
        self._call("linear_q4", _ptr(x), m, _ptr(q), _ptr(s), n, k, _ptr(b), _ptr(y))
        return y

    def unpack_q4(self, packed, n):
        packed = np.ascontiguousarray(packed, np.uint8)
        out = np.empty(n, np.int8)
        self._unpack(_ptr(packed), _ptr(out), n)
        return out

    def linear_f32(self, x, w, bias=None):
        x = _f32(x)
        w = _f32(w)
        b = None if bias is None else _f32(bias)
        m, k = x.shape
        n = w.shape[0]
        y = np.empty((m, n), np.float32)
        self._call("linear_f32", _ptr(x), m, _ptr(w), n, k, _ptr(b), _ptr(y))
        return y


_cache: dict[str, CpuQuant] = {}


def oracle() -> CpuQuant:
    """The C restatement (builds it on first use if missing)."""
    if "port" not in _cache:
        if not os.path.exists(ORACLE_SO):
            build(ref=False)
        _cache["port"] = CpuQuant(ORACLE_SO, "nqo_", "port")
    return _cache["port"]


def reference() -> CpuQuant | None:
    """The reference's own quant.cpp build, or None where it was not built."""
    if "reference" not in _cache:
        if not os.path.exists(REF_SO):
            return None
        _cache["reference"] = CpuQuant(REF_SO, "nqr_", "reference")
    return _cache["reference"]


class RefOps:
    """The reference's own ops.cpp functions (rmsnorm, RoPE, attention, silu)
    from the reference build, used only by tests/golden/gen_golden.py to write
    the fixtures that pin tests/model_ref.py's numpy restatements."""

    def __init__(self, path: str):
        L = ctypes.CDLL(path)
        F = ctypes.c_float
        sig = {
            "nqr_rmsnorm": [_P, _I, _I, _P, F, _P],
            "nqr_rope_cache": [_I, _I, F, _P, _P],
            "nqr_apply_rope": [_P, _I, _I, _I, _P, _P, _I, _I, _P],
            "nqr_attention": [_P, _P, _P, _I, _I, _I, _I, ctypes.c_int, _I, _P],
            "nqr_silu": [_P, _I, _P],
        }
        self._f = {}
        for name, args in sig.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = ctypes.c_int
            self._f[name] = f

    def _call(self, name, *args):
        if self._f[name](*args) != 0:
            raise OracleError(f"reference.{name}: invalid argument")

    def rmsnorm(self, x, w, eps):
        x, w = _f32(x), _f32(w)
        y = np.empty_like(x)
        self._call("nqr_rmsnorm", _ptr(x), x.shape[0], x.shape[1], _ptr(w), float(eps), _ptr(y))
        return y

    def rope_cache(self, seq, head_dim, theta):
        c = np.empty((seq, head_dim), np.float32)
        s = np.empty((seq, head_dim), np.float32)
        self._call("nqr_rope_cache", seq, head_dim, float(theta), _ptr(c), _ptr(s))
        return c, s

    def apply_rope(self, x, cos, sin, pos_offset=0):
        x, cos, sin = _f32(x), _f32(cos), _f32(sin)
        y = np.empty_like(x)
        self._call("nqr_apply_rope", _ptr(x), *x.shape, _ptr(cos), _ptr(sin), cos.shape[0], pos_offset, _ptr(y))
        return y

    def attention(self, q, k, v, causal=True, query_offset=0):
        q, k, v = _f32(q), _f32(k), _f32(v)
        y = np.empty_like(q)
        self._call("nqr_attention", _ptr(q), _ptr(k), _ptr(v), q.shape[0], q.shape[1], k.shape[1], q.shape[2],
                   int(causal), query_offset, _ptr(y))
        return y

    def silu(self, x):
        x = _f32(x)
        y = np.empty_like(x)
        self._call("nqr_silu", _ptr(x), x.size, _ptr(y))
        return y


def reference_ops() -> RefOps | None:
    """ops.cpp from the reference build, or None where it was not built."""
    if not os.path.exists(REF_SO):
        return None
    return RefOps(REF_SO)
