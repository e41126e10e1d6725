"""qwen3x_amd -- MI355X (gfx950) HIP backend for qwen3x's quantized weight matmul.

The work is done by ``libq3x_hip.so`` (C ABI declared in ``include/q3x_hip.h``);
this module binds it with ctypes and offers the reference's host-side
operations (arch/cuda/engine.cu ``mv`` :1531, ``mv_add`` :1547, ``batch_mv``
:1568, ``embed`` :1499, ``router_top_k_kernel`` :1153 and the routed part of
``moe`` :1709) on torch device tensors.  torch supplies device memory and the
current stream only; there is no torch or CPU fallback: every call goes to the
HIP library and raises if it is missing or returns an error.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from typing import Optional

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG_DIR, "libq3x_hip.so")

MATRIX_BF16 = 0
MATRIX_Q8_0 = 1
MATRIX_Q4_0 = 2
BLOCK = 32
BLOCK_BYTES = {MATRIX_Q8_0: 34, MATRIX_Q4_0: 18}

OK = 0
EINVAL = -1
ERUNTIME = -2
ENOTSUP = -3

# Every entry point of include/q3x_hip.h: name -> (restype, argtypes).
_P = ctypes.c_void_p
_I = ctypes.c_int
_U = ctypes.c_uint32
_S = ctypes.c_size_t
SIGNATURES = {
    "q3x_hip_strerror": (ctypes.c_char_p, [_I]),
    "q3x_hip_quantized_bytes": (_I, [_U, _I, _I, ctypes.POINTER(_S)]),
    "q3x_hip_mv": (_I, [_P, _U, _I, _I, _P, _P, _I, _P]),
    "q3x_hip_mv_multi": (_I, [_P, _I, _U, _I, _P, _P]),
    "q3x_hip_gemm": (_I, [_P, _U, _I, _I, _P, _I, _P, _I, _P]),
    "q3x_hip_dequant": (_I, [_P, _U, _I, _I, _I, _P, _P]),
    "q3x_hip_router_topk": (_I, [_P, _I, _I, _I, _P, _P, _P]),
    "q3x_hip_moe_workspace_bytes": (_S, [_I, _I, _I, _I, _I]),
    "q3x_hip_moe_routed": (_I, [_P, _P, _U, _I, _I, _I, _P, _I, _P, _P, _I, _P, _I, _P, _S, _P]),
    "q3x_hip_quantize": (_I, [_U, _P, _I, _I, _P, _P]),
    "q3x_hip_moe_layer_workspace_bytes": (_S, [_P, _I]),
    "q3x_hip_moe_layer": (_I, [_P, _P, _I, _P, _P, _P, _P, _S, _P]),
}


MV_MULTI_MAX = 8


class MoeLayerWeights(ctypes.Structure):
    """struct q3x_hip_moe_layer_weights of include/q3x_hip.h."""
    _fields_ = [("router", ctypes.c_void_p), ("gate_up", ctypes.c_void_p), ("down", ctypes.c_void_p),
                ("shared_gate", ctypes.c_void_p), ("shared_up", ctypes.c_void_p),
                ("shared_down", ctypes.c_void_p), ("shared_scale", ctypes.c_void_p), ("type", ctypes.c_uint32),
                ("experts", ctypes.c_int), ("top_k", ctypes.c_int), ("H", ctypes.c_int), ("I", ctypes.c_int),
                ("shared_I", ctypes.c_int)]


class MvItem(ctypes.Structure):
    """struct q3x_hip_mv_item of include/q3x_hip.h."""
    _fields_ = [("weight", ctypes.c_void_p), ("rows", ctypes.c_int), ("out", ctypes.c_void_p),
                ("accumulate", ctypes.c_int)]


class Q3xHipError(RuntimeError):
    def __init__(self, func: str, code: int, message: str):
        super().__init__(f"{func} failed: {message} ({code})")
        self.code = code


_lib = None


def lib() -> ctypes.CDLL:
    """Load libq3x_hip.so (built in-tree by ``make -C qwen3x_amd``)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `make -C {_PKG_DIR}` "
                "(or __graft_entry__.build()); there is no fallback path")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def strerror(code: int) -> str:
    return lib().q3x_hip_strerror(code).decode()


def _check(func: str, code: int) -> None:
    if code != OK:
        raise Q3xHipError(func, code, strerror(code))


def quantized_bytes(type_: int, rows: int, cols: int) -> Optional[int]:
    """Exact matrix byte size, or None when arch/cpu.cpp:161-179 rejects the shape."""
    out = ctypes.c_size_t(0)
    code = lib().q3x_hip_quantized_bytes(type_, rows, cols, ctypes.byref(out))
    return out.value if code == OK else None


def moe_workspace_bytes(tokens: int, experts: int, top_k: int, H: int, I: int) -> int:
    return lib().q3x_hip_moe_workspace_bytes(tokens, experts, top_k, H, I)


# ---------------------------------------------------------------- torch side

def _torch():
    import torch
    return torch


def _stream(stream=None) -> int:
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def _ptr(t) -> int:
    return t.data_ptr()


def _need_device(*tensors):
    for t in tensors:
        if not t.is_cuda:
            raise ValueError("qwen3x_amd operates on device tensors only")


@dataclass
class Linear:
    """One quantised matrix W[rows, columns] (reference engine.cu:68-73).

    ``weight`` is a uint8 device tensor holding the blocks."""
    weight: "object"
    rows: int
    columns: int
    type: int


@dataclass
class ExpertLinear:
    """Contiguous experts W[experts, rows, columns] (reference engine.cu:89-95)."""
    weight: "object"
    experts: int
    rows: int
    columns: int
    type: int


def mv(linear: Linear, x, y, accumulate: bool = False, stream=None):
    """y[rows] = W x, or y += W x with ``accumulate`` (mv / mv_add)."""
    _need_device(linear.weight, x, y)
    _check("q3x_hip_mv", lib().q3x_hip_mv(_ptr(linear.weight), linear.type, linear.rows, linear.columns,
                                          _ptr(x), _ptr(y), int(accumulate), _stream(stream)))
    return y


def mv_add(linear: Linear, x, y, stream=None):
    return mv(linear, x, y, True, stream)


def mv_multi(linears, x, outs, accumulate=None, stream=None):
    """outs[i] (+)= linears[i] x for matrices of one type and width, one launch
    (the projection helpers attention_projections / ffn_projections /
    delta_projections, engine.cu:1599-1661)."""
    n = len(linears)
    if n != len(outs) or not 1 <= n <= MV_MULTI_MAX:
        raise ValueError(f"mv_multi takes 1..{MV_MULTI_MAX} matrices with one output each")
    accumulate = accumulate or [False] * n
    first = linears[0]
    for m in linears:
        if m.type != first.type or m.columns != first.columns:
            raise ValueError("mv_multi: every matrix must share the type and the width")
    _need_device(x, *outs, *(m.weight for m in linears))
    items = (MvItem * n)(*[MvItem(_ptr(m.weight), m.rows, _ptr(o), int(a))
                           for m, o, a in zip(linears, outs, accumulate)])
    _check("q3x_hip_mv_multi", lib().q3x_hip_mv_multi(ctypes.cast(items, ctypes.c_void_p), n, first.type,
                                                      first.columns, _ptr(x), _stream(stream)))
    return outs


def batch_mv(linear: Linear, X, Y, count: int, add: bool = False, stream=None):
    """Y[count, rows] (+)= X[count, columns] W^T (prefill GEMM)."""
    _need_device(linear.weight, X, Y)
    _check("q3x_hip_gemm", lib().q3x_hip_gemm(_ptr(linear.weight), linear.type, linear.rows, linear.columns,
                                              _ptr(X), count, _ptr(Y), int(add), _stream(stream)))
    return Y


def dequant(linear: Linear, row0: int, nrows: int, out, stream=None):
    """out[nrows, columns] = dequantised rows [row0, row0 + nrows)."""
    _need_device(linear.weight, out)
    _check("q3x_hip_dequant", lib().q3x_hip_dequant(_ptr(linear.weight), linear.type, linear.columns, row0,
                                                    nrows, _ptr(out), _stream(stream)))
    return out


def embed(table: Linear, token: int, out, stream=None):
    if not 0 <= token < table.rows:
        raise ValueError(f"embedding token={token} rows={table.rows}")
    return dequant(table, token, 1, out, stream)


def router_top_k(logits, tokens: int, experts: int, top_k: int, ids, weights, stream=None):
    _need_device(logits, ids, weights)
    _check("q3x_hip_router_topk", lib().q3x_hip_router_topk(_ptr(logits), tokens, experts, top_k, _ptr(ids),
                                                            _ptr(weights), _stream(stream)))
    return ids, weights


def moe_routed(gate_up: ExpertLinear, down: ExpertLinear, X, tokens: int, ids, weights, top_k: int, Y,
               accumulate: bool = False, workspace=None, stream=None):
    """Routed experts: Y (+)= sum_slot w * down_e(silu(gate_e x) * up_e x)."""
    torch = _torch()
    _need_device(gate_up.weight, down.weight, X, ids, weights, Y)
    H, I = gate_up.columns, down.columns
    need = moe_workspace_bytes(tokens, gate_up.experts, top_k, H, I)
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=X.device)
    _check("q3x_hip_moe_routed",
           lib().q3x_hip_moe_routed(_ptr(gate_up.weight), _ptr(down.weight), gate_up.type, gate_up.experts, H, I,
                                    _ptr(X), tokens, _ptr(ids), _ptr(weights), top_k, _ptr(Y), int(accumulate),
                                    _ptr(workspace), workspace.numel(), _stream(stream)))
    return Y


@dataclass
class MoeLayer:
    """The weights of one MoE layer (reference MoeWeights, engine.cu:97-101):
    BF16 router [experts, H] and shared_scale [1, H] as uint16 device tensors,
    routed experts gate_up [experts, 2I, H] / down [experts, H, I] and the
    shared expert gate/up [shared_I, H] / down [H, shared_I] as uint8 block
    tensors of `type`."""
    router: "object"
    gate_up: "object"
    down: "object"
    shared_gate: "object"
    shared_up: "object"
    shared_down: "object"
    shared_scale: "object"
    type: int
    experts: int
    top_k: int
    H: int
    I: int
    shared_I: int

    def c_struct(self) -> MoeLayerWeights:
        return MoeLayerWeights(_ptr(self.router), _ptr(self.gate_up), _ptr(self.down), _ptr(self.shared_gate),
                               _ptr(self.shared_up), _ptr(self.shared_down), _ptr(self.shared_scale), self.type,
                               self.experts, self.top_k, self.H, self.I, self.shared_I)


def moe_layer_workspace_bytes(layer: MoeLayer, tokens: int) -> int:
    return lib().q3x_hip_moe_layer_workspace_bytes(ctypes.byref(layer.c_struct()), tokens)


def moe_layer(layer: MoeLayer, X, tokens: int, Y, ids=None, weights=None, workspace=None, stream=None):
    """The whole MoE layer (engine.cpp:406-430): Y = routed experts + sigmoid-gated shared expert."""
    torch = _torch()
    _need_device(X, Y, layer.router, layer.gate_up, layer.down, layer.shared_gate, layer.shared_up,
                 layer.shared_down, layer.shared_scale)
    if workspace is None:
        workspace = torch.empty(moe_layer_workspace_bytes(layer, tokens), dtype=torch.uint8, device=X.device)
    c = layer.c_struct()
    _check("q3x_hip_moe_layer",
           lib().q3x_hip_moe_layer(ctypes.byref(c), _ptr(X), tokens, _ptr(Y), _ptr(ids) if ids is not None else None,
                                   _ptr(weights) if weights is not None else None, _ptr(workspace),
                                   workspace.numel(), _stream(stream)))
    return Y


def quantize(type_: int, src, rows: int, cols: int, dst, stream=None):
    """dst = Q8_0/Q4_0 blocks of src[rows, cols] (scripts/pack_weights.py quantizers)."""
    _need_device(src, dst)
    _check("q3x_hip_quantize", lib().q3x_hip_quantize(type_, _ptr(src), rows, cols, _ptr(dst), _stream(stream)))
    return dst
