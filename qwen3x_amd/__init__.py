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
EMODEL = -4
ESCRATCH = -5
ESTATE = -6
# Static per-device scratch of q3x_hip_moe_routed_noalloc (Q3X_HIP_NOALLOC_SCRATCH_BYTES).
NOALLOC_SCRATCH_BYTES = 32 << 20

TENSOR_F32 = 3
MODEL_HEADER_BYTES = 72
# Tensor roles of model.bin, in the order of include/q3x_hip.h's enumeration.
TENSOR_ROLES = ("embedding", "lm_head", "final_norm", "input_norm", "post_norm",
                "delta_qkv", "delta_z", "delta_a", "delta_b", "delta_conv", "delta_alog", "delta_dt",
                "delta_norm", "delta_out", "attn_q", "attn_k", "attn_v", "attn_qnorm", "attn_knorm", "attn_out",
                "ffn_gate", "ffn_up", "ffn_down", "moe_router", "moe_gate_up", "moe_down", "moe_shared_gate",
                "moe_shared_up", "moe_shared_down", "moe_shared_scale")

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
    "q3x_hip_gemm_workspace_bytes": (_S, [_U, _I, _I, _I]),
    "q3x_hip_gemm_ws": (_I, [_P, _U, _I, _I, _P, _I, _P, _I, _P, _S, _P]),
    "q3x_hip_dequant": (_I, [_P, _U, _I, _I, _I, _P, _P]),
    "q3x_hip_router_topk": (_I, [_P, _I, _I, _I, _P, _P, _P]),
    "q3x_hip_moe_workspace_bytes": (_S, [_I, _I, _I, _I, _I]),
    "q3x_hip_moe_routed": (_I, [_P, _P, _U, _I, _I, _I, _P, _I, _P, _P, _I, _P, _I, _P, _S, _P]),
    "q3x_hip_moe_routed_noalloc": (_I, [_P, _P, _U, _I, _I, _I, _P, _I, _P, _P, _I, _P, _I, _P]),
    "q3x_hip_moe_routed_logits": (_I, [_P, _P, _U, _I, _I, _I, _P, _I, _P, _I, _P, _P, _P, _I, _P, _S, _P]),
    "q3x_hip_quantize": (_I, [_U, _P, _I, _I, _P, _P]),
    "q3x_hip_moe_layer_workspace_bytes": (_S, [_P, _I]),
    "q3x_hip_moe_layer": (_I, [_P, _P, _I, _P, _P, _P, _P, _S, _P]),
    "q3x_hip_quantize_bf16": (_I, [_U, _P, _I, _I, _P, _P]),
    "q3x_hip_read_probe": (_I, [_P, _S, _P, _P]),
    "q3x_hip_model_layout": (_I, [_P, _S, ctypes.c_uint64, _P, _P, _S, ctypes.POINTER(_S),
                                  ctypes.POINTER(ctypes.c_char_p)]),
    "q3x_hip_model_load": (_I, [ctypes.c_char_p, ctypes.POINTER(_P), ctypes.POINTER(ctypes.c_char_p)]),
    "q3x_hip_model_free": (None, [_P]),
    "q3x_hip_model_info": (_I, [_P, _P, ctypes.POINTER(_P), ctypes.POINTER(_S), ctypes.POINTER(_P),
                                ctypes.POINTER(ctypes.c_uint64)]),
    "q3x_hip_model_tensor": (_I, [_P, _U, _I, _P, ctypes.POINTER(_P)]),
    "q3x_hip_model_moe_layer": (_I, [_P, _I, _P]),
    "q3x_hip_model_schema": (_I, [_P, _P, _S, ctypes.POINTER(_S), ctypes.POINTER(ctypes.c_uint64)]),
    "q3x_hip_engine_create": (_I, [_P, _P, _I, _I, ctypes.POINTER(_P), ctypes.POINTER(ctypes.c_char_p)]),
    "q3x_hip_engine_destroy": (None, [_P]),
    "q3x_hip_engine_reset": (_I, [_P]),
    "q3x_hip_engine_forward": (_I, [_P, _P, _I, _I]),
    "q3x_hip_engine_logits": (_I, [_P, _P]),
    "q3x_hip_engine_argmax": (_I, [_P, ctypes.POINTER(_I)]),
    "q3x_hip_engine_checkpoint_save": (_I, [_P]),
    "q3x_hip_engine_checkpoint_restore": (_I, [_P]),
    "q3x_hip_engine_position": (_I, [_P]),
}


MV_MULTI_MAX = 8


class MoeLayerWeights(ctypes.Structure):
    """struct q3x_hip_moe_layer_weights of include/q3x_hip.h."""
    _fields_ = [("router", ctypes.c_void_p), ("gate_up", ctypes.c_void_p), ("down", ctypes.c_void_p),
                ("shared_gate", ctypes.c_void_p), ("shared_up", ctypes.c_void_p),
                ("shared_down", ctypes.c_void_p), ("shared_scale", ctypes.c_void_p), ("type", ctypes.c_uint32),
                ("experts", ctypes.c_int), ("top_k", ctypes.c_int), ("H", ctypes.c_int), ("I", ctypes.c_int),
                ("shared_I", ctypes.c_int)]


class ModelConfig(ctypes.Structure):
    """struct q3x_hip_model_config of include/q3x_hip.h (model_config.h:47-57)."""
    _fields_ = [("id", ctypes.c_uint32), ("name", ctypes.c_char_p)] + \
        [(f, ctypes.c_int) for f in ("V", "H", "I", "N", "AI", "AH", "KVH", "AD", "RD", "KH", "VH", "KD", "VD",
                                     "CK", "experts", "top_k", "shared_I")] + \
        [("matrix_type", ctypes.c_uint32), ("tied_embeddings", ctypes.c_int)]


class Tensor(ctypes.Structure):
    """struct q3x_hip_tensor of include/q3x_hip.h: one tensor of model.bin."""
    _fields_ = [("role", ctypes.c_uint32), ("layer", ctypes.c_int), ("type", ctypes.c_uint32),
                ("experts", ctypes.c_int), ("rows", ctypes.c_int), ("cols", ctypes.c_int),
                ("offset", ctypes.c_uint64), ("bytes", ctypes.c_uint64)]

    def key(self):
        return TENSOR_ROLES[self.role], self.layer


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
        # torch's ROCm wheel bundles its own libamdhip64 (the same soname).
        # Loaded after torch, this library binds to that runtime; loaded
        # first, it would pull in /opt/rocm's copy and the process would hold
        # two HIP runtimes, whose device memory and streams do not mix with
        # torch's tensors.  So torch, where installed, is loaded first.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
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


class ModelError(Q3xHipError):
    """model.bin rejected or not loaded; ``message`` is the loader's reason."""
    def __init__(self, func: str, code: int, message: str):
        super().__init__(func, code, message)
        self.message = message


def _check_model(func: str, code: int, error: ctypes.c_char_p) -> None:
    if code != OK:
        raise ModelError(func, code, error.value.decode() if error.value else strerror(code))


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


def gemm_workspace_bytes(linear: Linear, count: int) -> int:
    """Bytes of workspace with which batch_mv_ws splits K over workgroups
    for `count` tokens (0: no split)."""
    return int(lib().q3x_hip_gemm_workspace_bytes(linear.type, linear.rows, linear.columns, count))


def batch_mv_ws(linear: Linear, X, Y, count: int, workspace, add: bool = False, stream=None):
    """batch_mv with a workspace (a device tensor of at least
    gemm_workspace_bytes(linear, count) bytes, or None)."""
    _need_device(linear.weight, X, Y)
    ws, nbytes = (0, 0) if workspace is None else (_ptr(workspace), workspace.numel() * workspace.element_size())
    if workspace is not None:
        _need_device(workspace)
    _check("q3x_hip_gemm_ws", lib().q3x_hip_gemm_ws(_ptr(linear.weight), linear.type, linear.rows, linear.columns,
                                                    _ptr(X), count, _ptr(Y), int(add), ws, nbytes,
                                                    _stream(stream)))
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


def moe_routed_logits(gate_up: ExpertLinear, down: ExpertLinear, X, tokens: int, logits, top_k: int, ids,
                      weights, Y, accumulate: bool = False, workspace=None, stream=None):
    """Router top-k on logits, then the routed experts (ids / weights are written)."""
    torch = _torch()
    _need_device(gate_up.weight, down.weight, X, logits, ids, weights, Y)
    H, I = gate_up.columns, down.columns
    need = moe_workspace_bytes(tokens, gate_up.experts, top_k, H, I)
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=X.device)
    _check("q3x_hip_moe_routed_logits",
           lib().q3x_hip_moe_routed_logits(_ptr(gate_up.weight), _ptr(down.weight), gate_up.type, gate_up.experts,
                                           H, I, _ptr(X), tokens, _ptr(logits), top_k, _ptr(ids), _ptr(weights),
                                           _ptr(Y), int(accumulate), _ptr(workspace), workspace.numel(),
                                           _stream(stream)))
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


def quantize_bf16(type_: int, src, rows: int, cols: int, dst, stream=None):
    """dst = Q8_0/Q4_0 blocks of BF16 src[rows, cols] (int16/uint16/bfloat16
    device tensor), the packer's own input type."""
    _need_device(src, dst)
    _check("q3x_hip_quantize_bf16",
           lib().q3x_hip_quantize_bf16(type_, _ptr(src), rows, cols, _ptr(dst), _stream(stream)))
    return dst


def read_probe(buffer, sink, stream=None):
    """A plain streaming read of the device tensor `buffer` (no work on the
    data); sink: a device tensor of at least 4 bytes."""
    _need_device(buffer, sink)
    nbytes = buffer.numel() * buffer.element_size()
    _check("q3x_hip_read_probe", lib().q3x_hip_read_probe(_ptr(buffer), nbytes, _ptr(sink), _stream(stream)))


# ---------------------------------------------------------------- model.bin

def model_layout(header: bytes, file_size: int):
    """Validate a model.bin from its header bytes and size (engine.cpp:481-559
    checks) and return (ModelConfig, [Tensor] in file order).  Host only.
    Raises ModelError with the reference loader's message on rejection."""
    buf = ctypes.create_string_buffer(bytes(header), max(len(header), 1))
    config = ModelConfig()
    count = ctypes.c_size_t(0)
    error = ctypes.c_char_p()
    _check_model("q3x_hip_model_layout",
                 lib().q3x_hip_model_layout(buf, len(header), file_size, ctypes.byref(config), None, 0,
                                            ctypes.byref(count), ctypes.byref(error)), error)
    tensors = (Tensor * count.value)()
    _check_model("q3x_hip_model_layout",
                 lib().q3x_hip_model_layout(buf, len(header), file_size, None, tensors, count.value,
                                            ctypes.byref(count), ctypes.byref(error)), error)
    return config, list(tensors)


class DeviceRegion:
    """A device address range inside a loaded model, usable wherever the
    wrappers take a device tensor (data_ptr / is_cuda); it keeps the model
    alive while referenced."""
    is_cuda = True

    def __init__(self, model: "Model", address: int, nbytes: int):
        self._model = model
        self._address = address
        self.nbytes = nbytes

    def data_ptr(self) -> int:
        if self._model.handle is None:
            raise RuntimeError("the model was closed")
        return self._address

    def numel(self) -> int:
        return self.nbytes


class Model:
    """model.bin loaded into one device buffer of the current device (the
    reference's CUDA Model::load, arch/cuda/engine.cu:2032-2188)."""

    def __init__(self, path: str):
        handle = ctypes.c_void_p()
        error = ctypes.c_char_p()
        _check_model("q3x_hip_model_load",
                     lib().q3x_hip_model_load(os.fsencode(path), ctypes.byref(handle), ctypes.byref(error)), error)
        self.handle = handle
        config = ModelConfig()
        table = ctypes.c_void_p()
        count = ctypes.c_size_t()
        base = ctypes.c_void_p()
        nbytes = ctypes.c_uint64()
        _check("q3x_hip_model_info", lib().q3x_hip_model_info(handle, ctypes.byref(config), ctypes.byref(table),
                                                              ctypes.byref(count), ctypes.byref(base),
                                                              ctypes.byref(nbytes)))
        self.config = config
        self.tensors = list(ctypes.cast(table, ctypes.POINTER(Tensor * count.value)).contents)
        self.base = base.value
        self.nbytes = nbytes.value

    def close(self):
        if self.handle is not None:
            lib().q3x_hip_model_free(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensor(self, role: str, layer: int = -1):
        """(Tensor, DeviceRegion) of `role` in `layer`; a tied lm_head is the embedding."""
        t = Tensor()
        data = ctypes.c_void_p()
        _check("q3x_hip_model_tensor", lib().q3x_hip_model_tensor(self.handle, TENSOR_ROLES.index(role), layer,
                                                                  ctypes.byref(t), ctypes.byref(data)))
        return t, DeviceRegion(self, data.value, t.bytes)

    def linear(self, role: str, layer: int = -1) -> Linear:
        t, region = self.tensor(role, layer)
        return Linear(region, t.rows, t.cols, t.type)

    def expert_linear(self, role: str, layer: int) -> ExpertLinear:
        t, region = self.tensor(role, layer)
        return ExpertLinear(region, t.experts, t.rows, t.cols, t.type)

    def moe_layer(self, layer: int) -> MoeLayer:
        """The MoE weights of `layer`, ready for moe_layer()."""
        w = MoeLayerWeights()
        _check("q3x_hip_model_moe_layer", lib().q3x_hip_model_moe_layer(self.handle, layer, ctypes.byref(w)))
        c = self.config
        H, I, S, E = c.H, c.I, c.shared_I, c.experts
        qb = quantized_bytes
        t = c.matrix_type
        return MoeLayer(DeviceRegion(self, w.router, E * H * 2), DeviceRegion(self, w.gate_up, E * qb(t, 2 * I, H)),
                        DeviceRegion(self, w.down, E * qb(t, H, I)), DeviceRegion(self, w.shared_gate, qb(t, S, H)),
                        DeviceRegion(self, w.shared_up, qb(t, S, H)), DeviceRegion(self, w.shared_down, qb(t, H, S)),
                        DeviceRegion(self, w.shared_scale, H * 2), t, E, c.top_k, H, I, S)


CONFIG_FIELDS = ("id", "V", "H", "I", "N", "AI", "AH", "KVH", "AD", "RD", "KH", "VH", "KD", "VD", "CK", "experts",
                 "top_k", "shared_I", "matrix_type", "tied_embeddings")


def make_config(name: str = "synthetic", **fields) -> ModelConfig:
    """A ModelConfig from keyword fields (CONFIG_FIELDS); unnamed ones are 0."""
    c = ModelConfig()
    c.name = name.encode()
    for k in CONFIG_FIELDS:
        setattr(c, k, int(fields.get(k, 0)))
    return c


def config_dict(c: ModelConfig) -> dict:
    return {k: getattr(c, k) for k in CONFIG_FIELDS}


def model_schema(config: ModelConfig):
    """([Tensor] in file order, file bytes) for any configuration."""
    count = ctypes.c_size_t(0)
    nbytes = ctypes.c_uint64(0)
    _check("q3x_hip_model_schema", lib().q3x_hip_model_schema(ctypes.byref(config), None, 0, ctypes.byref(count),
                                                              ctypes.byref(nbytes)))
    table = (Tensor * count.value)()
    _check("q3x_hip_model_schema", lib().q3x_hip_model_schema(ctypes.byref(config), table, count.value,
                                                              ctypes.byref(count), ctypes.byref(nbytes)))
    return list(table), nbytes.value


class Engine:
    """The decode engine (q3x_hip_engine_*): a model's weights (a device
    buffer in model.bin layout) plus device-resident state for `context`
    tokens.  Mirrors the reference backend's state_* operations
    (internal.h:11-34)."""

    def __init__(self, config: ModelConfig, weights, context: int, chunk: int = 0):
        self.config = config
        self._weights = weights  # keeps the buffer alive
        handle = ctypes.c_void_p()
        error = ctypes.c_char_p()
        ptr = weights if isinstance(weights, int) else _ptr(weights)
        _check_model("q3x_hip_engine_create",
                     lib().q3x_hip_engine_create(ctypes.byref(config), ptr, context, chunk, ctypes.byref(handle),
                                                 ctypes.byref(error)), error)
        self.handle = handle

    @classmethod
    def from_model(cls, model: "Model", context: int, chunk: int = 0) -> "Engine":
        return cls(model.config, DeviceRegion(model, model.base, model.nbytes), context, chunk)

    def close(self):
        if getattr(self, "handle", None) is not None:
            lib().q3x_hip_engine_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def forward(self, tokens, logits: bool = True):
        import numpy as np
        t = np.ascontiguousarray(tokens, np.int32).reshape(-1)
        _check("q3x_hip_engine_forward", lib().q3x_hip_engine_forward(self.handle, t.ctypes.data, t.size, int(logits)))

    def logits(self):
        import numpy as np
        out = np.empty(self.config.V, np.float32)
        _check("q3x_hip_engine_logits", lib().q3x_hip_engine_logits(self.handle, out.ctypes.data))
        return out

    def argmax(self) -> int:
        out = ctypes.c_int(-1)
        _check("q3x_hip_engine_argmax", lib().q3x_hip_engine_argmax(self.handle, ctypes.byref(out)))
        return out.value

    def reset(self):
        _check("q3x_hip_engine_reset", lib().q3x_hip_engine_reset(self.handle))

    def checkpoint_save(self):
        _check("q3x_hip_engine_checkpoint_save", lib().q3x_hip_engine_checkpoint_save(self.handle))

    def checkpoint_restore(self):
        _check("q3x_hip_engine_checkpoint_restore", lib().q3x_hip_engine_checkpoint_restore(self.handle))

    @property
    def position(self) -> int:
        return lib().q3x_hip_engine_position(self.handle)
