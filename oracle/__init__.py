"""CPU parity oracle for qwen3x's quantized matmul path -- TEST INFRASTRUCTURE ONLY.

Python access to ``liboracle.so`` (this repository's C restatement of the
reference CPU path, q3x_oracle.c) and, when it was built, to
``_ref/libq3x_ref.so`` (the reference's own CPU sources compiled where they
lie).  Only tests/, ``__graft_entry__.smoke()`` and bench.py's cpu_baseline
leg may use this package; the product library never does.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_DIR, "liboracle.so")
REF_PATH = os.path.join(_DIR, "_ref", "libq3x_ref.so")
REF_AVX512_PATH = os.path.join(_DIR, "_ref", "libq3x_ref_avx512.so")

Q8_0 = 1
Q4_0 = 2
BLOCK_BYTES = {Q8_0: 34, Q4_0: 18}

_P = ctypes.c_void_p
_I = ctypes.c_int
_U = ctypes.c_uint32
_S = ctypes.c_size_t
_F = ctypes.c_float
_SIGS = {
    "q3xo_f16": (_F, [ctypes.c_uint16]),
    "q3xo_quantized_bytes": (_I, [_U, _I, _I, ctypes.POINTER(_S)]),
    "q3xo_embed": (_I, [_P, _U, _I, _I, _P]),
    "q3xo_mv_rows": (_I, [_P, _U, _I, _I, _I, _P, _P]),
    "q3xo_mv": (_I, [_P, _U, _I, _I, _P, _P, _I]),
    "q3xo_gemm": (_I, [_P, _U, _I, _I, _P, _I, _P, _I]),
    "q3xo_sigmoid": (_F, [_F]),
    "q3xo_silu": (_F, [_F]),
    "q3xo_router_top_k": (_I, [_P, _I, _I, _P, _P, _P]),
    "q3xo_moe_routed": (_I, [_P, _P, _U, _I, _I, _I, _P, _I, _P, _P, _I, _P, _I]),
    "q3xo_quantize": (_I, [_U, _P, _S, _P]),
    "q3xo_mv_bf16": (_I, [_P, _I, _I, _P, _P]),
    "q3xo_moe_layer": (_I, [_P, _P, _P, _P, _P, _P, _P, _U, _I, _I, _I, _I, _I, _P, _I, _P, _P, _P, _I]),
    "q3xo_set_bf16_lanes": (_I, [_I]),
}
_REF_SIGS = {
    "q3xr_quantized_bytes": (_I, [_U, _I, _I, ctypes.POINTER(_S)]),
    "q3xr_try_embed": (_I, [_P, _U, _I, _I, _P]),
    "q3xr_try_mv": (_I, [_P, _U, _I, _I, _P, _P]),
    "q3xr_router_top_k": (None, [_P, _I, _I, _P, _P]),
    "q3xr_sigmoid": (_F, [_F]),
    "q3xr_silu": (_F, [_F]),
    "q3xr_moe_q4": (None, [_P, _P, _P, _I, _I, _I, _I, _P, _P, _P, _P]),
    "q3xr_mv_bf16": (None, [_P, _I, _I, _P, _P]),
    "q3xr_moe_layer": (None, [_U, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P, _P]),
    "q3xr_model_load": (_I, [ctypes.c_char_p, _P, _P, _S, ctypes.POINTER(_S), ctypes.POINTER(ctypes.c_char_p)]),
    "q3xr_forward": (_I, [_P, _P, _P, _P, _P, _I, _P, _I, _P]),
    "q3xr_moe_routed": (None, [_U, _P, _P, _I, _I, _I, _P, _P, _P, _I, _P]),
}

_lib = None
_ref = None


def _bind(path, sigs):
    handle = ctypes.CDLL(path)
    for name, (restype, argtypes) in sigs.items():
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return handle


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C {_DIR}`")
        _lib = _bind(LIB_PATH, _SIGS)
    return _lib


def host_has_avx512() -> bool:
    """Whether this host's CPU reports AVX-512 F and BW (the reference's
    x86 kernels need both, arch/cpu.cpp:112)."""
    try:
        flags = open("/proc/cpuinfo").read().split()
    except OSError:
        return False
    return "avx512f" in flags and "avx512bw" in flags


_builds = {}


def ref_builds():
    """The reference builds this host can run: [(name, handle, bf16_lanes)].
    "x86-64-v3" is the portable build (scalar BF16 dots); "avx512" is built
    with AVX-512 as the reference's -march=native build is on such a host
    (BF16 matvec and FP32 dots through arch/x86/kernels.h)."""
    out = []
    for name, path, lanes, ok in (("x86-64-v3", REF_PATH, 1, True),
                                  ("avx512", REF_AVX512_PATH, 16, host_has_avx512())):
        if ok and os.path.exists(path):
            if name not in _builds:
                _builds[name] = _bind(path, _REF_SIGS)
            out.append((name, _builds[name], lanes))
    return out


def ref():
    """The reference build matching this host's -march=native build: the
    AVX-512 one where the CPU has AVX-512 F and BW, else the portable one;
    None when neither was built (no reference tree)."""
    global _ref
    if _ref is None:
        builds = ref_builds()
        if builds:
            _ref = builds[-1][1]
    return _ref


def ref_variant():
    """(name, bf16_lanes) of the build ref() returns, or None."""
    h = ref()
    for name, handle, lanes in ref_builds():
        if handle is h:
            return name, lanes
    return None


def set_bf16_lanes(lanes: int) -> None:
    """Which reference BF16 dot the oracle restates: 1 (portable loop) or 16
    (AVX-512)."""
    assert lib().q3xo_set_bf16_lanes(lanes)


def default_threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def f16(bits: int) -> float:
    return float(lib().q3xo_f16(bits))


def quantized_bytes(type_: int, rows: int, cols: int):
    out = ctypes.c_size_t(123)
    ok = lib().q3xo_quantized_bytes(type_, rows, cols, ctypes.byref(out))
    return out.value if ok else None


def embed(w: np.ndarray, type_: int, cols: int, row: int) -> np.ndarray:
    out = np.empty(cols, np.float32)
    assert lib().q3xo_embed(_p(w), type_, cols, row, _p(out))
    return out


def dequant(w: np.ndarray, type_: int, rows: int, cols: int) -> np.ndarray:
    out = np.empty((rows, cols), np.float32)
    for r in range(rows):
        assert lib().q3xo_embed(_p(w), type_, cols, r, _p(out[r]))
    return out


def mv(w: np.ndarray, type_: int, rows: int, cols: int, x: np.ndarray, threads: int | None = None) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(rows, np.float32)
    assert lib().q3xo_mv(_p(w), type_, rows, cols, _p(x), _p(y), threads or default_threads())
    return y


def mv_serial(w: np.ndarray, type_: int, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(rows, np.float32)
    assert lib().q3xo_mv_rows(_p(w), type_, 0, rows, cols, _p(x), _p(y))
    return y


def gemm(w: np.ndarray, type_: int, rows: int, cols: int, X: np.ndarray, threads: int | None = None) -> np.ndarray:
    X = np.ascontiguousarray(X, np.float32)
    count = X.shape[0]
    Y = np.empty((count, rows), np.float32)
    assert lib().q3xo_gemm(_p(w), type_, rows, cols, _p(X), count, _p(Y), threads or default_threads())
    return Y


def sigmoid(x: float) -> float:
    return float(lib().q3xo_sigmoid(x))


def silu(x: float) -> float:
    return float(lib().q3xo_silu(x))


def router_top_k(logits: np.ndarray, top_k: int):
    """Per token (rows of ``logits``): ids [T, k], weights [T, k], probabilities [T, E]."""
    logits = np.ascontiguousarray(np.atleast_2d(logits), np.float32)
    T, E = logits.shape
    ids = np.empty((T, top_k), np.int32)
    weights = np.empty((T, top_k), np.float32)
    probs = np.empty((T, E), np.float32)
    for t in range(T):
        assert lib().q3xo_router_top_k(_p(logits[t]), E, top_k, _p(ids[t]), _p(weights[t]), _p(probs[t]))
    return ids, weights, probs


def moe_routed(gate_up: np.ndarray, down: np.ndarray, type_: int, experts: int, H: int, I: int,
               X: np.ndarray, ids: np.ndarray, weights: np.ndarray, threads: int | None = None) -> np.ndarray:
    X = np.ascontiguousarray(np.atleast_2d(X), np.float32)
    ids = np.ascontiguousarray(np.atleast_2d(ids), np.int32)
    weights = np.ascontiguousarray(np.atleast_2d(weights), np.float32)
    T = X.shape[0]
    top_k = ids.shape[1]
    Y = np.empty((T, H), np.float32)
    assert lib().q3xo_moe_routed(_p(gate_up), _p(down), type_, experts, H, I, _p(X), T, _p(ids), _p(weights),
                                 top_k, _p(Y), threads or default_threads())
    return Y


def mv_bf16(weights: np.ndarray, x: np.ndarray, bf16_lanes: int = 1) -> np.ndarray:
    """y = W x for a BF16 matrix given as uint16 [rows, cols] (engine.cpp:200-212;
    bf16_lanes 16: the AVX-512 dot of arch/x86/kernels.h:21-37)."""
    weights = np.ascontiguousarray(weights, np.uint16)
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = weights.shape
    y = np.empty(rows, np.float32)
    set_bf16_lanes(bf16_lanes)
    try:
        assert lib().q3xo_mv_bf16(_p(weights), rows, cols, _p(x), _p(y))
    finally:
        set_bf16_lanes(1)
    return y


def moe_layer(router: np.ndarray, gate_up: np.ndarray, down: np.ndarray, shared_gate: np.ndarray,
              shared_up: np.ndarray, shared_down: np.ndarray, shared_scale: np.ndarray, type_: int,
              experts: int, H: int, I: int, shared_I: int, top_k: int, X: np.ndarray,
              threads: int | None = None, bf16_lanes: int = 1):
    """The whole MoE layer (engine.cpp:406-430) for every row of X, its BF16
    router and gate dots as the portable loop (bf16_lanes 1) or the AVX-512
    kernel (16) computes them.  Returns (Y [T, H], ids [T, top_k], weights
    [T, top_k])."""
    X = np.ascontiguousarray(np.atleast_2d(X), np.float32)
    T = X.shape[0]
    Y = np.empty((T, H), np.float32)
    ids = np.empty((T, top_k), np.int32)
    weights = np.empty((T, top_k), np.float32)
    router = np.ascontiguousarray(router, np.uint16)
    shared_scale = np.ascontiguousarray(shared_scale, np.uint16)
    set_bf16_lanes(bf16_lanes)
    try:
        assert lib().q3xo_moe_layer(_p(router), _p(gate_up), _p(down), _p(shared_gate), _p(shared_up),
                                    _p(shared_down), _p(shared_scale), type_, experts, H, I, shared_I, top_k,
                                    _p(X), T, _p(Y), _p(ids), _p(weights), threads or default_threads())
    finally:
        set_bf16_lanes(1)
    return Y, ids, weights


def quantize(type_: int, values: np.ndarray) -> np.ndarray:
    values = np.ascontiguousarray(values, np.float32).reshape(-1)
    out = np.empty(values.size // 32 * BLOCK_BYTES[type_], np.uint8)
    ok = lib().q3xo_quantize(type_, _p(values), values.size, _p(out))
    if not ok:
        raise ValueError("quantize: partial block or non-finite input")
    return out


def ref_model_load(path: str, capacity: int = 4096):
    """The reference's own loader (engine.cpp:481-559) on `path`, through the
    reference build.  Returns (None, offsets [n], shapes [n, 4] = rows, cols,
    experts, type with -1 for bare vectors) or (message, None, None)."""
    offsets = np.zeros(capacity, np.uint64)
    shapes = np.zeros((capacity, 4), np.int32)
    count = ctypes.c_size_t(0)
    error = ctypes.c_char_p()
    ok = ref().q3xr_model_load(path.encode(), _p(offsets), _p(shapes), capacity, ctypes.byref(count),
                               ctypes.byref(error))
    if not ok:
        return error.value.decode(), None, None
    assert count.value <= capacity
    return None, offsets[:count.value].copy(), shapes[:count.value].copy()


def ref_forward(config: dict, image: np.ndarray, table, tokens) -> np.ndarray:
    """The reference's CPU forward (engine.cpp:431-454) token by token on
    weights `image` (uint8, model.bin layout) whose tensors `table` lists as
    (role, layer, offset); returns logits [len(tokens), V]."""
    keys = ("id", "V", "H", "I", "N", "AI", "AH", "KVH", "AD", "RD", "KH", "VH", "KD", "VD", "CK", "experts",
            "top_k", "shared_I", "matrix_type", "tied_embeddings")
    cfg = np.array([int(config[k]) for k in keys], np.int32)
    roles = np.array([t[0] for t in table], np.int32)
    layers = np.array([t[1] for t in table], np.int32)
    offsets = np.array([t[2] for t in table], np.uint64)
    tokens = np.ascontiguousarray(tokens, np.int32)
    out = np.empty((tokens.size, int(config["V"])), np.float32)
    image = np.ascontiguousarray(image, np.uint8)
    assert ref().q3xr_forward(_p(cfg), _p(image), _p(roles), _p(layers), _p(offsets), len(table), _p(tokens),
                              tokens.size, _p(out))
    return out
