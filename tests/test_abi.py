"""CPU tests of the C ABI: the library loads, exports every entry point
include/q3x_hip.h declares, and rejects invalid arguments before touching the
device (so these calls need no GPU)."""
import ctypes
import os
import re
import subprocess

import pytest

import oracle
import qwen3x_amd as q3x

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "q3x_hip.h")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w[\w\s\*]*?\b(q3x_hip_\w+)\s*\(", text, re.M)))


def test_header_declares_the_entry_points():
    names = declared_functions()
    assert names == sorted(q3x.SIGNATURES), names


def test_library_exports_every_declared_symbol():
    lib = q3x.lib()
    out = subprocess.run(["nm", "-D", "--defined-only", q3x.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT (q3x_hip_\w+)", out))
    for name in declared_functions():
        assert name in exported, name
        assert getattr(lib, name) is not None


def test_strerror():
    assert q3x.strerror(q3x.OK) == "ok"
    assert "invalid" in q3x.strerror(q3x.EINVAL)
    assert q3x.strerror(q3x.ENOTSUP)
    assert q3x.strerror(12345) == "unknown error"
    assert "reset" in q3x.strerror(q3x.ESTATE)
    assert "scratch" in q3x.strerror(q3x.ESCRATCH)


def test_quantized_bytes_match_the_oracle_rules():
    cases = [(0, 3, 17), (1, 3, 64), (2, 3, 64), (1, 0, 32), (2, 1, -32), (1, 1, 33), (2, 1, 16), (999, 1, 32),
             (1, 151936, 4096), (2, 17408, 5120), (1, 2147483647, 2147483616)]
    for t, r, c in cases:
        assert q3x.quantized_bytes(t, r, c) == oracle.quantized_bytes(t, r, c), (t, r, c)
    out = ctypes.c_size_t(123)
    assert q3x.lib().q3x_hip_quantized_bytes(1, 3, 64, None) == q3x.EINVAL
    assert q3x.lib().q3x_hip_quantized_bytes(1, 1, 33, ctypes.byref(out)) == q3x.EINVAL
    assert out.value == 123  # untouched on rejection


def test_invalid_arguments_are_rejected_without_device_work():
    lib = q3x.lib()
    P = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first
    N = None
    assert lib.q3x_hip_mv(N, 1, 4, 64, P, P, 0, N) == q3x.EINVAL
    assert lib.q3x_hip_mv(P, 1, 4, 64, N, P, 0, N) == q3x.EINVAL
    assert lib.q3x_hip_mv(P, 1, 4, 64, P, N, 0, N) == q3x.EINVAL
    assert lib.q3x_hip_mv(P, 1, 0, 64, P, P, 0, N) == q3x.EINVAL
    assert lib.q3x_hip_mv(P, 1, 4, 48, P, P, 0, N) == q3x.EINVAL
    assert lib.q3x_hip_mv(P, 7, 4, 64, P, P, 0, N) == q3x.EINVAL
    assert lib.q3x_hip_mv(P, 0, 4, 64, P, P, 0, N) == q3x.ENOTSUP   # BF16: caller's own path
    assert lib.q3x_hip_gemm(P, 1, 4, 64, P, 0, P, 0, N) == q3x.EINVAL
    assert lib.q3x_hip_gemm(P, 2, 4, 40, P, 3, P, 0, N) == q3x.EINVAL
    assert lib.q3x_hip_gemm(P, 0, 4, 64, P, 3, P, 0, N) == q3x.ENOTSUP
    gw = lib.q3x_hip_gemm_ws
    assert gw(P, 1, 4, 64, P, 0, P, 0, P, 1024, N) == q3x.EINVAL
    assert gw(P, 0, 4, 64, P, 3, P, 0, P, 1024, N) == q3x.ENOTSUP
    assert gw(P, 1, 4, 64, P, 3, P, 0, N, 1024, N) == q3x.EINVAL       # bytes but no workspace
    assert lib.q3x_hip_dequant(P, 1, 64, -1, 1, P, N) == q3x.EINVAL
    assert lib.q3x_hip_dequant(P, 2, 64, 0, 0, P, N) == q3x.EINVAL
    assert lib.q3x_hip_read_probe(N, 16, P, N) == q3x.EINVAL
    assert lib.q3x_hip_read_probe(P, 24, P, N) == q3x.EINVAL                   # not a multiple of 16
    assert lib.q3x_hip_read_probe(ctypes.c_void_p(0x1008), 32, P, N) == q3x.EINVAL  # not 16-byte aligned
    assert lib.q3x_hip_read_probe(P, 0, P, N) == q3x.EINVAL
    assert lib.q3x_hip_router_topk(P, 1, 256, 9, P, P, N) == q3x.EINVAL       # top_k > 8
    assert lib.q3x_hip_router_topk(P, 1, 4, 5, P, P, N) == q3x.EINVAL         # top_k > experts
    assert lib.q3x_hip_router_topk(P, 1, 2048, 8, P, P, N) == q3x.EINVAL      # experts > 1024
    assert lib.q3x_hip_router_topk(P, 0, 256, 8, P, P, N) == q3x.EINVAL
    ws = lib.q3x_hip_moe_workspace_bytes(2048, 256, 8, 2048, 512)
    assert lib.q3x_hip_moe_routed(P, P, 2, 256, 2048, 512, P, 2048, P, P, 8, P, 0, P, ws - 1, N) == q3x.EINVAL
    assert lib.q3x_hip_moe_routed(P, P, 2, 256, 2048, 500, P, 2048, P, P, 8, P, 0, P, ws, N) == q3x.EINVAL
    assert lib.q3x_hip_moe_routed(P, P, 2, 4, 2048, 512, P, 1, P, P, 5, P, 0, P, ws, N) == q3x.EINVAL
    assert lib.q3x_hip_moe_routed(P, P, 0, 4, 2048, 512, P, 1, P, P, 2, P, 0, P, ws, N) == q3x.ENOTSUP
    rl = lib.q3x_hip_moe_routed_logits
    ws1 = lib.q3x_hip_moe_workspace_bytes(1, 256, 8, 2048, 512)
    assert rl(P, P, 2, 256, 2048, 512, P, 1, P, 8, P, P, P, 0, P, ws1 - 1, N) == q3x.EINVAL  # short workspace
    assert rl(P, P, 2, 256, 2048, 512, P, 1, N, 8, P, P, P, 0, P, ws, N) == q3x.EINVAL      # no logits
    assert rl(P, P, 2, 256, 2048, 512, P, 1, P, 8, N, P, P, 0, P, ws, N) == q3x.EINVAL      # no ids output
    assert rl(P, P, 2, 256, 2048, 512, P, 1, P, 9, P, P, P, 0, P, ws, N) == q3x.EINVAL      # top_k > 8
    assert rl(P, P, 2, 2048, 2048, 512, P, 1, P, 8, P, P, P, 0, P, ws, N) == q3x.EINVAL     # experts > 1024
    assert rl(P, P, 0, 256, 2048, 512, P, 1, P, 8, P, P, P, 0, P, ws, N) == q3x.ENOTSUP
    item = q3x.MvItem(0x1000, 4, 0x1000, 0)
    items = (q3x.MvItem * 9)(*([item] * 9))
    ip = ctypes.cast(items, ctypes.c_void_p)
    assert lib.q3x_hip_mv_multi(ip, 0, 1, 64, P, N) == q3x.EINVAL
    assert lib.q3x_hip_mv_multi(ip, 9, 1, 64, P, N) == q3x.EINVAL          # more than 8 matrices
    assert lib.q3x_hip_mv_multi(N, 1, 1, 64, P, N) == q3x.EINVAL
    assert lib.q3x_hip_mv_multi(ip, 2, 1, 48, P, N) == q3x.EINVAL
    assert lib.q3x_hip_mv_multi(ip, 2, 1, 64, N, N) == q3x.EINVAL
    assert lib.q3x_hip_mv_multi(ip, 2, 0, 64, P, N) == q3x.ENOTSUP
    bad = (q3x.MvItem * 2)(item, q3x.MvItem(0x1000, 0, 0x1000, 0))
    assert lib.q3x_hip_mv_multi(ctypes.cast(bad, ctypes.c_void_p), 2, 2, 64, P, N) == q3x.EINVAL
    bad = (q3x.MvItem * 2)(item, q3x.MvItem(None, 4, 0x1000, 0))
    assert lib.q3x_hip_mv_multi(ctypes.cast(bad, ctypes.c_void_p), 2, 2, 64, P, N) == q3x.EINVAL
    assert ctypes.sizeof(q3x.MvItem) == 32  # struct q3x_hip_mv_item on LP64
    assert lib.q3x_hip_quantize(1, N, 4, 64, P, N) == q3x.EINVAL
    assert lib.q3x_hip_quantize(2, P, 4, 48, P, N) == q3x.EINVAL


def test_moe_layer_invalid_arguments_are_rejected_without_device_work():
    lib = q3x.lib()
    P = 0x1000  # never dereferenced: validation fails first
    N = None

    def layer(**kw):
        f = dict(router=P, gate_up=P, down=P, shared_gate=P, shared_up=P, shared_down=P, shared_scale=P, type=2,
                 experts=256, top_k=8, H=2048, I=512, shared_I=512)
        f.update(kw)
        return q3x.MoeLayerWeights(*(f[name] for name, _ in q3x.MoeLayerWeights._fields_))

    good = layer()
    ws = lib.q3x_hip_moe_layer_workspace_bytes(ctypes.byref(good), 16)
    assert ws > 0
    call = lambda lw, X=P, T=16, Y=P, w=ws: lib.q3x_hip_moe_layer(ctypes.byref(lw), X, T, Y, N, N, P, w, N)  # noqa
    assert call(good, w=ws - 1) == q3x.EINVAL                     # workspace too small
    assert call(good, X=N) == q3x.EINVAL
    assert call(good, Y=N) == q3x.EINVAL
    assert call(good, T=0) == q3x.EINVAL
    assert call(layer(shared_I=1024)) == q3x.EINVAL               # shared_I > I
    assert call(layer(shared_I=48)) == q3x.EINVAL                 # not a multiple of 32
    assert call(layer(top_k=9)) == q3x.EINVAL
    assert call(layer(router=None)) == q3x.EINVAL
    assert call(layer(shared_scale=None)) == q3x.EINVAL
    assert call(layer(router=P + 2)) == q3x.EINVAL                # BF16 router must be 16-byte aligned
    assert call(layer(type=0)) == q3x.ENOTSUP                     # BF16 experts: caller's own path
    assert lib.q3x_hip_moe_layer(N, P, 16, P, N, N, P, ws, N) == q3x.EINVAL
    assert lib.q3x_hip_moe_layer_workspace_bytes(N, 16) == 0
    assert lib.q3x_hip_moe_layer_workspace_bytes(ctypes.byref(good), 0) == 0


def test_moe_layer_workspace_covers_the_routed_workspace():
    lw = q3x.MoeLayerWeights(1, 1, 1, 1, 1, 1, 1, 2, 256, 8, 2048, 512, 512)
    for T in (1, 2048):
        layer_ws = q3x.lib().q3x_hip_moe_layer_workspace_bytes(ctypes.byref(lw), T)
        assert layer_ws >= q3x.moe_workspace_bytes(T, 256, 8, 2048, 512) + 4 * T * (256 + 1 + 2 * 8 + 3 * 512)


def test_moe_workspace_sizes():
    decode = q3x.moe_workspace_bytes(1, 256, 8, 2048, 512)
    assert decode >= 4 * 8 * (2 * 512 + 512 + 2048)
    prefill = q3x.moe_workspace_bytes(2048, 256, 8, 2048, 512)
    pairs = 2048 * 8
    assert prefill >= 4 * pairs * (2 * 512 + 512 + 2048) + 4 * 2 * pairs
    assert q3x.moe_workspace_bytes(0, 256, 8, 2048, 512) == 0


def test_cpp_host_interface_binary_skips_without_gpu():
    exe = os.path.join(ROOT, "qwen3x_amd", "q3x_hip_host_test")
    assert os.path.exists(exe), "build it with make -C qwen3x_amd"
    import torch
    if torch.cuda.is_available():
        pytest.skip("GPU present: the binary runs in the GPU suite")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert r.returncode == 77, r.stdout + r.stderr


def test_gemm_workspace_sizes():
    # Splits only where few output tiles meet a long K; a pure function of
    # the shape (the plan a call makes with that many bytes).
    lib = q3x.lib()
    Q8, Q4 = q3x.MATRIX_Q8_0, q3x.MATRIX_Q4_0
    assert lib.q3x_hip_gemm_workspace_bytes(Q8, 12288, 4096, 4096) == 0      # 1536 tiles: no split
    down = lib.q3x_hip_gemm_workspace_bytes(Q4, 5120, 17408, 512)            # 80 tiles, 544 K blocks
    assert down > 0 and down % (128 * 256 * 4 * 80) == 0
    assert down == lib.q3x_hip_gemm_workspace_bytes(Q4, 5120, 17408, 512)
    assert lib.q3x_hip_gemm_workspace_bytes(Q8, 256, 8192, 64) > 0          # one tile, 256 K blocks
    assert lib.q3x_hip_gemm_workspace_bytes(Q8, 4, 64, 3) == 0
    assert lib.q3x_hip_gemm_workspace_bytes(Q8, 4, 40, 3) == 0              # invalid shape
    assert lib.q3x_hip_gemm_workspace_bytes(0, 4096, 4096, 512) == 0        # BF16
