"""GPU tests of the model.bin device loader (q3x_hip_model_load).

Files are sparse and full-size, as in the reference's loader tests
(tests/q8_cpu_test.cpp:222-264, tests/q4_cpu_test.cpp:85-136), with real
bytes written where a test reads them:
  - every tensor of a Qwen3.5-0.8B file carries markers at both ends, read
    back through the device addresses the loader hands out;
  - one FFN of a Qwen3.5-9B (Q8_0) file and one MoE layer of a
    Qwen3.6-35B-A3B (Q4_0) file hold random blocks, and the matvec, GEMM and
    MoE-layer entry points run on the loaded weights against the oracle.
The layout itself (offsets, shapes, messages) is pinned on the CPU in
tests/test_model_file.py."""
import ctypes
import time

import numpy as np
import pytest

import oracle
from oracle import model_file as mf
import qwen3x_amd as q3x
from tests.helpers import BLOCK_BYTES, Q4_0, Q8_0, dequant_numpy, row_bound
from tests.test_gpu_moe_layer import bf16, check_layer, run_layer
from tests.test_gpu_parity import _torch, dev, host, say

pytestmark = pytest.mark.gpu


def _hip():
    _torch().cuda.init()
    hip = ctypes.CDLL("libamdhip64.so.7")  # the runtime torch and the library share
    hip.hipMemcpy.restype = ctypes.c_int
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    return hip


def _read_device(hip, address, n):
    out = np.empty(n, np.uint8)
    assert hip.hipMemcpy(out.ctypes.data, address, n, 2) == 0  # hipMemcpyDeviceToHost
    return out.tobytes()


def _sparse_file(path, model_id):
    size = mf.layout(model_id)[1]
    with open(path, "wb") as f:
        f.truncate(size)
        f.write(mf.header(model_id))
    return size


def _load(path, size):
    t0 = time.perf_counter()
    model = q3x.Model(path)
    dt = time.perf_counter() - t0
    say(f"loaded {size / 1e9:.2f} GB in {dt:.2f} s ({size / dt / 1e9:.1f} GB/s, sparse file)")
    assert model.nbytes == size
    return model


def _random_pool(rng, type_, rows, cols):
    """Random blocks as flat bytes without the int64 temporaries of random_blocks."""
    nb = rows * cols // 32
    out = rng.integers(0, 256, (nb, BLOCK_BYTES[type_]), dtype=np.uint8)
    out[:, 0:2] = rng.normal(0.0, 0.02, nb).astype(np.float16).view(np.uint8).reshape(nb, 2)
    return out.reshape(-1)


def _offsets(model_id):
    return {(role, layer): (offset, nbytes) for role, layer, _, offset, nbytes in mf.layout(model_id)[0]}


def test_loader_binds_every_tensor_of_a_tied_model(tmp_path):
    # Qwen3.5-0.8B: BF16, tied embeddings, 320 tensors over 1.5 GB.
    hip = _hip()
    path = str(tmp_path / "model.bin")
    size = _sparse_file(path, 800)
    rows = mf.layout(800)[0]
    with open(path, "r+b") as f:
        for i, (role, layer, _, offset, nbytes) in enumerate(rows):
            f.seek(offset)
            f.write(np.array([i, 0x5A000000 | q3x.TENSOR_ROLES.index(role)], np.uint32).tobytes())
            f.seek(offset + nbytes - 8)
            f.write(np.array([~i & 0xFFFFFFFF, layer & 0xFFFFFFFF], np.uint32).tobytes())
    say("loader markers: Qwen3.5-0.8B")
    with _load(path, size) as model:
        assert model.config.id == 800 and model.config.tied_embeddings
        assert [(q3x.TENSOR_ROLES[t.role], t.layer, t.offset) for t in model.tensors] == \
            [(r, l, o) for r, l, _, o, _ in rows]
        for i, (role, layer, _, offset, nbytes) in enumerate(rows):
            t, region = model.tensor(role, layer)
            assert region.data_ptr() == model.base + offset and region.data_ptr() % 64 == 0
            head = np.frombuffer(_read_device(hip, region.data_ptr(), 8), np.uint32)
            tail = np.frombuffer(_read_device(hip, region.data_ptr() + nbytes - 8, 8), np.uint32)
            assert head.tolist() == [i, 0x5A000000 | q3x.TENSOR_ROLES.index(role)], (role, layer)
            assert tail.tolist() == [~i & 0xFFFFFFFF, layer & 0xFFFFFFFF], (role, layer)
        # Tied: lm_head is the embedding (engine.cpp:500); the header is on the device too.
        assert model.tensor("lm_head")[1].data_ptr() == model.tensor("embedding")[1].data_ptr()
        assert _read_device(hip, model.base, 72) == mf.header(800)
        with pytest.raises(q3x.Q3xHipError):
            model.tensor("moe_router", 0)
        with pytest.raises(q3x.Q3xHipError):
            model.moe_layer(0)


def test_matvec_and_gemm_on_a_loaded_q8_model(tmp_path):
    # Qwen3.5-9B (Q8_0, 9.5 GB): layer 5's FFN gate [12288, 4096] and down
    # [4096, 12288] hold random blocks; the rest of the file is zero.
    torch = _torch()
    rng = np.random.default_rng(9000)
    path = str(tmp_path / "model.bin")
    size = _sparse_file(path, 9000)
    where = _offsets(9000)
    gate = _random_pool(rng, Q8_0, 12288, 4096)
    down = _random_pool(rng, Q8_0, 4096, 12288)
    with open(path, "r+b") as f:
        for key, data in ((("ffn_gate", 5), gate), (("ffn_down", 5), down)):
            offset, nbytes = where[key]
            assert nbytes == data.size
            f.seek(offset)
            f.write(data.tobytes())
    say("loader: Qwen3.5-9B matvec / GEMM")
    with _load(path, size) as model:
        for role, w, rows, cols in (("ffn_gate", gate, 12288, 4096), ("ffn_down", down, 4096, 12288)):
            lin = model.linear(role, 5)
            assert (lin.rows, lin.columns, lin.type) == (rows, cols, Q8_0)
            x = rng.normal(0, 1, cols).astype(np.float32)
            y = torch.empty(rows, dtype=torch.float32, device="cuda:0")
            q3x.mv(lin, dev(x), y)
            want = oracle.mv(w, Q8_0, rows, cols, x)
            wd = dequant_numpy(w, Q8_0, rows, cols)
            assert np.all(np.abs(host(y) - want) <= row_bound(wd, x)), role
            X = rng.normal(0, 1, (7, cols)).astype(np.float32)
            Y = torch.empty((7, rows), dtype=torch.float32, device="cuda:0")
            q3x.batch_mv(lin, dev(X), Y, 7)
            want = oracle.gemm(w, Q8_0, rows, cols, X)
            assert np.all(np.abs(host(Y) - want) <= row_bound(wd, X)), role
        # An untouched (all-zero) matrix of the same file gives exact zeros.
        lin = model.linear("lm_head")
        y = torch.full((lin.rows,), 7.0, dtype=torch.float32, device="cuda:0")
        q3x.mv(lin, dev(rng.normal(0, 1, 4096).astype(np.float32)), y)
        assert not host(y).any()


@pytest.fixture(scope="module")
def q4_model(tmp_path_factory):
    """Qwen3.6-35B-A3B (Q4_0, 19.5 GB) loaded once: layer 7's MoE (256
    experts, top 8, shared expert) holds random weights."""
    rng = np.random.default_rng(36035)
    E, H, I, SI = 256, 2048, 512, 512
    w = dict(router=bf16(rng, E, H, 0.5), gate_up=_random_pool(rng, Q4_0, E * 2 * I, H),
             down=_random_pool(rng, Q4_0, E * H, I), shared_gate=_random_pool(rng, Q4_0, SI, H),
             shared_up=_random_pool(rng, Q4_0, SI, H), shared_down=_random_pool(rng, Q4_0, H, SI),
             shared_scale=bf16(rng, 1, H, 0.05))
    path = str(tmp_path_factory.mktemp("q4") / "model.bin")
    size = _sparse_file(path, 36035)
    where = _offsets(36035)
    with open(path, "r+b") as f:
        for name, data in w.items():
            offset, nbytes = where[("moe_" + name, 7)]
            assert nbytes == data.nbytes, name
            f.seek(offset)
            f.write(data.tobytes())
    say("loader: Qwen3.6-35B-A3B")
    model = _load(path, size)
    yield model, w
    model.close()


@pytest.mark.parametrize("tokens", [1, 5])
def test_moe_layer_on_a_loaded_q4_model(tokens, q4_model):
    torch = _torch()
    model, w = q4_model
    E, H, I, SI, k = 256, 2048, 512, 512, 8
    rng = np.random.default_rng(tokens)
    X = rng.normal(0, 1, (tokens, H)).astype(np.float32)
    say(f"loaded MoE layer tokens={tokens}")
    layer = model.moe_layer(7)
    assert (layer.type, layer.experts, layer.top_k, layer.H, layer.I, layer.shared_I) == (Q4_0, E, k, H, I, SI)
    got, ids_g, wts_g, logits_g = run_layer(layer, X, tokens, k)
    want, ids_o, wts_o = oracle.moe_layer(w["router"], w["gate_up"], w["down"], w["shared_gate"], w["shared_up"],
                                          w["shared_down"], w["shared_scale"], Q4_0, E, H, I, SI, k, X)
    check_layer(w, Q4_0, E, H, I, SI, k, X, got, ids_g, wts_g, want, ids_o, wts_o, logits_g)


def test_loaded_q4_layers_bind_through_the_table(q4_model):
    # Every MoE layer binds; the pools sit where the packer's schema puts them.
    model, _ = q4_model
    where = _offsets(36035)
    for layer in range(40):
        m = model.moe_layer(layer)
        assert m.gate_up.data_ptr() == model.base + where[("moe_gate_up", layer)][0]
        assert m.shared_scale.data_ptr() == model.base + where[("moe_shared_scale", layer)][0]
    with pytest.raises(q3x.Q3xHipError):
        model.moe_layer(40)
    pool = model.expert_linear("moe_down", 39)
    assert (pool.experts, pool.rows, pool.columns, pool.type) == (256, 2048, 512, Q4_0)


def test_quantize_bf16_matches_the_fp32_entry_point():
    # BF16 rows (the packer's input) quantize exactly as their FP32 widening.
    torch = _torch()
    rng = np.random.default_rng(16)
    vals = rng.normal(0, 0.02, (300, 2048)).astype(np.float32)
    vals[0, :32] = 0
    vals[1, :32] = np.linspace(-8, 7.5, 32)
    vals[2, :32] *= 1e4
    bits = (vals.view(np.uint32) >> 16).astype(np.uint16)
    widened = (bits.astype(np.uint32) << 16).view(np.float32)
    for type_ in (Q8_0, Q4_0):
        want = oracle.quantize(type_, widened)
        out = torch.empty(want.size, dtype=torch.uint8, device="cuda:0")
        say(f"quantize_bf16 type={type_}")
        q3x.quantize_bf16(type_, dev(bits.view(np.int16)), 300, 2048, out)
        assert np.array_equal(host(out), want)


def test_quantize_bf16_matches_llama_cpp_sha256():
    # tests/q4_llama_reference.py:24-30 and its published digest
    # (eval/qwen36-35b-q4.md:53-57), on the device from the BF16 bits.
    import hashlib
    torch = _torch()
    rng = np.random.default_rng(20260907)
    values = rng.normal(size=4096 * 32).astype("<f4")
    values[:32] = 0
    values[32:64] = np.linspace(-8, 7.5, 32, dtype="<f4")
    values[64:96] = np.linspace(8, -7.5, 32, dtype="<f4")
    bits = (values.view(np.uint32) >> 16).astype(np.uint16)
    out = torch.empty(4096 * 18, dtype=torch.uint8, device="cuda:0")
    q3x.quantize_bf16(Q4_0, dev(bits.view(np.int16)), 4096, 32, out)
    digest = hashlib.sha256(host(out).tobytes()).hexdigest()
    assert digest == "735e40577b24f36e3ff4cc1a12bd085e7648b1b0099d0ae0b0700b371a64532c"
