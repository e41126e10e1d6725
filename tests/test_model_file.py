"""model.bin header check and tensor layout (CPU only).

The library's layout (q3x_hip_model_layout, the loader's validation) is held
to two independent sources:
  - the packer's schema (scripts/pack_weights.py:171-283, restated in
    oracle/model_file.py), itself pinned by the reference's known file sizes
    (tests/q8_cpu_test.cpp:228, tests/q4_cpu_test.cpp:15);
  - the reference's own loader (engine.cpp:481-559, built from the reference
    sources into oracle/_ref) run on sparse full-size files, as the
    reference's loader tests do (q8_cpu_test.cpp:222-264,
    q4_cpu_test.cpp:85-136): offsets, shapes and rejection messages.
The device loader validates before any device work, so its rejections are
tested here too; the upload itself is a GPU test."""
import ctypes
import os
import struct

import pytest

import oracle
from oracle import model_file as mf
import qwen3x_amd as q3x

IDS = sorted(mf.MODELS)


def test_packer_schema_reproduces_the_reference_file_sizes():
    assert mf.layout(9000)[1] == 9514418816       # q8_cpu_test.cpp:228
    assert mf.layout(36035)[1] == 19528534784     # q4_cpu_test.cpp:15


@pytest.mark.parametrize("model_id", IDS)
def test_layout_matches_the_packer_schema(model_id):
    rows, size = mf.layout(model_id)
    config, tensors = q3x.model_layout(mf.header(model_id), size)
    assert config.id == model_id and config.name.decode() == mf.MODELS[model_id]["name"]
    assert [struct.unpack("<I", struct.pack("<i", getattr(config, f)))[0] for f in
            ("V", "H", "I", "N", "AI", "AH", "KVH", "AD", "RD", "KH", "VH", "KD", "VD", "CK")] == \
        list(mf.header_fields(model_id)[1:15])
    m = mf.MODELS[model_id]
    assert (config.experts, config.top_k, config.shared_I) == (m["experts"], m["top_k"], m["shared"])
    assert config.matrix_type == mf.MATRIX_TYPE[m["matrix"]] and bool(config.tied_embeddings) == m["tied"]
    assert len(tensors) == len(rows)
    for t, (role, layer, stored, offset, nbytes), (_, _, _, shape, matrix) in zip(tensors, rows,
                                                                                   mf.tensors(model_id)):
        assert (q3x.TENSOR_ROLES[t.role], t.layer, t.type, t.offset, t.bytes) == (role, layer, stored, offset,
                                                                                nbytes)
        assert t.offset % 64 == 0
        if len(shape) == 3 and matrix:          # expert pool [E, rows, cols]
            assert (t.experts, t.rows, t.cols) == shape
        elif len(shape) == 3:                   # conv1d [DQKV, 1, CK]
            assert (t.experts, t.rows, t.cols) == (0, shape[0], shape[2])
        elif len(shape) == 2:
            assert (t.experts, t.rows, t.cols) == (0,) + shape
        else:
            assert (t.experts, t.rows, t.cols) == (0, 1, shape[0])
    last = tensors[-1]
    assert last.offset + last.bytes == size


def _sparse(path, model_id, size=None):
    size = mf.layout(model_id)[1] if size is None else size
    with open(path, "wb") as f:
        f.truncate(size)
        f.write(mf.header(model_id))
    return size


def _need_ref():
    if oracle.ref() is None:
        pytest.skip("reference build (oracle/_ref) absent: the reference tree is not here")


@pytest.mark.parametrize("model_id", IDS)
def test_layout_matches_the_reference_loader_on_sparse_files(model_id, tmp_path):
    _need_ref()
    path = str(tmp_path / "model.bin")
    size = _sparse(path, model_id)
    error, offsets, shapes = oracle.ref_model_load(path)
    assert error is None, error
    _, tensors = q3x.model_layout(mf.header(model_id), size)
    assert [t.offset for t in tensors] == [int(o) for o in offsets]
    for t, (rows, cols, experts, type_) in zip(tensors, shapes):
        if rows >= 0:   # a Linear / ExpertLinear of the reference
            assert (t.rows, t.cols, t.experts, t.type) == (rows, cols, experts, type_)


def _header_with(model_id, offset, value):
    h = bytearray(mf.header(model_id))
    h[offset:offset + 4] = struct.pack("<I", value)
    return bytes(h)


# Rejections of the reference's loader tests, plus every header field.
REJECTIONS = [
    (9000, "size", -1, "truncated"),                            # q8_cpu_test.cpp:236-238
    (9000, "size", +1, "size does not match schema"),           # :239-241
    (9000, "byte", (0, ord("X")), "wrong model.bin magic"),     # :243-246
    (9000, "field", (8, 9001), "unsupported Qwen model ID"),    # :248-253
    (9000, "field", (8 + 2 * 4, 4095), "header mismatch"),      # :255-260
    (36035, "field", (0, 0), "magic"),                          # q4_cpu_test.cpp:115
    (36035, "field", (8, 12345), "model ID"),                   # :116
    (36035, "field", (12, 1), "header mismatch"),               # :117-118
    (36035, "size", -1, "truncated"),                           # :119-125
    (36035, "size", +1, "size does not match schema"),          # :126-132
    (9000, "field", (8, 4000), "header mismatch"),              # another model's ID over this one's fields
    (800, "size", -64, "truncated"),
    (38027, "size", +4096, "size does not match schema"),
] + [(36035, "field", (8 + 4 * f, 7), "header mismatch") for f in range(1, 16)]


def _mutated(model_id, kind, arg):
    size = mf.layout(model_id)[1]
    header = mf.header(model_id)
    if kind == "size":
        size += arg
    elif kind == "byte":
        header = header[:arg[0]] + bytes([arg[1]]) + header[arg[0] + 1:]
    else:
        header = _header_with(model_id, *arg)
    return header, size


@pytest.mark.parametrize("model_id,kind,arg,expected", REJECTIONS)
def test_rejections_match_the_reference_loader(model_id, kind, arg, expected, tmp_path):
    header, size = _mutated(model_id, kind, arg)
    with pytest.raises(q3x.ModelError) as info:
        q3x.model_layout(header, size)
    assert info.value.code == q3x.EMODEL and expected in info.value.message
    if oracle.ref() is not None:
        path = str(tmp_path / "model.bin")
        with open(path, "wb") as f:
            f.truncate(size)
            f.write(header)
        error, _, _ = oracle.ref_model_load(path)
        assert error == info.value.message


def test_device_loader_rejects_before_device_work(tmp_path):
    # Every rejection returns before the library touches the HIP runtime, so
    # these run without a GPU.
    with pytest.raises(q3x.ModelError, match="cannot open model.bin"):
        q3x.Model(str(tmp_path / "absent.bin"))
    short = tmp_path / "short.bin"
    short.write_bytes(mf.header(9000)[:71])
    with pytest.raises(q3x.ModelError, match="bad model.bin"):
        q3x.Model(str(short))
    for model_id, kind, arg, expected in REJECTIONS[:5]:
        header, size = _mutated(model_id, kind, arg)
        path = tmp_path / f"bad-{kind}.bin"
        with open(path, "wb") as f:
            f.truncate(size)
            f.write(header)
        with pytest.raises(q3x.ModelError) as info:
            q3x.Model(str(path))
        assert expected in info.value.message and info.value.code == q3x.EMODEL


def test_layout_arguments():
    lib = q3x.lib()
    count = ctypes.c_size_t(0)
    error = ctypes.c_char_p()
    header = mf.header(36035)
    size = mf.layout(36035)[1]
    assert lib.q3x_hip_model_layout(None, 72, size, None, None, 0, ctypes.byref(count), None) == q3x.EINVAL
    assert lib.q3x_hip_model_layout(header, 72, size, None, None, 0, None, None) == q3x.EINVAL
    assert lib.q3x_hip_model_layout(header, 71, size, None, None, 0, ctypes.byref(count), None) == q3x.EINVAL
    # Shorter than a header: the reference's "bad model.bin" whatever the bytes.
    assert lib.q3x_hip_model_layout(header, 8, 71, None, None, 0, ctypes.byref(count),
                                    ctypes.byref(error)) == q3x.EMODEL
    assert error.value == b"bad model.bin"
    assert lib.q3x_hip_model_layout(header, 72, size, None, None, 0, ctypes.byref(count), None) == q3x.OK
    assert count.value == len(mf.layout(36035)[0])
    small = (q3x.Tensor * 10)()
    assert lib.q3x_hip_model_layout(header, 72, size, None, small, 10, ctypes.byref(count), None) == q3x.EINVAL
    assert count.value == len(mf.layout(36035)[0])
    # Model handles: NULL is rejected, never dereferenced.
    assert lib.q3x_hip_model_info(None, None, None, None, None, None) == q3x.EINVAL
    assert lib.q3x_hip_model_tensor(None, 0, -1, None, None) == q3x.EINVAL
    assert lib.q3x_hip_model_moe_layer(None, 0, None) == q3x.EINVAL
    lib.q3x_hip_model_free(None)
    handle = ctypes.c_void_p(123)
    assert lib.q3x_hip_model_load(None, ctypes.byref(handle), None) == q3x.EINVAL


def test_quantize_bf16_arguments_are_rejected_without_device_work():
    lib = q3x.lib()
    P = ctypes.c_void_p(0x1000)
    assert lib.q3x_hip_quantize_bf16(0, P, 1, 32, P, None) == q3x.ENOTSUP
    assert lib.q3x_hip_quantize_bf16(1, None, 1, 32, P, None) == q3x.EINVAL
    assert lib.q3x_hip_quantize_bf16(2, ctypes.c_void_p(0x1002), 1, 32, P, None) == q3x.EINVAL
    assert lib.q3x_hip_quantize_bf16(1, P, 1, 48, P, None) == q3x.EINVAL
    assert lib.q3x_hip_quantize_bf16(7, P, 1, 32, P, None) == q3x.EINVAL


def test_schema_for_any_configuration_and_its_rejections():
    from tests.engine_models import CONFIGS
    for model_id in IDS:   # the fixed configurations give the file layout
        m = mf.MODELS[model_id]
        cfg = q3x.make_config(id=model_id, V=m["vocab"], H=m["hidden"], I=m["intermediate"], N=m["layers"],
                              AI=m["interval"], AH=m["heads"], KVH=m["kv_heads"], AD=m["head_dim"],
                              RD=m["rotary_dim"], KH=m["key_heads"], VH=m["value_heads"], KD=m["key_dim"],
                              VD=m["value_dim"], CK=m["conv"], experts=m["experts"], top_k=m["top_k"],
                              shared_I=m["shared"], matrix_type=mf.MATRIX_TYPE[m["matrix"]],
                              tied_embeddings=int(m["tied"]))
        table, nbytes = q3x.model_schema(cfg)
        rows, size = mf.layout(model_id)
        assert nbytes == size
        assert [(q3x.TENSOR_ROLES[t.role], t.layer, t.offset, t.bytes) for t in table] == \
            [(r, l, o, b) for r, l, _, o, b in rows]
    base = dict(CONFIGS["moe_q4"])
    lib = q3x.lib()
    count = ctypes.c_size_t(0)
    for bad in (dict(H=0), dict(H=250), dict(AH=3, KVH=2), dict(VH=3, KH=2), dict(top_k=9), dict(shared_I=0), dict(I=40),
                dict(matrix_type=5)):
        cfg = q3x.make_config(**dict(base, **bad))
        assert lib.q3x_hip_model_schema(ctypes.byref(cfg), None, 0, ctypes.byref(count), None) == q3x.EINVAL, bad


def test_engine_rejects_before_device_work():
    from tests.engine_models import CONFIGS
    lib = q3x.lib()
    handle = ctypes.c_void_p()
    error = ctypes.c_char_p()
    P = ctypes.c_void_p(0x1000)   # never dereferenced: validation fails first
    bf16 = q3x.make_config(**dict(CONFIGS["dense_q8"], matrix_type=0))
    assert lib.q3x_hip_engine_create(ctypes.byref(bf16), P, 8, 0, ctypes.byref(handle), ctypes.byref(error)) == \
        q3x.ENOTSUP
    assert b"BF16" in error.value
    for bad in (dict(KD=256), dict(VD=160), dict(RD=128), dict(CK=1), dict(H=250), dict(AD=80, RD=16)):
        cfg = q3x.make_config(**dict(CONFIGS["dense_q8"], **bad))
        assert lib.q3x_hip_engine_create(ctypes.byref(cfg), P, 8, 0, ctypes.byref(handle), ctypes.byref(error)) == \
            q3x.EINVAL, bad
    good = q3x.make_config(**CONFIGS["dense_q8"])
    for context in (0, 262145):
        assert lib.q3x_hip_engine_create(ctypes.byref(good), P, context, 0, ctypes.byref(handle), None) == q3x.EINVAL
    assert lib.q3x_hip_engine_create(ctypes.byref(good), None, 8, 0, ctypes.byref(handle), None) == q3x.EINVAL
    assert lib.q3x_hip_engine_create(ctypes.byref(good), P, 8, -1, ctypes.byref(handle), None) == q3x.EINVAL
    assert lib.q3x_hip_engine_forward(None, P, 1, 1) == q3x.EINVAL
    assert lib.q3x_hip_engine_logits(None, P) == q3x.EINVAL
    assert lib.q3x_hip_engine_reset(None) == q3x.EINVAL
    assert lib.q3x_hip_engine_position(None) == -1
    lib.q3x_hip_engine_destroy(None)
