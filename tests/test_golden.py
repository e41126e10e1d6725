"""The oracle against golden vectors written by the reference's own compiled CPU
code (tests/golden/make_golden.py), bit for bit.  Runs without the reference
tree."""
import os

import numpy as np
import pytest

import oracle
from tests.helpers import Q4_0, Q8_0, bits

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    path = os.path.join(GOLDEN, name)
    if not os.path.exists(path):
        pytest.fail(f"missing fixture {path}: run tests/golden/make_golden.py")
    return np.load(path, allow_pickle=False)


@pytest.mark.parametrize("type_,name", [(Q8_0, "mv_q8_0.npz"), (Q4_0, "mv_q4_0.npz")])
def test_mv_and_embed_match_reference_fixture(type_, name):
    f = load(name)
    i = 0
    while f"w{i}" in f:
        rows, cols = (int(v) for v in f[f"shape{i}"])
        w, x = f[f"w{i}"], f[f"x{i}"]
        assert np.array_equal(bits(oracle.mv_serial(w, type_, rows, cols, x)), bits(f[f"y{i}"]))
        assert np.array_equal(bits(oracle.dequant(w, type_, rows, cols)), bits(f[f"embed{i}"]))
        i += 1
    assert i == 4


def test_router_matches_reference_fixture():
    f = load("router.npz")
    i = 0
    while f"logits{i}" in f:
        k = f[f"ids{i}"].shape[1]
        ids, weights, _ = oracle.router_top_k(f[f"logits{i}"], k)
        assert np.array_equal(ids, f[f"ids{i}"])
        assert np.array_equal(bits(weights), bits(f[f"weights{i}"]))
        i += 1
    assert i == 4


def test_silu_matches_reference_fixture():
    f = load("silu.npz")
    sig = np.array([oracle.sigmoid(float(v)) for v in f["x"]], np.float32)
    silu = np.array([oracle.silu(float(v)) for v in f["x"]], np.float32)
    assert np.array_equal(bits(sig), bits(f["sigmoid"]))
    assert np.array_equal(bits(silu), bits(f["silu"]))


def test_moe_matches_reference_fixture():
    f = load("moe_q4_0.npz")
    E, H, I, k = (int(v) for v in f["shape"])
    ids, weights, _ = oracle.router_top_k(f["logits"], k)
    assert np.array_equal(ids, f["ids"])
    Y = oracle.moe_routed(f["gate_up"], f["down"], Q4_0, E, H, I, f["X"], ids, weights, threads=1)
    # The reference adds a zero shared expert: -0.0 becomes +0.0.
    assert np.array_equal(bits(Y + np.float32(0.0)), bits(f["Y"]))


def test_moe_layer_matches_reference_fixture():
    # engine.cpp moe() with every weight real, and the BF16 router mv().
    f = load("moe_layer_q8_0.npz")
    E, H, I, SI, k = (int(v) for v in f["shape"])
    for t in range(f["X"].shape[0]):
        assert np.array_equal(bits(oracle.mv_bf16(f["router"], f["X"][t])), bits(f["logits"][t]))
    Y, ids, _ = oracle.moe_layer(f["router"], f["gate_up"], f["down"], f["shared_gate"], f["shared_up"],
                                 f["shared_down"], f["shared_scale"], Q8_0, E, H, I, SI, k, f["X"], threads=1)
    assert np.array_equal(ids, f["ids"])
    assert np.array_equal(bits(Y), bits(f["Y"]))


@pytest.mark.parametrize("type_,key", [(Q8_0, "q8_0"), (Q4_0, "q4_0")])
def test_quantizer_matches_reference_packer_fixture(type_, key):
    # Vectors from scripts/pack_weights.py quantize_q8_0 / quantize_q4_0
    # (tests/golden/make_quantizer_golden.py), BF16 inputs widened exactly.
    f = load("quantizer.npz")
    values = (f["bf16"].astype(np.uint32) << 16).view(np.float32)
    assert np.array_equal(oracle.quantize(type_, values), f[key])
