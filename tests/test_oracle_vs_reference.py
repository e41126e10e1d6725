"""The oracle against the reference's own CPU code (oracle/_ref, compiled from
the reference sources where they lie), bit for bit, for every build this host
can run: the portable x86-64-v3 build and, on a CPU with AVX-512 F and BW,
the AVX-512 build (the reference's -march=native build on such a host, whose
BF16 matvec takes arch/x86/kernels.h; the oracle restates both dots).
Skipped where the reference tree was not available to build it; tests/golden/
carries vectors from the portable build for those hosts."""
import ctypes

import numpy as np
import pytest

import oracle
from tests.helpers import Q4_0, Q8_0, bits, random_blocks

BUILDS = oracle.ref_builds()
pytestmark = pytest.mark.skipif(not BUILDS, reason="oracle/_ref not built (no reference tree)")


@pytest.fixture(params=BUILDS, ids=[b[0] for b in BUILDS])
def build(request):
    """(handle, bf16_lanes) of one reference build."""
    return request.param[1], request.param[2]


def _p(a):
    return a.ctypes.data


def ref_mv(ref, w, type_, rows, cols, x):
    y = np.empty(rows, np.float32)
    assert ref.q3xr_try_mv(_p(w), type_, rows, cols, _p(x), _p(y)) == 1
    return y


def ref_embed(ref, w, type_, cols, row):
    out = np.empty(cols, np.float32)
    assert ref.q3xr_try_embed(_p(w), type_, cols, row, _p(out)) == 1
    return out


SPECIAL_SCALES = np.array([0x3555, 0x2E66, 0x0400, 0x0001, 0x8001, 0x03FF, 0x7BFF, 0xFBFF, 0x0000, 0x8000,
                           0x3C00, 0xB800], np.uint16)


@pytest.mark.parametrize("type_", [Q8_0, Q4_0])
@pytest.mark.parametrize("rows,cols", [(1, 32), (3, 64), (17, 96), (64, 256), (33, 4096), (5, 12288)])
@pytest.mark.parametrize("special", [False, True])
def test_mv_and_embed_bit_exact(build, type_, rows, cols, special):
    ref = build[0]
    rng = np.random.default_rng(rows * 7919 + cols + type_ + 1000 * special)
    w = random_blocks(rng, type_, rows, cols, SPECIAL_SCALES if special else None)
    x = rng.normal(0, 1, cols).astype(np.float32)
    assert np.array_equal(bits(oracle.mv_serial(w, type_, rows, cols, x)), bits(ref_mv(ref, w, type_, rows, cols, x)))
    for row in {0, rows // 2, rows - 1}:
        assert np.array_equal(bits(oracle.embed(w, type_, cols, row)), bits(ref_embed(ref, w, type_, cols, row)))


def test_quantized_bytes_agree(build):
    ref = build[0]
    for t in (0, Q8_0, Q4_0, 7):
        for rows, cols in [(3, 64), (0, 32), (1, -32), (1, 33), (1, 16), (4096, 4096), (151936, 4096),
                           (2147483647, 2147483616)]:
            a = ctypes.c_size_t(123)
            ok = ref.q3xr_quantized_bytes(t, rows, cols, ctypes.byref(a))
            mine = oracle.quantized_bytes(t, rows, cols)
            assert (mine is not None) == bool(ok)
            if ok:
                assert mine == a.value


@pytest.mark.parametrize("experts,top_k", [(6, 3), (256, 8), (64, 1), (256, 2)])
def test_router_bit_exact(build, experts, top_k):
    ref = build[0]
    rng = np.random.default_rng(experts * 31 + top_k)
    for t in range(50):
        logits = rng.normal(0, 1 + 3 * (t % 3), experts).astype(np.float32)
        if t % 5 == 0:
            logits[rng.integers(0, experts, 4)] = logits.max()  # exact ties
        ids_r = np.zeros(top_k, np.int32)
        probs_r = np.zeros(experts, np.float32)
        ref.q3xr_router_top_k(_p(logits), experts, top_k, _p(ids_r), _p(probs_r))
        ids, weights, _ = oracle.router_top_k(logits, top_k)
        assert np.array_equal(ids[0], ids_r)
        assert np.array_equal(bits(weights[0]), bits(probs_r[ids_r]))


def test_silu_sigmoid_bit_exact(build):
    ref = build[0]
    rng = np.random.default_rng(9)
    values = np.concatenate([rng.normal(0, 6, 2000), [0.0, -0.0, 88.0, -88.0, 1e-30, -1e-30, 20.0]])
    for v in values.astype(np.float32):
        assert np.float32(ref.q3xr_sigmoid(float(v))).view(np.uint32) == np.float32(oracle.sigmoid(float(v))).view(np.uint32)
        assert np.float32(ref.q3xr_silu(float(v))).view(np.uint32) == np.float32(oracle.silu(float(v))).view(np.uint32)


@pytest.mark.parametrize("experts,H,I,top_k", [(8, 64, 32, 2), (16, 256, 64, 8), (256, 2048, 512, 8)])
def test_moe_routed_bit_exact_against_reference_moe(build, experts, H, I, top_k):
    ref = build[0]
    # The reference moe() (engine.cpp:406-430) with a BF16 router and an
    # all-zero shared expert, against this oracle's router + routed loop fed
    # the reference's router logits.
    rng = np.random.default_rng(experts + H + I)
    router = (rng.normal(0, 0.5, (experts, H)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    gate_up = random_blocks(rng, Q4_0, experts * 2 * I, H)
    down = random_blocks(rng, Q4_0, experts * H, I)
    for t in range(3 if experts < 256 else 1):
        x = rng.normal(0, 1, H).astype(np.float32)
        logits = np.zeros(experts, np.float32)
        ids_r = np.zeros(top_k, np.int32)
        out_r = np.zeros(H, np.float32)
        ref.q3xr_moe_q4(_p(router), _p(gate_up), _p(down), experts, H, I, top_k, _p(x), _p(logits), _p(ids_r),
                        _p(out_r))
        ids, weights, _ = oracle.router_top_k(logits, top_k)
        assert np.array_equal(ids[0], ids_r)
        y = oracle.moe_routed(gate_up, down, Q4_0, experts, H, I, x, ids, weights, threads=1)
        # shared expert adds sigmoid(0) * 0: -0.0 becomes +0.0, nothing else changes
        assert np.array_equal(bits(y[0] + np.float32(0.0)), bits(out_r))


def bf16_matrix(rng, rows, cols, scale):
    """Random BF16 values (float32 truncated to its top 16 bits) as uint16."""
    return (rng.normal(0, scale, (rows, cols)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)


@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 64), (256, 2048), (7, 1000)])
def test_mv_bf16_bit_exact(build, rows, cols):
    ref, lanes = build
    rng = np.random.default_rng(rows * 7 + cols)
    w = bf16_matrix(rng, rows, cols, 0.05)
    x = rng.normal(0, 1, cols).astype(np.float32)
    y_ref = np.empty(rows, np.float32)
    ref.q3xr_mv_bf16(_p(w), rows, cols, _p(x), _p(y_ref))
    assert np.array_equal(bits(oracle.mv_bf16(w, x, bf16_lanes=lanes)), bits(y_ref))


@pytest.mark.parametrize("type_,experts,H,I,shared_I,top_k", [
    (Q4_0, 8, 64, 32, 32, 2),
    (Q8_0, 16, 256, 64, 32, 8),        # shared expert narrower than the routed ones
    (Q4_0, 256, 2048, 512, 512, 8),    # 35B-A3B shapes
])
def test_moe_layer_bit_exact_against_reference_moe(build, type_, experts, H, I, shared_I, top_k):
    # The reference moe() (engine.cpp:406-430) with every weight real: BF16
    # router and shared-expert gate, routed experts and shared expert of one
    # quantised type; the oracle restates the whole layer.
    ref, lanes = build
    rng = np.random.default_rng(experts + H + I + shared_I)
    router = bf16_matrix(rng, experts, H, 0.5)
    scale = bf16_matrix(rng, 1, H, 0.05)
    gate_up = random_blocks(rng, type_, experts * 2 * I, H)
    down = random_blocks(rng, type_, experts * H, I)
    sg = random_blocks(rng, type_, shared_I, H)
    su = random_blocks(rng, type_, shared_I, H)
    sd = random_blocks(rng, type_, H, shared_I)
    X = rng.normal(0, 1, (3 if experts < 256 else 1, H)).astype(np.float32)
    Y, ids, _ = oracle.moe_layer(router, gate_up, down, sg, su, sd, scale, type_, experts, H, I, shared_I,
                                 top_k, X, threads=1, bf16_lanes=lanes)
    for t in range(X.shape[0]):
        out_r = np.empty(H, np.float32)
        ids_r = np.empty(top_k, np.int32)
        ref.q3xr_moe_layer(type_, _p(router), _p(gate_up), _p(down), _p(sg), _p(su), _p(sd), _p(scale), experts,
                           H, I, shared_I, top_k, _p(X[t]), _p(out_r), _p(ids_r))
        assert np.array_equal(ids[t], ids_r)
        assert np.array_equal(bits(Y[t]), bits(out_r))


@pytest.mark.skipif(len(BUILDS) < 2, reason="one reference build on this host")
def test_the_two_builds_sum_bf16_differently():
    # The AVX-512 build takes arch/x86/kernels.h for BF16 (16 lane sums), the
    # portable build the scalar loop: on a long row they round differently,
    # so matching each bit for bit pins two distinct restatements.
    rng = np.random.default_rng(11)
    w = bf16_matrix(rng, 64, 2048, 0.05)
    x = rng.normal(0, 1, 2048).astype(np.float32)
    outs = []
    for _, handle, _ in BUILDS:
        y = np.empty(64, np.float32)
        handle.q3xr_mv_bf16(_p(w), 64, 2048, _p(x), _p(y))
        outs.append(y)
    assert not np.array_equal(bits(outs[0]), bits(outs[1]))
