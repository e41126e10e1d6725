"""CPU tests of the oracle (oracle/q3x_oracle.c): pinned against the reference's
known answers, closed forms, exhaustive checks and double-precision brute
force.  Bit-exact equality with the reference's own build lives in
test_oracle_vs_reference.py and test_golden.py."""
import hashlib
import math
import struct

import numpy as np
import pytest

import oracle
from tests.helpers import (Q4_0, Q8_0, bits, dequant_numpy, lcg_sampler, q4_blocks, q8_blocks,
                           random_blocks)


# ---------------------------------------------------------------- f16 -------

@pytest.mark.parametrize("bits_,value", [
    (0x3C00, 1.0), (0x3800, 0.5), (0x4000, 2.0), (0x3400, 0.25),        # q8_cpu_test.cpp:272-283
    (0x3555, 0.333251953125), (0x2E66, 0.0999755859375),                 # q8_cpu_test.cpp:110-112
    (0x0400, 0.00006103515625), (0x0001, 0.000000059604644775390625),
    (0x8000, -0.0), (0x7C00, math.inf), (0xFC00, -math.inf), (0x7BFF, 65504.0),
])
def test_f16_known_answers(bits_, value):
    got = oracle.f16(bits_)
    assert got == value and math.copysign(1.0, got) == math.copysign(1.0, value)


def test_f16_exhaustive_matches_ieee_conversion():
    # Closed form: IEEE binary16 -> binary32 is exact; numpy converts by bit
    # manipulation (payload-preserving for NaN), so all 65536 patterns match.
    allbits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = allbits.view(np.float16).astype(np.float32).view(np.uint32)
    got = np.array([oracle.lib().q3xo_f16(int(b)) for b in allbits], np.float32).view(np.uint32)
    finite = np.isfinite(allbits.view(np.float16))
    assert np.array_equal(got[finite], want[finite])
    nan = np.isnan(allbits.view(np.float16))
    assert np.isnan(got.view(np.float32)[nan]).all()
    inf = np.isinf(allbits.view(np.float16))
    assert np.array_equal(got[inf], want[inf])


# ------------------------------------------------------- quantized_bytes ----

def test_quantized_bytes_known_answers():
    # tests/q8_cpu_test.cpp:17-43
    assert oracle.quantized_bytes(0, 3, 17) is None           # BF16 is not quantised
    assert oracle.quantized_bytes(Q8_0, 3, 64) == 204
    assert oracle.quantized_bytes(Q4_0, 3, 64) == 108
    for t in (0, Q8_0, Q4_0):
        assert oracle.quantized_bytes(t, 0, 32) is None
        assert oracle.quantized_bytes(t, 1, -32) is None
    assert oracle.quantized_bytes(Q8_0, 1, 33) is None
    assert oracle.quantized_bytes(Q4_0, 1, 16) is None
    assert oracle.quantized_bytes(999, 1, 32) is None
    large_cols = 2147483616
    assert oracle.quantized_bytes(Q8_0, 2147483647, large_cols) == 2147483647 * (large_cols // 32) * 34


# --------------------------------------------------------- known answers ----

def _q8_fixed():
    """tests/q8_cpu_test.cpp:271-283: four blocks, two rows of 64."""
    scales = [0x3C00, 0x3800, 0x4000, 0x3400]
    values = [[(i % 9) - 4 + b for i in range(32)] for b in range(4)]
    x = np.array([(i % 7 - 3) * 0.125 for i in range(64)], np.float32)
    return q8_blocks(scales, values), values, x, [1.0, 0.5, 2.0, 0.25]


def test_q8_fixed_vector_and_embed():
    w, values, x, dec = _q8_fixed()
    expected = []
    for row in range(2):
        acc = np.float32(0)
        for blk in range(2):
            inner = np.float32(0)
            for i in range(32):
                inner = np.float32(inner + np.float32(values[row * 2 + blk][i]) * x[blk * 32 + i])
            acc = np.float32(acc + np.float32(dec[row * 2 + blk]) * inner)
        expected.append(acc)
    y = oracle.mv(w, Q8_0, 2, 64, x)
    assert abs(y[0] - expected[0]) < 1e-6 and abs(y[1] - expected[1]) < 1e-6
    emb = oracle.embed(w, Q8_0, 64, 1)
    for blk in range(2):
        for i in range(32):
            assert emb[blk * 32 + i] == np.float32(dec[2 + blk]) * np.float32(values[2 + blk][i])


def test_q4_math_fixed_vector_and_embed():
    # tests/q4_cpu_test.cpp:138-178
    scales = [0x3C00, 0x3800, 0x4000, 0x3400]
    nib = [[((i + b) % 16) | (((15 - i + b) % 16) << 4) for i in range(16)] for b in range(4)]
    w = q4_blocks(scales, nib)
    x = np.array([(i % 7 - 3) * 0.125 for i in range(64)], np.float32)
    dec = [1.0, 0.5, 2.0, 0.25]
    expected = np.zeros(2)
    for row in range(2):
        for blk in range(2):
            for i in range(16):
                p = nib[row * 2 + blk][i]
                expected[row] += dec[row * 2 + blk] * ((p & 15) - 8) * x[blk * 32 + i]
                expected[row] += dec[row * 2 + blk] * ((p >> 4) - 8) * x[blk * 32 + i + 16]
    y = oracle.mv(w, Q4_0, 2, 64, x)
    assert np.all(np.abs(y - expected) < 1e-6)
    emb = oracle.embed(w, Q4_0, 64, 1)
    for i in range(16):
        assert emb[i] == 2.0 * ((nib[2][i] & 15) - 8)
        assert emb[i + 16] == 2.0 * ((nib[2][i] >> 4) - 8)


def test_q4_single_row_from_q8_test():
    # tests/q8_cpu_test.cpp:336-360: one Q4 row of two blocks.
    scales = [0x3C00, 0x3800]
    nib = [[((i + b) % 16) | (((i + b + 3) % 16) << 4) for i in range(16)] for b in range(2)]
    w = q4_blocks(scales, nib)
    x = np.array([(i % 7 - 3) * 0.125 for i in range(64)], np.float32)
    deq = dequant_numpy(w, Q4_0, 1, 64)
    expected = float(np.dot(deq[0].astype(np.float64), x.astype(np.float64)))
    assert abs(oracle.mv(w, Q4_0, 1, 64, x)[0] - expected) < 1e-6
    assert np.array_equal(oracle.embed(w, Q4_0, 64, 0), deq[0])


# ------------------------------------------------ double-precision brute force

@pytest.mark.parametrize("rows", [3, 1023, 1024, 1031])
def test_q8_random_rows_against_double(rows):
    # tests/q8_cpu_test.cpp:110-134: non-binary-exact and subnormal scales,
    # LCG data, bound 2e-6 * (1 + sum |p|).
    sample = lcg_sampler(42 + rows)
    cols, blocks = 96, 3
    scales = np.array([0x3555, 0x2E66, 0x0400, 0x0001], np.uint16)
    decoded = [0.333251953125, 0.0999755859375, 0.00006103515625, 0.000000059604644775390625]
    x = np.array([sample() for _ in range(cols)], np.float32)
    vals = np.array([[int(np.float32(sample() * np.float32(127))) for _ in range(32)]
                     for _ in range(rows * blocks)])
    w = q8_blocks(scales[np.arange(rows * blocks) % 4], vals)
    y = oracle.mv(w, Q8_0, rows, cols, x)
    for row in range(rows):
        idx = row * blocks + np.arange(blocks)
        prod = (np.array([decoded[i % 4] for i in idx])[:, None] * vals[idx].astype(np.float64)
                * x.reshape(blocks, 32).astype(np.float64))
        assert abs(y[row] - prod.sum()) <= 2e-6 * (1.0 + np.abs(prod).sum())


@pytest.mark.parametrize("type_", [Q8_0, Q4_0])
@pytest.mark.parametrize("rows,cols", [(5, 32), (7, 96), (16, 256), (9, 2048)])
def test_random_mv_against_double(type_, rows, cols):
    rng = np.random.default_rng(1000 * type_ + rows + cols)
    w = random_blocks(rng, type_, rows, cols)
    x = rng.normal(0, 1, cols).astype(np.float32)
    deq = dequant_numpy(w, type_, rows, cols).astype(np.float64)
    y = oracle.mv(w, type_, rows, cols, x)
    prod = deq * x.astype(np.float64)
    assert np.all(np.abs(y - prod.sum(1)) <= 2e-6 * (1.0 + np.abs(prod).sum(1)))
    # A transposed or shifted operand would fail this: rows are distinct.
    assert np.array_equal(oracle.dequant(w, type_, rows, cols), deq.astype(np.float32))


def test_parallel_mv_and_gemm_are_bit_identical_to_serial():
    rng = np.random.default_rng(7)
    for type_ in (Q8_0, Q4_0):
        rows, cols = 301, 512
        w = random_blocks(rng, type_, rows, cols)
        X = rng.normal(0, 1, (5, cols)).astype(np.float32)
        serial = np.stack([oracle.mv_serial(w, type_, rows, cols, X[t]) for t in range(5)])
        assert np.array_equal(bits(oracle.gemm(w, type_, rows, cols, X, threads=7)), bits(serial))
        assert np.array_equal(bits(oracle.mv(w, type_, rows, cols, X[2], threads=3)), bits(serial[2]))


def test_mv_uses_the_reference_fused_accumulation():
    # The reference build contracts `inner += q * x` into one FMA per step
    # (a single rounding).  With q = 127 and x = 2^20 + 3 the exact product
    # needs 27 significant bits, so an unfused multiply would round it first;
    # the oracle must reproduce the fused sequence bit for bit.
    w = q8_blocks([0x3C00], [[127] * 32])
    x = np.full(32, np.float32(2.0 ** 20 + 3), np.float32)
    inner = np.float32(0)
    unfused = np.float32(0)
    for _ in range(32):
        inner = np.float32(np.float64(inner) + 127.0 * np.float64(x[0]))  # exact sum, one rounding
        unfused = np.float32(unfused + np.float32(127.0) * x[0])          # product rounded first
    assert inner != unfused
    assert oracle.mv(w, Q8_0, 1, 32, x)[0] == inner


# ---------------------------------------------------------------- router ----

def test_router_known_answers():
    # tests/q4_cpu_test.cpp:180-202
    ids, weights, _ = oracle.router_top_k(np.array([-2, 3, 1, 4, -1, 2], np.float32), 3)
    assert list(ids[0]) == [3, 1, 5]
    assert abs(weights[0].sum() - 1.0) < 1e-6
    ids, weights, _ = oracle.router_top_k(np.arange(256, dtype=np.float32) * 0.03125, 8)
    assert list(ids[0]) == [255 - s for s in range(8)]
    assert abs(weights[0].sum() - 1.0) < 1e-6


def test_router_matches_brute_force_sort():
    rng = np.random.default_rng(11)
    logits = rng.normal(0, 1, (64, 256)).astype(np.float32)
    ids, weights, probs = oracle.router_top_k(logits, 8)
    for t in range(64):
        # stable descending sort by probability, ties to the lower index
        order = sorted(range(256), key=lambda e: (-probs[t, e], e))[:8]
        assert list(ids[t]) == order
        expect = probs[t, order].astype(np.float64) / probs[t, order].astype(np.float64).sum()
        assert np.allclose(weights[t], expect, rtol=1e-6, atol=0)
        soft = np.exp(logits[t].astype(np.float64) - logits[t].max())
        assert np.allclose(probs[t], soft / soft.sum(), rtol=1e-5, atol=1e-12)


def test_router_ties_go_to_lowest_index():
    logits = np.zeros(16, np.float32)
    ids, weights, _ = oracle.router_top_k(logits, 4)
    assert list(ids[0]) == [0, 1, 2, 3]
    assert np.all(weights[0] == np.float32(0.25))


# ------------------------------------------------------------------- MoE ----

def test_moe_constant_nibble_closed_form():
    # tests/q4_cuda_test.cu:62-107: nibble 9 (value 1) everywhere, expert scales
    # 0.25 / 0.5 / 1 / 2, ids {2, 1}, weights {0.75, 0.25}.
    E, H, I = 4, 32, 32
    scales = [0x3400, 0x3800, 0x3C00, 0x4000]
    gate_up = np.concatenate([q4_blocks([scales[e]] * (2 * I * H // 32), np.full((2 * I * H // 32, 16), 0x99))
                              for e in range(E)])
    down = np.concatenate([q4_blocks([scales[e]] * (H * I // 32), np.full((H * I // 32, 16), 0x99))
                           for e in range(E)])
    x = (0.03125 * (np.arange(H) + 1)).astype(np.float32)
    y = oracle.moe_routed(gate_up, down, Q4_0, E, H, I, x, np.array([[2, 1]]), np.array([[0.75, 0.25]]))
    silu = lambda v: v / (1.0 + math.exp(-v))  # noqa: E731
    g2, g1 = 16.5, 8.25
    expected = 0.75 * I * silu(g2) * g2 + 0.25 * 0.5 * I * silu(g1) * g1
    assert np.all(np.abs(y - expected) < 1e-2)


def test_moe_is_composition_of_pinned_matvecs():
    # Routed loop restated from pinned pieces: for each slot, mv(gate_up_e) ->
    # silu(g)*u -> mv(down_e) -> out += w*d, slot order from zero.
    rng = np.random.default_rng(5)
    E, H, I, k = 6, 64, 32, 3
    gu = random_blocks(rng, Q4_0, E * 2 * I, H)
    dn = random_blocks(rng, Q4_0, E * H, I)
    X = rng.normal(0, 1, (4, H)).astype(np.float32)
    ids = np.array([[5, 0, 2], [1, 1 + 2, 4], [0, 5, 3], [2, 4, 1]], np.int32)
    w = rng.random((4, k)).astype(np.float32)
    Y = oracle.moe_routed(gu, dn, Q4_0, E, H, I, X, ids, w)
    gstride, dstride = 2 * I * H // 32 * 18, H * I // 32 * 18
    for t in range(4):
        out = np.zeros(H, np.float32)
        for s in range(k):
            e = ids[t, s]
            g = oracle.mv_serial(gu[e * gstride:(e + 1) * gstride], Q4_0, 2 * I, H, X[t])
            h = np.array([np.float32(np.float32(oracle.silu(float(g[i]))) * g[I + i]) for i in range(I)],
                         np.float32)
            d = oracle.mv_serial(dn[e * dstride:(e + 1) * dstride], Q4_0, H, I, h)
            out = (np.float64(w[t, s]) * d.astype(np.float64) + out.astype(np.float64)).astype(np.float32)
        assert np.array_equal(bits(Y[t]), bits(out))


def test_silu_sigmoid_closed_forms():
    assert oracle.sigmoid(0.0) == 0.5
    for v in (-30.0, -3.5, -1e-3, 0.0, 1e-3, 2.0, 17.0):
        exact = 1.0 / (1.0 + math.exp(-v))
        assert abs(oracle.sigmoid(v) - exact) <= 2e-7 * exact
        assert abs(oracle.silu(v) - v * exact) <= 3e-7 * abs(v * exact) + 1e-30


# ------------------------------------------------------------- quantizer ----

def _bf16_bytes(values):
    v = np.asarray(values, np.float32)
    return (v.view(np.uint32) >> 16).astype(np.uint16)


def _from_bf16(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def test_q8_quantizer_boundaries():
    # tests/test_pack_weights.py:204-211
    values = np.zeros(64, np.float32)
    values[32:38] = [127.0, -127.0, 126.5, -126.5, 0.5, -0.5]
    packed = oracle.quantize(Q8_0, values)
    assert packed[:34].tobytes() == bytes(34)
    assert struct.unpack_from("<6b", packed.tobytes(), 36) == (127, -127, 127, -127, 1, -1)


def test_q4_quantizer_zero_block_and_layout():
    # tests/test_pack_weights.py:227-236
    rng = np.random.default_rng(20260906)
    values = rng.normal(size=32 * 17).astype(np.float32)
    values[:32] = 0
    values[32:40] = [8.0, -8.0, 7.5, -7.5, 0.5, -0.5, 1.5, -1.5]
    values = _from_bf16(_bf16_bytes(values))
    packed = oracle.quantize(Q4_0, values).tobytes()
    assert packed[:2] == b"\0\x80"
    assert packed[2:18] == bytes([0x88] * 16)


def test_q4_quantizer_matches_llama_cpp_sha256():
    # tests/q4_llama_reference.py:24-30 with the published digest
    # (eval/qwen36-35b-q4.md:53-57): byte-exact with llama.cpp's
    # quantize_row_q4_0_ref on these 4096 BF16 blocks.
    rng = np.random.default_rng(20260907)
    values = rng.normal(size=4096 * 32).astype("<f4")
    values[:32] = 0
    values[32:64] = np.linspace(-8, 7.5, 32, dtype="<f4")
    values[64:96] = np.linspace(8, -7.5, 32, dtype="<f4")
    values = _from_bf16(_bf16_bytes(values))
    digest = hashlib.sha256(oracle.quantize(Q4_0, values).tobytes()).hexdigest()
    assert digest == "735e40577b24f36e3ff4cc1a12bd085e7648b1b0099d0ae0b0700b371a64532c"


def test_q8_quantizer_properties():
    rng = np.random.default_rng(3)
    values = rng.normal(0, 0.02, 32 * 512).astype(np.float32)
    values[:32] *= 1e-3
    packed = oracle.quantize(Q8_0, values)
    blk = packed.reshape(-1, 34)
    v = values.reshape(-1, 32)
    scale32 = np.abs(v).max(1) / np.float32(127)
    assert np.array_equal(blk[:, :2].copy().view(np.uint16).reshape(-1),
                          scale32.astype(np.float16).view(np.uint16))
    q = blk[:, 2:].view(np.int8).astype(np.int32)
    # the largest magnitude maps to +-127 and every value rounds to nearest
    assert np.all(np.abs(q).max(1) == 127)
    inv = (np.float32(1) / scale32).astype(np.float32)
    n = (v * inv[:, None]).astype(np.float32)
    assert np.all(np.abs(q - n) <= 0.5 + 1e-6)
    assert np.all(np.sign(q) * np.sign(n) >= 0)


def test_quantizer_rejects_partial_and_nonfinite():
    with pytest.raises(ValueError):
        oracle.quantize(Q8_0, np.zeros(31, np.float32))
    bad = np.zeros(32, np.float32)
    bad[4] = np.inf
    with pytest.raises(ValueError):
        oracle.quantize(Q4_0, bad)
