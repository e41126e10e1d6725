"""Small synthetic models for the engine tests: a configuration with the real
head sizes (KD = VD = 128, AD = 256, RD = 64) and few heads, layers and
experts, and its weights as a model.bin image built on the host (matrices
quantized by the oracle's restatement of the packer's quantizers, vectors
drawn at scales that keep activations near unit size through the layers)."""
import numpy as np

import oracle
import qwen3x_amd as q3x

Q8_0, Q4_0 = q3x.MATRIX_Q8_0, q3x.MATRIX_Q4_0

BASE = dict(V=512, H=256, I=512, N=4, AI=4, AH=2, KVH=1, AD=256, RD=64, KH=1, VH=2, KD=128, VD=128, CK=4,
            experts=0, top_k=0, shared_I=0, tied_embeddings=0)

CONFIGS = {
    # three DeltaNet layers and one attention layer, dense FFN
    "dense_q8": dict(BASE, id=1, matrix_type=Q8_0),
    # two rounds of the layer pattern, Q4_0, GQA with two query heads per KV head
    "dense_q4": dict(BASE, id=2, matrix_type=Q4_0, N=8, AH=4, KVH=2, KH=2, VH=4),
    # MoE layers: 8 experts, top 2, shared expert (VH * VD >= H, as the reference's work buffers need)
    "moe_q4": dict(BASE, id=3, matrix_type=Q4_0, I=64, experts=8, top_k=2, shared_I=64),
    # tied embeddings, Q8_0 MoE, a shared expert narrower than the routed ones
    "moe_q8_tied": dict(BASE, id=4, matrix_type=Q8_0, I=128, experts=8, top_k=3, shared_I=64, tied_embeddings=1),
    # eight query heads per KV head (the 35B-A3B's grouping) and four value heads per key head
    "gqa8_q8": dict(BASE, id=5, matrix_type=Q8_0, AH=8, KVH=1, KH=1, VH=4),
    # narrow recurrent heads (KD = 64, VD = 96, three value heads per key head):
    # zero-padded key and value slots in the scans, the gated norm over heads
    # that are not 128 wide, an output projection 288 columns wide
    "narrow_q4": dict(BASE, id=6, matrix_type=Q4_0, KD=64, VD=96, KH=1, VH=3),
    # head sizes that are not multiples of 32 (KD = 48, VD = 80): the prefill
    # recurrence runs token by token instead of in chunks on the matrix cores
    "odd_q8": dict(BASE, id=7, matrix_type=Q8_0, KD=48, VD=80, KH=2, VH=4),
}


# The production widths of the three quantized models (model_config.h:77-102:
# Qwen3.5-9B Q8_0, Qwen3.8-27B Q4_0, Qwen3.6-35B-A3B Q4_0) with four layers
# (three DeltaNet and one attention) and a small vocabulary.
WIDE_BASE = dict(V=1024, N=4, AI=4, AD=256, RD=64, KD=128, VD=128, CK=4, experts=0, top_k=0, shared_I=0,
                 tied_embeddings=0)
WIDE = {
    "wide_9b_q8": dict(WIDE_BASE, id=11, matrix_type=Q8_0, H=4096, I=12288, AH=16, KVH=4, KH=16, VH=32),
    "wide_27b_q4": dict(WIDE_BASE, id=12, matrix_type=Q4_0, H=5120, I=17408, AH=24, KVH=4, KH=16, VH=48),
    "wide_35b_a3b_q4": dict(WIDE_BASE, id=13, matrix_type=Q4_0, H=2048, I=512, AH=16, KVH=2, KH=16, VH=32,
                            experts=256, top_k=8, shared_I=512),
}


def _bf16(values):
    return (np.ascontiguousarray(values, np.float32).view(np.uint32) >> 16).astype(np.uint16)


# Root mean square of the block values: Q8_0 q uniform in [-128, 127], Q4_0
# nibble - 8 uniform in [-8, 7].
_VALUE_RMS = {Q8_0: np.sqrt(np.mean(np.arange(-128, 128) ** 2.0)), Q4_0: np.sqrt(np.mean(np.arange(-8, 8) ** 2.0))}


def _quantized_oracle(rng, type_, n, std):
    return oracle.quantize(type_, rng.normal(0, std, n).astype(np.float32))


def _quantized_random(rng, type_, n, std):
    # Uniform block values with fp16 scales drawn from N(0, std / value rms):
    # weights of standard deviation std, symmetric through the scale's sign.
    # Fast for the production widths, where quantizing normal draws is slow.
    nb = n // 32
    block = 34 if type_ == Q8_0 else 18
    words = (nb * block + 7) // 8
    data = rng.integers(0, 2**64 - 1, words, dtype=np.uint64, endpoint=True).view(np.uint8)
    data = data[:nb * block].reshape(nb, block)
    scales = rng.normal(0, std / _VALUE_RMS[type_], nb).astype(np.float16)
    data[:, 0:2] = scales.view(np.uint8).reshape(nb, 2)
    return data.reshape(-1)


def synthetic_model(fields: dict, seed: int, quantized=_quantized_oracle, head_std=1.0):
    """(ModelConfig, image uint8, table [(role, layer, offset)]) for `fields`.
    Matrices are drawn with standard deviation 1/sqrt(cols), so activations
    stay near unit size; the embedding with 1, lm_head with `head_std`."""
    config = q3x.make_config(**fields)
    table, nbytes = q3x.model_schema(config)
    image = np.zeros(nbytes, np.uint8)
    rng = np.random.default_rng(seed)
    H = fields["H"]
    for t in table:
        role = q3x.TENSOR_ROLES[t.role]
        n = max(t.experts, 1) * t.rows * t.cols
        if t.type in (Q8_0, Q4_0):
            std = 1.0 if role == "embedding" else head_std if role == "lm_head" else 1.0 / np.sqrt(t.cols)
            data = quantized(rng, t.type, n, std)
        elif t.type == q3x.TENSOR_F32:
            base = -1.0 if role == "delta_alog" else 1.0
            data = (base + rng.normal(0, 0.2, n)).astype(np.float32).view(np.uint8)
        else:
            std = {"moe_router": 1.0 / np.sqrt(H), "moe_shared_scale": 1.0 / np.sqrt(H), "delta_conv": 0.5,
                   "delta_dt": 0.5}.get(role, 0.1)
            data = _bf16(rng.normal(0, std, n)).view(np.uint8)
        assert data.size == t.bytes, role
        image[t.offset:t.offset + t.bytes] = data
    return config, image, [(t.role, t.layer, t.offset) for t in table]


def wide_model(fields: dict, seed: int):
    """synthetic_model at production widths, matrices from random blocks.
    lm_head is drawn like the layer matrices (1/sqrt(H)), so the logits are
    of order one, as in the reference's own forward test (its weights carry
    fp16 scales near 2^-11, tests/metal_test.mm:41-47), whose bound
    2e-4 + 2e-4 |a| assumes logits of that size."""
    return synthetic_model(fields, seed, quantized=_quantized_random, head_std=1.0 / np.sqrt(fields["H"]))
