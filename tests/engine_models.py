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
}


def _bf16(values):
    return (np.ascontiguousarray(values, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def synthetic_model(fields: dict, seed: int):
    """(ModelConfig, image uint8, table [(role, layer, offset)]) for `fields`."""
    config = q3x.make_config(**fields)
    table, nbytes = q3x.model_schema(config)
    image = np.zeros(nbytes, np.uint8)
    rng = np.random.default_rng(seed)
    H = fields["H"]
    for t in table:
        role = q3x.TENSOR_ROLES[t.role]
        n = max(t.experts, 1) * t.rows * t.cols
        if t.type in (Q8_0, Q4_0):
            std = 1.0 if role in ("embedding", "lm_head") else 1.0 / np.sqrt(t.cols)
            data = oracle.quantize(t.type, rng.normal(0, std, n).astype(np.float32))
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
