"""Synthetic workloads of the benchmark configurations, generated on the GPU.

Weights are FP32 N(0, 0.02) values quantised to Q8_0 / Q4_0 in 32-element
blocks by the library's own quantizer (q3x_hip_quantize, the reference
packer's algorithm); activations and router logits are FP32 N(0, 1).  Every
tensor has a fixed seed: SEED_BASE + config index, plus a per-tensor offset.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Tuple

import qwen3x_amd as q3x

SEED_BASE = 20261201

# (name, rows, cols) of each matrix; rows = output features.
CONFIGS = {
    0: dict(name="q8_0_matvec_4096x4096", type=q3x.MATRIX_Q8_0, tokens=(1,),
            mats=[("w", 4096, 4096)]),
    1: dict(name="q8_0_decode_9b_layer_and_lm_head", type=q3x.MATRIX_Q8_0, tokens=(1,),
            mats=[("q", 4096, 4096), ("k", 4096, 4096), ("v", 4096, 4096), ("o", 4096, 4096),
                  ("gate", 12288, 4096), ("up", 12288, 4096), ("down", 4096, 12288),
                  ("lm_head", 151936, 4096)]),
    2: dict(name="q8_0_prefill_9b_ffn", type=q3x.MATRIX_Q8_0, tokens=(512, 4096),
            mats=[("gate", 12288, 4096), ("up", 12288, 4096), ("down", 4096, 12288)]),
    3: dict(name="q4_0_27b_ffn", type=q3x.MATRIX_Q4_0, tokens=(1, 512),
            mats=[("gate", 17408, 5120), ("up", 17408, 5120), ("down", 5120, 17408)]),
    4: dict(name="q4_0_moe_35b_a3b_routed", type=q3x.MATRIX_Q4_0, tokens=(1, 2048),
            experts=256, H=2048, I=512, top_k=8, shared_I=512),
}


def _torch():
    import torch
    return torch


def normal(shape, seed: int, std: float = 1.0, device="cuda"):
    torch = _torch()
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    out = torch.randn(shape, generator=g, device=device, dtype=torch.float32)
    if std != 1.0:
        out.mul_(std)
    return out


def quantized_matrix(type_: int, rows: int, cols: int, seed: int, device="cuda", chunk_rows: int = 16384):
    """Q8_0/Q4_0 bytes of an N(0, 0.02) FP32 matrix, quantised on the GPU."""
    torch = _torch()
    nbytes = q3x.quantized_bytes(type_, rows, cols)
    out = torch.empty(nbytes, dtype=torch.uint8, device=device)
    row_bytes = nbytes // rows
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    for r0 in range(0, rows, chunk_rows):
        n = min(chunk_rows, rows - r0)
        src = torch.randn((n, cols), generator=g, device=device, dtype=torch.float32).mul_(0.02)
        q3x.quantize(type_, src, n, cols, out[r0 * row_bytes:(r0 + n) * row_bytes])
    return out


@dataclass
class Matrix:
    name: str
    type: int
    rows: int
    cols: int
    weight: object  # uint8 device tensor

    @property
    def linear(self) -> q3x.Linear:
        return q3x.Linear(self.weight, self.rows, self.cols, self.type)

    @property
    def nbytes(self) -> int:
        return self.weight.numel()


def dense_matrices(index: int, device="cuda") -> List[Matrix]:
    cfg = CONFIGS[index]
    seed = SEED_BASE + index
    return [Matrix(name, cfg["type"], rows, cols, quantized_matrix(cfg["type"], rows, cols, seed * 1000 + i, device))
            for i, (name, rows, cols) in enumerate(cfg["mats"])]


def activations(index: int, count: int, cols: int, device="cuda", salt: int = 0):
    seed = (SEED_BASE + index) * 1000 + 500 + salt
    return normal((count, cols), seed, 1.0, device)


@dataclass
class MoeWeights:
    type: int
    experts: int
    H: int
    I: int
    gate_up: object
    down: object

    @property
    def gate_up_linear(self) -> q3x.ExpertLinear:
        return q3x.ExpertLinear(self.gate_up, self.experts, 2 * self.I, self.H, self.type)

    @property
    def down_linear(self) -> q3x.ExpertLinear:
        return q3x.ExpertLinear(self.down, self.experts, self.H, self.I, self.type)


def moe_weights(index: int = 4, device="cuda") -> MoeWeights:
    cfg = CONFIGS[index]
    seed = (SEED_BASE + index) * 1000
    E, H, I = cfg["experts"], cfg["H"], cfg["I"]
    gate_up = quantized_matrix(cfg["type"], E * 2 * I, H, seed + 1, device)
    down = quantized_matrix(cfg["type"], E * H, I, seed + 2, device)
    return MoeWeights(cfg["type"], E, H, I, gate_up, down)


def bf16_matrix(rows: int, cols: int, seed: int, std: float, device="cuda"):
    """BF16 bits (int16 tensor) of an N(0, std) FP32 matrix, truncated to BF16."""
    return normal((rows, cols), seed, std, device).view(_torch().int16)[:, 1::2].contiguous()


def moe_layer_weights(index: int = 4, device="cuda") -> q3x.MoeLayer:
    """Config 4's routed experts plus the rest of the layer (engine.cpp:406-430):
    a BF16 router with N(0, 1/H) weights (logits of N(0, 1) inputs come out
    N(0, 1), as the routed-only benchmark feeds them), a BF16 shared-expert
    gate and a shared expert of shared_I = 512 (the 35B-A3B configuration,
    model_config.h) quantised like the experts."""
    cfg = CONFIGS[index]
    routed = moe_weights(index, device)
    seed = (SEED_BASE + index) * 1000
    E, H, I, SI, t = cfg["experts"], cfg["H"], cfg["I"], cfg["shared_I"], cfg["type"]
    return q3x.MoeLayer(bf16_matrix(E, H, seed + 11, H ** -0.5, device), routed.gate_up, routed.down,
                        quantized_matrix(t, SI, H, seed + 12, device), quantized_matrix(t, SI, H, seed + 13, device),
                        quantized_matrix(t, H, SI, seed + 14, device), bf16_matrix(1, H, seed + 15, 0.02, device),
                        t, E, cfg["top_k"], H, I, SI)


def router_logits(index: int, tokens: int, experts: int, device="cuda"):
    return normal((tokens, experts), (SEED_BASE + index) * 1000 + 700 + tokens, 1.0, device)


# ------------------------------------------------------------ whole models

MODEL_HEADER = "Q3XMODL\0".encode()


def model_header(model_id: int, fields) -> bytes:
    """The 72-byte model.bin header of a fixed model: magic + 16 uint32
    fields (id, V, H, I, N, AI, AH, KVH, AD, RD, KH, VH, KD, VD, CK, 262144)."""
    import struct
    return struct.pack("<8s16I", MODEL_HEADER, *fields)


def synthetic_model_weights(model_id: int, seed: int, device="cuda"):
    """(ModelConfig, uint8 device tensor) of a full-size model whose weights
    are drawn on the GPU in model.bin layout: matrices N(0, 1/sqrt(cols))
    (the embedding N(0, 1)) quantised by q3x_hip_quantize, BF16 norm and conv
    vectors N(0, 0.1)/N(0, 0.5), FP32 A_log -1 + N(0, 0.2) and norm
    1 + N(0, 0.2), router and shared-expert gate N(0, 1/sqrt(H)).  The
    header is written too, so the buffer is a valid model.bin image."""
    torch = _torch()
    sizes = {
        9000: (248320, 4096, 12288, 32, 4, 16, 4, 256, 64, 16, 32, 128, 128, 4),
        36035: (248320, 2048, 512, 40, 4, 16, 2, 256, 64, 16, 32, 128, 128, 4),
        38027: (248320, 5120, 17408, 64, 4, 24, 4, 256, 64, 16, 48, 128, 128, 4),
    }[model_id]
    header = model_header(model_id, (model_id,) + sizes + (262144,))
    # The file size: the schema of the configuration the header names.
    probe = q3x.make_config(id=model_id, V=sizes[0], H=sizes[1], I=sizes[2], N=sizes[3], AI=sizes[4],
                            AH=sizes[5], KVH=sizes[6], AD=sizes[7], RD=sizes[8], KH=sizes[9], VH=sizes[10],
                            KD=sizes[11], VD=sizes[12], CK=sizes[13], experts=256 if model_id == 36035 else 0,
                            top_k=8 if model_id == 36035 else 0, shared_I=512 if model_id == 36035 else 0,
                            matrix_type=q3x.MATRIX_Q8_0 if model_id == 9000 else q3x.MATRIX_Q4_0)
    _, nbytes = q3x.model_schema(probe)
    config, tensors = q3x.model_layout(header, nbytes)
    buf = torch.zeros(nbytes, dtype=torch.uint8, device=device)
    buf[:len(header)] = torch.frombuffer(bytearray(header), dtype=torch.uint8).to(device)
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    H = config.H
    chunk = 1 << 26  # elements per generated piece
    for t in tensors:
        role = q3x.TENSOR_ROLES[t.role]
        out = buf[t.offset:t.offset + t.bytes]
        rows = max(t.experts, 1) * t.rows
        if t.type in (q3x.MATRIX_Q8_0, q3x.MATRIX_Q4_0):
            std = 1.0 if role in ("embedding", "lm_head") else 1.0 / t.cols ** 0.5
            row_bytes = t.bytes // rows
            step = max(1, chunk // t.cols)
            for r0 in range(0, rows, step):
                n = min(step, rows - r0)
                src = torch.randn((n, t.cols), generator=g, device=device, dtype=torch.float32).mul_(std)
                q3x.quantize(t.type, src, n, t.cols, out[r0 * row_bytes:(r0 + n) * row_bytes])
        elif t.type == q3x.TENSOR_F32:
            base = -1.0 if role == "delta_alog" else 1.0
            vals = torch.randn(rows * t.cols, generator=g, device=device, dtype=torch.float32).mul_(0.2).add_(base)
            out.copy_(vals.view(torch.uint8))
        else:
            std = {"moe_router": H ** -0.5, "moe_shared_scale": H ** -0.5, "delta_conv": 0.5,
                   "delta_dt": 0.5}.get(role, 0.1)
            vals = torch.randn(rows * t.cols, generator=g, device=device, dtype=torch.float32).mul_(std)
            out.copy_((vals.view(torch.int32) >> 16).to(torch.int16).view(torch.uint8))
    torch.cuda.synchronize()
    return config, buf
