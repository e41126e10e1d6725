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
