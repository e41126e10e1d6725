"""model.bin layout as the reference's PACKER writes it -- TEST INFRASTRUCTURE ONLY.

A plain-Python restatement of scripts/pack_weights.py's supported-model table
(:42-109), header (:21-22, 199-209), tensor schema (:212-283) and storage
walk (:171-196): the writer's side of the format, independent of the loader
(engine.cpp:481-559) that the library mirrors.  The tests check this
restatement against the reference's known file sizes (tests/q8_cpu_test.cpp:
228, tests/q4_cpu_test.cpp:15) and against the reference's own loader run on
sparse files, then hold the library's layout to it.
"""
from __future__ import annotations

import struct

ALIGNMENT = 64
MAGIC = b"Q3XMODL\0"
HEADER = struct.Struct("<8s16I")
MAX_CONTEXT = 262144

# Roles in the order of the library's tensor-role enumeration.
ROLES = ("embedding", "lm_head", "final_norm", "input_norm", "post_norm",
         "delta_qkv", "delta_z", "delta_a", "delta_b", "delta_conv", "delta_alog", "delta_dt", "delta_norm",
         "delta_out", "attn_q", "attn_k", "attn_v", "attn_qnorm", "attn_knorm", "attn_out",
         "ffn_gate", "ffn_up", "ffn_down", "moe_router", "moe_gate_up", "moe_down", "moe_shared_gate",
         "moe_shared_up", "moe_shared_down", "moe_shared_scale")

# pack_weights.py:42-109 (model ID -> shapes); keys as the packer's.
MODELS = {
    800: dict(name="Qwen3.5-0.8B", vocab=248320, hidden=1024, intermediate=3584, layers=24, interval=4,
              heads=8, kv_heads=2, head_dim=256, rotary_dim=64, key_heads=16, value_heads=16, key_dim=128,
              value_dim=128, conv=4, experts=0, top_k=0, shared=0, matrix="BF16", tied=True),
    4000: dict(name="Qwen3.5-4B", vocab=248320, hidden=2560, intermediate=9216, layers=32, interval=4,
               heads=16, kv_heads=4, head_dim=256, rotary_dim=64, key_heads=16, value_heads=32, key_dim=128,
               value_dim=128, conv=4, experts=0, top_k=0, shared=0, matrix="BF16", tied=True),
    9000: dict(name="Qwen3.5-9B", vocab=248320, hidden=4096, intermediate=12288, layers=32, interval=4,
               heads=16, kv_heads=4, head_dim=256, rotary_dim=64, key_heads=16, value_heads=32, key_dim=128,
               value_dim=128, conv=4, experts=0, top_k=0, shared=0, matrix="Q8_0", tied=False),
    36035: dict(name="Qwen3.6-35B-A3B", vocab=248320, hidden=2048, intermediate=512, layers=40, interval=4,
                heads=16, kv_heads=2, head_dim=256, rotary_dim=64, key_heads=16, value_heads=32, key_dim=128,
                value_dim=128, conv=4, experts=256, top_k=8, shared=512, matrix="Q4_0", tied=False),
    38027: dict(name="Qwen3.8-27B", vocab=248320, hidden=5120, intermediate=17408, layers=64, interval=4,
                heads=24, kv_heads=4, head_dim=256, rotary_dim=64, key_heads=16, value_heads=48, key_dim=128,
                value_dim=128, conv=4, experts=0, top_k=0, shared=0, matrix="Q4_0", tied=False),
}
MATRIX_TYPE = {"BF16": 0, "Q8_0": 1, "Q4_0": 2}
F32 = 3


def header_fields(model_id: int):
    """pack_weights.py:199-209: the 16 uint32 fields in ConfigField order."""
    m = MODELS[model_id]
    return (model_id, m["vocab"], m["hidden"], m["intermediate"], m["layers"], m["interval"], m["heads"],
            m["kv_heads"], m["head_dim"], m["rotary_dim"], m["key_heads"], m["value_heads"], m["key_dim"],
            m["value_dim"], m["conv"], MAX_CONTEXT)


def header(model_id: int) -> bytes:
    return HEADER.pack(MAGIC, *header_fields(model_id))


def tensors(model_id: int):
    """pack_weights.py:212-283: (role, layer, dtype, shape, matrix) in file order."""
    m = MODELS[model_id]
    H, I, V = m["hidden"], m["intermediate"], m["vocab"]
    dqkv = 2 * m["key_heads"] * m["key_dim"] + m["value_heads"] * m["value_dim"]
    do = m["value_heads"] * m["value_dim"]
    AS, KVW = m["heads"] * m["head_dim"], m["kv_heads"] * m["head_dim"]
    out = [("embedding", -1, "BF16", (V, H), True)]
    if not m["tied"]:
        out.append(("lm_head", -1, "BF16", (V, H), True))
    out.append(("final_norm", -1, "BF16", (H,), False))
    for layer in range(m["layers"]):
        out.append(("input_norm", layer, "BF16", (H,), False))
        if layer % m["interval"] != m["interval"] - 1:
            out += [("delta_qkv", layer, "BF16", (dqkv, H), True),
                    ("delta_z", layer, "BF16", (do, H), True),
                    ("delta_a", layer, "BF16", (m["value_heads"], H), True),
                    ("delta_b", layer, "BF16", (m["value_heads"], H), True),
                    ("delta_conv", layer, "BF16", (dqkv, 1, m["conv"]), False),
                    ("delta_alog", layer, "F32", (m["value_heads"],), False),
                    ("delta_dt", layer, "BF16", (m["value_heads"],), False),
                    ("delta_norm", layer, "F32", (m["value_dim"],), False),
                    ("delta_out", layer, "BF16", (H, do), True)]
        else:
            out += [("attn_q", layer, "BF16", (2 * AS, H), True),
                    ("attn_k", layer, "BF16", (KVW, H), True),
                    ("attn_v", layer, "BF16", (KVW, H), True),
                    ("attn_qnorm", layer, "BF16", (m["head_dim"],), False),
                    ("attn_knorm", layer, "BF16", (m["head_dim"],), False),
                    ("attn_out", layer, "BF16", (H, AS), True)]
        out.append(("post_norm", layer, "BF16", (H,), False))
        if m["experts"]:
            E, S = m["experts"], m["shared"]
            out += [("moe_router", layer, "BF16", (E, H), False),
                    ("moe_gate_up", layer, "BF16", (E, 2 * I, H), True),
                    ("moe_down", layer, "BF16", (E, H, I), True),
                    ("moe_shared_gate", layer, "BF16", (S, H), True),
                    ("moe_shared_up", layer, "BF16", (S, H), True),
                    ("moe_shared_down", layer, "BF16", (H, S), True),
                    ("moe_shared_scale", layer, "BF16", (1, H), False)]
        else:
            out += [("ffn_gate", layer, "BF16", (I, H), True),
                    ("ffn_up", layer, "BF16", (I, H), True),
                    ("ffn_down", layer, "BF16", (H, I), True)]
    return out


def layout(model_id: int):
    """pack_weights.py:171-196: per tensor (role, layer, stored type, offset,
    bytes), and the file size.  Matrices take the model's matrix type."""
    m = MODELS[model_id]
    cursor = HEADER.size
    rows = []
    for role, layer, dtype, shape, matrix in tensors(model_id):
        cursor += (-cursor) % ALIGNMENT
        count = 1
        for d in shape:
            count *= d
        if matrix and m["matrix"] == "Q8_0":
            stored, nbytes = 1, count // 32 * 34
        elif matrix and m["matrix"] == "Q4_0":
            stored, nbytes = 2, count // 32 * 18
        else:
            stored, nbytes = (0, count * 2) if dtype == "BF16" else (F32, count * 4)
        rows.append((role, layer, stored, cursor, nbytes))
        cursor += nbytes
    return rows, cursor
