"""Writes tests/golden/quantizer.npz: input/output vectors of the reference
packer's quantizers (scripts/pack_weights.py quantize_q8_0 / quantize_q4_0),
imported from the reference tree in the container that has it.

The Q4_0 quantizer is also pinned by the published SHA-256 of llama.cpp's
reference quantizer output (tests/q4_llama_reference.py in the reference); the
Q8_0 quantizer has no published digest, so these vectors pin it.  Only data is
kept: BF16 input bits and the packed output bytes.
Run: python tests/golden/make_quantizer_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REFERENCE_SCRIPTS = "/root/reference/scripts"


def bf16_bits(values):
    return (np.asarray(values, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def inputs():
    rng = np.random.default_rng(20261213)
    blocks = [rng.normal(0, 0.02, 32 * 512), rng.normal(0, 1.0, 32 * 256), rng.standard_cauchy(32 * 128)]
    edge = np.zeros(32 * 8, np.float32)
    edge[32:38] = [127.0, -127.0, 126.5, -126.5, 0.5, -0.5]       # test_pack_weights.py:205-206
    edge[64:96] = np.linspace(-8, 7.5, 32)
    edge[96:128] = np.linspace(8, -7.5, 32)
    edge[128:160] = 1e-30
    edge[160:192] = -3.0e38
    edge[192:224] = [0.25 * (i - 16) for i in range(32)]
    edge[224:256] = np.float32(2.0) ** np.arange(-16, 16)
    values = np.concatenate([b.astype(np.float32) for b in blocks] + [edge])
    values = np.clip(values, -3.0e38, 3.0e38)
    return bf16_bits(values)


def main():
    if not os.path.isdir(REFERENCE_SCRIPTS):
        raise SystemExit("the reference tree is not present")
    sys.path.insert(0, REFERENCE_SCRIPTS)
    import pack_weights  # the reference packer

    bits = inputs()
    q8 = np.frombuffer(pack_weights.quantize_q8_0(bits.tobytes()), np.uint8)
    q4 = np.frombuffer(pack_weights.quantize_q4_0(bits.tobytes()), np.uint8)
    np.savez_compressed(os.path.join(HERE, "quantizer.npz"), bf16=bits, q8_0=q8, q4_0=q4)
    print("quantizer fixture:", bits.size // 32, "blocks")


if __name__ == "__main__":
    main()
