"""Writes the golden fixtures of tests/golden/ from the reference's own CPU
code (oracle/_ref/libq3x_ref.so, compiled from the reference sources where
they lie by `make -C oracle ref`).

Each .npz holds seeded inputs and the reference's outputs for them:
  mv_q8_0.npz, mv_q4_0.npz   arch/cpu.cpp try_mv / try_embed (matvec + rows)
  router.npz                 engine.cpp router_top_k
  silu.npz                   engine.cpp sigmoid / silu
  moe_q4_0.npz               engine.cpp moe() with a BF16 router and a zero
                             shared expert (routed experts only)
  moe_layer_q8_0.npz         engine.cpp moe() with every weight real (BF16
                             router and shared-expert gate, Q8_0 experts and
                             shared expert) and the BF16 mv() of the router
Run: python tests/golden/make_golden.py [fixture ...]   (needs the reference
build; with names, only those fixtures are written)
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402
from tests.helpers import Q4_0, Q8_0, random_blocks  # noqa: E402

SPECIAL = np.array([0x3555, 0x2E66, 0x0400, 0x0001, 0x8001, 0x7BFF, 0x0000, 0x8000, 0x3C00, 0xB800], np.uint16)


def p(a):
    return a.ctypes.data


def mv_fixture(ref, type_, name):
    rng = np.random.default_rng(20261201 + type_)
    out = {}
    for i, (rows, cols, special) in enumerate([(3, 64, True), (17, 96, False), (8, 256, True), (5, 2048, False)]):
        w = random_blocks(rng, type_, rows, cols, SPECIAL if special else None)
        x = rng.normal(0, 1, cols).astype(np.float32)
        y = np.empty(rows, np.float32)
        assert ref.q3xr_try_mv(p(w), type_, rows, cols, p(x), p(y)) == 1
        emb = np.empty((rows, cols), np.float32)
        for r in range(rows):
            assert ref.q3xr_try_embed(p(w), type_, cols, r, p(emb[r])) == 1
        out[f"w{i}"], out[f"x{i}"], out[f"y{i}"], out[f"embed{i}"] = w, x, y, emb
        out[f"shape{i}"] = np.array([rows, cols], np.int64)
    np.savez_compressed(os.path.join(HERE, name), **out)


def router_fixture(ref):
    rng = np.random.default_rng(20261210)
    cases = [(256, 8), (6, 3), (64, 1), (256, 2)]
    out = {}
    for i, (E, k) in enumerate(cases):
        logits = rng.normal(0, 1 + i, (16, E)).astype(np.float32)
        logits[3, :4] = logits[3].max()  # exact ties
        ids = np.empty((16, k), np.int32)
        wts = np.empty((16, k), np.float32)
        for t in range(16):
            probs = np.empty(E, np.float32)
            ref.q3xr_router_top_k(p(logits[t]), E, k, p(ids[t]), p(probs))
            wts[t] = probs[ids[t]]
        out[f"logits{i}"], out[f"ids{i}"], out[f"weights{i}"] = logits, ids, wts
    np.savez_compressed(os.path.join(HERE, "router.npz"), **out)


def silu_fixture(ref):
    rng = np.random.default_rng(20261211)
    x = np.concatenate([rng.normal(0, 8, 500), [0.0, -0.0, 88.0, -88.0, 20.0, -20.0, 1e-30]]).astype(np.float32)
    sig = np.array([ref.q3xr_sigmoid(float(v)) for v in x], np.float32)
    silu = np.array([ref.q3xr_silu(float(v)) for v in x], np.float32)
    np.savez_compressed(os.path.join(HERE, "silu.npz"), x=x, sigmoid=sig, silu=silu)


def moe_fixture(ref):
    rng = np.random.default_rng(20261212)
    E, H, I, k = 8, 64, 32, 2
    router = (rng.normal(0, 0.5, (E, H)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    gate_up = random_blocks(rng, Q4_0, E * 2 * I, H)
    down = random_blocks(rng, Q4_0, E * H, I)
    X = rng.normal(0, 1, (4, H)).astype(np.float32)
    logits = np.empty((4, E), np.float32)
    ids = np.empty((4, k), np.int32)
    Y = np.empty((4, H), np.float32)
    for t in range(4):
        ref.q3xr_moe_q4(p(router), p(gate_up), p(down), E, H, I, k, p(X[t]), p(logits[t]), p(ids[t]), p(Y[t]))
    np.savez_compressed(os.path.join(HERE, "moe_q4_0.npz"), router=router, gate_up=gate_up, down=down, X=X,
                        logits=logits, ids=ids, Y=Y, shape=np.array([E, H, I, k], np.int64))


def moe_layer_fixture(ref):
    rng = np.random.default_rng(20261213)
    E, H, I, SI, k, T = 8, 64, 64, 32, 3, 4
    bf16 = lambda rows, cols, s: (rng.normal(0, s, (rows, cols)).astype(np.float32).view(np.uint32)  # noqa: E731
                                  >> 16).astype(np.uint16)
    router = bf16(E, H, 0.5)
    scale = bf16(1, H, 0.05)
    gate_up = random_blocks(rng, Q8_0, E * 2 * I, H)
    down = random_blocks(rng, Q8_0, E * H, I)
    sg = random_blocks(rng, Q8_0, SI, H)
    su = random_blocks(rng, Q8_0, SI, H)
    sd = random_blocks(rng, Q8_0, H, SI)
    X = rng.normal(0, 1, (T, H)).astype(np.float32)
    logits = np.empty((T, E), np.float32)
    ids = np.empty((T, k), np.int32)
    Y = np.empty((T, H), np.float32)
    for t in range(T):
        ref.q3xr_mv_bf16(p(router), E, H, p(X[t]), p(logits[t]))
        ref.q3xr_moe_layer(Q8_0, p(router), p(gate_up), p(down), p(sg), p(su), p(sd), p(scale), E, H, I, SI, k,
                           p(X[t]), p(Y[t]), p(ids[t]))
    np.savez_compressed(os.path.join(HERE, "moe_layer_q8_0.npz"), router=router, shared_scale=scale,
                        gate_up=gate_up, down=down, shared_gate=sg, shared_up=su, shared_down=sd, X=X,
                        logits=logits, ids=ids, Y=Y, shape=np.array([E, H, I, SI, k], np.int64))


FIXTURES = {
    "mv_q8_0": lambda ref: mv_fixture(ref, Q8_0, "mv_q8_0.npz"),
    "mv_q4_0": lambda ref: mv_fixture(ref, Q4_0, "mv_q4_0.npz"),
    "router": router_fixture,
    "silu": silu_fixture,
    "moe_q4_0": moe_fixture,
    "moe_layer_q8_0": moe_layer_fixture,
}


def main():
    ref = oracle.ref()
    if ref is None:
        raise SystemExit("oracle/_ref/libq3x_ref.so is missing: run `make -C oracle ref` first")
    for name in sys.argv[1:] or FIXTURES:
        FIXTURES[name](ref)
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
