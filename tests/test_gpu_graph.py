"""HIP graph capture of the backend's launches: a decode step (projections,
accumulating matvecs, lm_head-style matvec) and a routed-MoE decode are
captured once and replayed several times, with eager work between replays
(and the whole MoE layer, decode and prefill);
every replay must equal the eager result bit for bit (the kernels are
deterministic and record no memset nodes)."""
import numpy as np
import pytest

import qwen3x_amd as q3x
from tests.helpers import Q4_0, Q8_0, random_blocks

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    assert torch.cuda.is_available(), "GPU tests need cuda:0"
    return torch


def dev(a):
    return _torch().from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def replay_matches_eager(torch, fn, outputs, reset, times=3):
    reset()
    fn()
    torch.cuda.synchronize()
    want = [o.clone() for o in outputs]
    g = torch.cuda.CUDAGraph()
    reset()
    with torch.cuda.graph(g):
        fn()
    for _ in range(times):
        reset()
        g.replay()
        torch.cuda.synchronize()
        for o, w in zip(outputs, want):
            assert torch.equal(o.view(torch.int32), w.view(torch.int32)), "graph replay differs from eager"
        reset()
        fn()  # eager work between replays
        torch.cuda.synchronize()


def test_decode_step_graph_replays_bitwise():
    torch = _torch()
    rng = np.random.default_rng(5)
    h, f = 1024, 3072
    mats = {n: q3x.Linear(dev(random_blocks(rng, Q8_0, r, c)), r, c, Q8_0)
            for n, r, c in [("q", h, h), ("k", 256, h), ("v", 256, h), ("o", h, h), ("gate", f, h), ("up", f, h),
                            ("down", h, f), ("lm", 5000, h)]}
    x = dev(rng.normal(0, 1, h).astype(np.float32))
    hid = dev(rng.normal(0, 1, f).astype(np.float32))
    resid0 = dev(rng.normal(0, 1, h).astype(np.float32))
    resid = resid0.clone()
    outs = {n: torch.full((m.rows,), float("nan"), dtype=torch.float32, device="cuda:0") for n, m in mats.items()
            if n not in ("o", "down")}

    def step():
        q3x.mv_multi([mats["q"], mats["k"], mats["v"]], x, [outs["q"], outs["k"], outs["v"]])
        q3x.mv_add(mats["o"], x, resid)
        q3x.mv_multi([mats["gate"], mats["up"]], x, [outs["gate"], outs["up"]])
        q3x.mv_add(mats["down"], hid, resid)
        q3x.mv(mats["lm"], x, outs["lm"])

    replay_matches_eager(torch, step, [resid] + list(outs.values()), lambda: resid.copy_(resid0))


def test_moe_decode_graph_replays_bitwise():
    torch = _torch()
    rng = np.random.default_rng(6)
    E, H, I, k = 16, 512, 128, 4
    gu = q3x.ExpertLinear(dev(random_blocks(rng, Q4_0, E * 2 * I, H)), E, 2 * I, H, Q4_0)
    dn = q3x.ExpertLinear(dev(random_blocks(rng, Q4_0, E * H, I)), E, H, I, Q4_0)
    logits = dev(rng.normal(0, 1, (1, E)).astype(np.float32))
    X = dev(rng.normal(0, 1, (1, H)).astype(np.float32))
    ids = torch.empty((1, k), dtype=torch.int32, device="cuda:0")
    wts = torch.empty((1, k), dtype=torch.float32, device="cuda:0")
    Y = torch.empty((1, H), dtype=torch.float32, device="cuda:0")
    ws = torch.empty(q3x.moe_workspace_bytes(1, E, k, H, I), dtype=torch.uint8, device="cuda:0")

    def run():
        q3x.router_top_k(logits, 1, E, k, ids, wts)
        q3x.moe_routed(gu, dn, X, 1, ids, wts, k, Y, workspace=ws)

    replay_matches_eager(torch, run, [ids, wts, Y], lambda: Y.fill_(float("nan")))


@pytest.mark.parametrize("tokens", [1, 7])
def test_moe_layer_graph_replays_bitwise(tokens):
    # The whole layer (router GEMV or GEMM, top-k, routed and shared experts).
    torch = _torch()
    rng = np.random.default_rng(7 + tokens)
    E, H, I, SI, k = 16, 512, 256, 256, 4
    bf16 = lambda r, c, s: dev((rng.normal(0, s, (r, c)).astype(np.float32).view(np.uint32) >> 16)  # noqa: E731
                               .astype(np.uint16).view(np.int16))
    layer = q3x.MoeLayer(bf16(E, H, 0.05), dev(random_blocks(rng, Q4_0, E * 2 * I, H)),
                         dev(random_blocks(rng, Q4_0, E * H, I)), dev(random_blocks(rng, Q4_0, SI, H)),
                         dev(random_blocks(rng, Q4_0, SI, H)), dev(random_blocks(rng, Q4_0, H, SI)),
                         bf16(1, H, 0.05), Q4_0, E, k, H, I, SI)
    X = dev(rng.normal(0, 1, (tokens, H)).astype(np.float32))
    ids = torch.empty((tokens, k), dtype=torch.int32, device="cuda:0")
    wts = torch.empty((tokens, k), dtype=torch.float32, device="cuda:0")
    Y = torch.empty((tokens, H), dtype=torch.float32, device="cuda:0")
    ws = torch.empty(q3x.moe_layer_workspace_bytes(layer, tokens), dtype=torch.uint8, device="cuda:0")

    def run():
        q3x.moe_layer(layer, X, tokens, Y, ids, wts, workspace=ws)

    replay_matches_eager(torch, run, [ids, wts, Y], lambda: Y.fill_(float("nan")))
