"""GPU parity of the whole MoE layer (q3x_hip_moe_layer) against the oracle's
restatement of engine.cpp:406-430, which tests/test_oracle_vs_reference.py
pins bit for bit to the reference's own moe()."""
import numpy as np
import pytest

import oracle
import qwen3x_amd as q3x
from tests.helpers import BLOCK_BYTES, Q4_0, Q8_0, dequant_numpy, random_blocks
from tests.test_gpu_parity import TOL, _torch, dev, host, moe_bound, say

pytestmark = pytest.mark.gpu


def bf16(rng, rows, cols, scale):
    return (rng.normal(0, scale, (rows, cols)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)


def devb(a):
    """A device copy of any array; BF16 (uint16) goes as int16, the same bytes."""
    return dev(a.view(np.int16) if a.dtype == np.uint16 else a)


def bf16_values(a):
    return (a.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def silu_parts(G, U, X):
    """h = silu(G x) * (U x) in double and the first-order bound of h's error
    from TOL-bounded errors of the two products (as in moe_bound)."""
    xn = np.linalg.norm(X, axis=1)
    g, u = X @ G.T, X @ U.T
    sig = 1 / (1 + np.exp(-g))
    h = g * sig * u
    dg = TOL * np.linalg.norm(G, axis=1)[None, :] * xn[:, None]
    du = TOL * np.linalg.norm(U, axis=1)[None, :] * xn[:, None]
    dh = np.abs(sig * (1 + g * (1 - sig)) * u) * dg + np.abs(g * sig) * du + 1e-6 * np.abs(h)
    return h, TOL * np.linalg.norm(h, axis=1) + np.linalg.norm(dh, axis=1)


def layer_bound(w, type_, E, H, I, SI, X, ids, wts):
    """Per-element bound of |GPU - oracle| for the layer."""
    Xd = X.astype(np.float64)
    xn = np.linalg.norm(Xd, axis=1)
    routed = moe_bound(w["gate_up"], w["down"], type_, E, H, I, X, ids, wts)
    # Router logits within TOL*||row||*||x||: softmax and renormalisation move
    # each weight by at most 4x that, relative.
    rn = np.linalg.norm(bf16_values(w["router"]), axis=1).max()
    rel = 4 * TOL * rn * xn                                           # [T]
    gdq = dequant_numpy(w["gate_up"], type_, E * 2 * I, H).reshape(E, 2 * I, H).astype(np.float64)
    ddq = dequant_numpy(w["down"], type_, E * H, I).reshape(E, H, I).astype(np.float64)
    weight_term = np.zeros((X.shape[0], H))
    for t in range(X.shape[0]):
        for s, e in enumerate(ids[t]):
            h, _ = silu_parts(gdq[e, :I], gdq[e, I:], Xd[t:t + 1])
            weight_term[t] += abs(wts[t, s]) * np.abs(h[0] @ ddq[e].T)
    weight_term *= rel[:, None]
    # Shared expert, scaled by s = sigmoid(gate logit), whose own error moves s
    # by at most s(1-s) * TOL * ||row|| * ||x||.
    G = dequant_numpy(w["shared_gate"], type_, SI, H).astype(np.float64)
    U = dequant_numpy(w["shared_up"], type_, SI, H).astype(np.float64)
    D = dequant_numpy(w["shared_down"], type_, H, SI).astype(np.float64)
    h, coef = silu_parts(G, U, Xd)
    out = h @ D.T
    row = bf16_values(w["shared_scale"])[0]
    z = Xd @ row
    s = 1 / (1 + np.exp(-z))
    ds = s * (1 - s) * TOL * np.linalg.norm(row) * xn
    shared = s[:, None] * coef[:, None] * np.linalg.norm(D, axis=1)[None, :] + ds[:, None] * np.abs(out)
    return routed + weight_term + shared


def logit_error(router, x):
    """Bound of |GPU logit - oracle logit| relative to 1: TOL * ||row|| * ||x||."""
    return TOL * np.linalg.norm(bf16_values(router), axis=1).max() * np.linalg.norm(x.astype(np.float64))


def near_tie(router, x, k, a, b):
    """Experts a and b may trade places when their probabilities lie within
    the logits' own error of each other."""
    logits = oracle.mv_bf16(router, x)
    _, _, probs = oracle.router_top_k(logits, k)
    p = probs[0]
    top = max(p[a], p[b])
    return abs(p[a] - p[b]) <= 2 * top * logit_error(router, x) + 4 * np.spacing(np.float32(top))


CASES = [
    # type, experts, H, I, shared_I, top_k, tokens
    (Q8_0, 8, 512, 256, 256, 2, 1),      # fused decode: routed slots + shared slot
    (Q8_0, 8, 512, 256, 256, 2, 70),     # prefill: grouped GEMMs + paired shared GEMM
    (Q4_0, 64, 2048, 512, 512, 8, 1),    # 35B-A3B-like decode
    (Q4_0, 64, 2048, 512, 512, 8, 40),
    (Q4_0, 32, 2048, 512, 256, 8, 1),    # shared expert narrower than the routed ones (fused decode)
    (Q4_0, 16, 256, 64, 64, 4, 1),       # unaligned down rows: decode through the grouped path
    (Q8_0, 16, 256, 256, 32, 4, 1),      # shared_I % 64 != 0: two strided GEMMs + SwiGLU
    (Q8_0, 16, 256, 256, 32, 4, 9),
    (Q4_0, 8, 512, 128, 128, 4, 160),    # 80 pairs per expert: whole 80-pair grouped tiles
    (Q4_0, 32, 2048, 512, 256, 8, 40),   # prefill, shared expert narrower: its paired GEMM, K split
]


@pytest.mark.parametrize("type_,E,H,I,SI,k,tokens", CASES)
def test_moe_layer_parity(type_, E, H, I, SI, k, tokens):
    torch = _torch()
    rng = np.random.default_rng(E * 7 + H + I + SI + tokens)
    w = dict(router=bf16(rng, E, H, 0.5), shared_scale=bf16(rng, 1, H, 0.05),
             gate_up=random_blocks(rng, type_, E * 2 * I, H), down=random_blocks(rng, type_, E * H, I),
             shared_gate=random_blocks(rng, type_, SI, H), shared_up=random_blocks(rng, type_, SI, H),
             shared_down=random_blocks(rng, type_, H, SI))
    X = rng.normal(0, 1, (tokens, H)).astype(np.float32)
    want, ids_o, wts_o = oracle.moe_layer(w["router"], w["gate_up"], w["down"], w["shared_gate"], w["shared_up"],
                                          w["shared_down"], w["shared_scale"], type_, E, H, I, SI, k, X)
    layer = q3x.MoeLayer(devb(w["router"]), devb(w["gate_up"]), devb(w["down"]), devb(w["shared_gate"]),
                         devb(w["shared_up"]), devb(w["shared_down"]), devb(w["shared_scale"]), type_, E, k, H, I, SI)
    say(f"moe_layer type={type_} E={E} H={H} I={I} SI={SI} k={k} tokens={tokens}")
    got, ids_g, wts_g, logits_g = run_layer(layer, X, tokens, k)
    check_layer(w, type_, E, H, I, SI, k, X, got, ids_g, wts_g, want, ids_o, wts_o, logits_g)


def run_layer(layer, X, tokens, k):
    """q3x_hip_moe_layer on host X; returns Y, ids, weights and the router
    logits the routing was computed from (the workspace begins with them)."""
    torch = _torch()
    E = layer.experts
    Y = torch.full((tokens, layer.H), float("nan"), dtype=torch.float32, device="cuda:0")
    ids = torch.full((tokens, k), -7, dtype=torch.int32, device="cuda:0")
    wts = torch.zeros((tokens, k), dtype=torch.float32, device="cuda:0")
    ws = torch.empty(q3x.moe_layer_workspace_bytes(layer, tokens), dtype=torch.uint8, device="cuda:0")
    q3x.moe_layer(layer, dev(X), tokens, Y, ids, wts, workspace=ws)
    torch.cuda.synchronize()
    logits = host(ws[:tokens * E * 4]).view(np.float32).reshape(tokens, E)
    return host(Y), host(ids), host(wts), logits.copy()


def check_layer(w, type_, E, H, I, SI, k, X, got, ids_g, wts_g, want, ids_o, wts_o, logits_g):
    """GPU layer output against the oracle's.  The routing is pinned exactly:
    ids and weights equal the reference's router (oracle.router_top_k,
    engine.cpp:377-405) applied to the GPU's own logits, bit for bit, and
    those logits lie within the BF16 dot's bound of the oracle's.  Where the
    two sets of logits order a near tie differently (a swap the logits' own
    error allows), the output is checked against the oracle's layer with the
    GPU's routing put in; every token's output is checked.  The bound only
    needs the selected experts, so their blocks are gathered first (full
    pools can be large)."""
    tokens = X.shape[0]
    assert np.all(np.isfinite(got))
    ids_r, wts_r, _ = oracle.router_top_k(logits_g, k)
    assert np.array_equal(ids_g, ids_r)
    assert np.array_equal(wts_g.view(np.uint32), wts_r.view(np.uint32))
    for t in range(tokens):
        lo = oracle.mv_bf16(w["router"], X[t])
        assert np.all(np.abs(logits_g[t].astype(np.float64) - lo) <= logit_error(w["router"], X[t])), t
    sel = np.unique(np.concatenate([ids_o.reshape(-1), ids_g.reshape(-1)]))
    bb = BLOCK_BYTES[type_]
    gsz, dsz = 2 * I * H // 32 * bb, H * I // 32 * bb
    ws = dict(w, gate_up=np.concatenate([w["gate_up"][e * gsz:(e + 1) * gsz] for e in sel]),
              down=np.concatenate([w["down"][e * dsz:(e + 1) * dsz] for e in sel]))
    bound_o = layer_bound(ws, type_, len(sel), H, I, SI, X, np.searchsorted(sel, ids_o), wts_o)
    bound_g = layer_bound(ws, type_, len(sel), H, I, SI, X, np.searchsorted(sel, ids_g), wts_g)
    swapped = 0
    for t in range(tokens):
        if np.array_equal(ids_g[t], ids_o[t]):
            assert np.allclose(wts_g[t], wts_o[t], rtol=4 * logit_error(w["router"], X[t]), atol=0), t
            expect, bound = want[t], bound_o[t]
        else:
            for a, b in zip(ids_g[t], ids_o[t]):
                if a != b:
                    assert near_tie(w["router"], X[t], k, a, b), (t, a, b)
            swapped += 1
            # The oracle's layer with the GPU's routing: its routed sum
            # replaced, the shared expert's part kept.
            routed_o = oracle.moe_routed(w["gate_up"], w["down"], type_, E, H, I, X[t:t + 1], ids_o[t:t + 1],
                                         wts_o[t:t + 1])[0].astype(np.float64)
            routed_g = oracle.moe_routed(w["gate_up"], w["down"], type_, E, H, I, X[t:t + 1], ids_g[t:t + 1],
                                         wts_g[t:t + 1])[0].astype(np.float64)
            expect = want[t].astype(np.float64) - routed_o + routed_g
            bound = bound_g[t] + 2 * np.spacing(np.abs(want[t]).astype(np.float32)).astype(np.float64)
        diff = np.abs(got[t].astype(np.float64) - expect)
        assert np.all(diff <= bound), f"token {t}: {(diff > bound).sum()} outside; worst {diff.max()}"
    assert swapped <= max(1, tokens // 8)


def test_moe_layer_without_routing_outputs_matches_with_them():
    # ids / weights NULL: the routing lives in the workspace; same result bits.
    torch = _torch()
    type_, E, H, I, SI, k = Q4_0, 16, 2048, 512, 512, 8
    rng = np.random.default_rng(5)
    w = [bf16(rng, E, H, 0.5), random_blocks(rng, type_, E * 2 * I, H), random_blocks(rng, type_, E * H, I),
         random_blocks(rng, type_, SI, H), random_blocks(rng, type_, SI, H), random_blocks(rng, type_, H, SI),
         bf16(rng, 1, H, 0.05)]
    layer = q3x.MoeLayer(*(devb(a) for a in w), type_, E, k, H, I, SI)
    for tokens in (1, 5):
        X = dev(rng.normal(0, 1, (tokens, H)).astype(np.float32))
        Y1 = torch.empty((tokens, H), dtype=torch.float32, device="cuda:0")
        Y2 = torch.empty_like(Y1)
        ids = torch.empty((tokens, k), dtype=torch.int32, device="cuda:0")
        wts = torch.empty((tokens, k), dtype=torch.float32, device="cuda:0")
        say(f"moe_layer outputs tokens={tokens}")
        q3x.moe_layer(layer, X, tokens, Y1, ids, wts)
        q3x.moe_layer(layer, X, tokens, Y2)
        assert torch.equal(Y1.view(torch.int32), Y2.view(torch.int32))
