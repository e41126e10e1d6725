"""q3x_hip_moe_routed_logits: router top-k and routed experts in one call.
At one token the gate/up launch routes the token itself; its ids, weights and
output must equal the two calls it replaces (q3x_hip_router_topk, then
q3x_hip_moe_routed) bit for bit, and the ids the oracle's restatement of
engine.cpp:377-405 exactly."""
import numpy as np
import pytest

import oracle
import qwen3x_amd as q3x
from tests.helpers import Q4_0, Q8_0, random_blocks
from tests.test_gpu_parity import _torch, dev, host, moe_bound, say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("type_,E,H,I,k,tokens", [
    (Q4_0, 256, 2048, 512, 8, 1),     # config 4 decode
    (Q4_0, 256, 2048, 512, 8, 33),    # prefill: router kernel, then the grouped GEMMs
    (Q8_0, 8, 512, 256, 2, 1),
    (Q4_0, 600, 256, 256, 4, 1),      # more experts than 256: eight per lane in the router
    (Q4_0, 16, 256, 64, 4, 1),        # unaligned down rows: the grouped path at one token
])
def test_routed_logits_equals_router_then_routed(type_, E, H, I, k, tokens):
    torch = _torch()
    rng = np.random.default_rng(E + H + I + k + tokens)
    gu = dev(random_blocks(rng, type_, E * 2 * I, H))
    dn = dev(random_blocks(rng, type_, E * H, I))
    logits_h = rng.normal(0, 1, (tokens, E)).astype(np.float32)
    logits_h[0, :4] = logits_h[0, 4]      # ties: the lowest expert index wins
    X = dev(rng.normal(0, 1, (tokens, H)).astype(np.float32))
    logits = dev(logits_h)
    gul, dnl = q3x.ExpertLinear(gu, E, 2 * I, H, type_), q3x.ExpertLinear(dn, E, H, I, type_)
    ids0 = torch.empty((tokens, k), dtype=torch.int32, device="cuda:0")
    w0 = torch.empty((tokens, k), dtype=torch.float32, device="cuda:0")
    Y0 = torch.empty((tokens, H), dtype=torch.float32, device="cuda:0")
    say(f"routed_logits type={type_} E={E} H={H} I={I} k={k} tokens={tokens}")
    q3x.router_top_k(logits, tokens, E, k, ids0, w0)
    q3x.moe_routed(gul, dnl, X, tokens, ids0, w0, k, Y0)
    ids1 = torch.full((tokens, k), -5, dtype=torch.int32, device="cuda:0")
    w1 = torch.full((tokens, k), float("nan"), dtype=torch.float32, device="cuda:0")
    Y1 = torch.full((tokens, H), float("nan"), dtype=torch.float32, device="cuda:0")
    q3x.moe_routed_logits(gul, dnl, X, tokens, logits, k, ids1, w1, Y1)
    torch.cuda.synchronize()
    assert np.array_equal(host(ids1), host(ids0))
    assert np.array_equal(host(w1).view(np.uint32), host(w0).view(np.uint32))
    assert np.array_equal(host(Y1).view(np.uint32), host(Y0).view(np.uint32))
    ids_o, w_o, _ = oracle.router_top_k(logits_h, k)
    assert np.array_equal(host(ids1), ids_o)
    assert np.array_equal(host(w1).view(np.uint32), w_o.view(np.uint32))
    # accumulate: Y += the same routed sum
    q3x.moe_routed_logits(gul, dnl, X, tokens, logits, k, ids1, w1, Y1, accumulate=True)
    q3x.moe_routed(gul, dnl, X, tokens, ids0, w0, k, Y0, accumulate=True)
    torch.cuda.synchronize()
    assert np.array_equal(host(Y1).view(np.uint32), host(Y0).view(np.uint32))


def test_routed_logits_config4_against_the_oracle():
    """Config 4 decode over several tokens in turn (different experts each
    call, one workspace): every output within the routed bound of the oracle."""
    torch = _torch()
    type_, E, H, I, k = Q4_0, 256, 2048, 512, 8
    rng = np.random.default_rng(404)
    gu_h, dn_h = random_blocks(rng, type_, E * 2 * I, H), random_blocks(rng, type_, E * H, I)
    gul = q3x.ExpertLinear(dev(gu_h), E, 2 * I, H, type_)
    dnl = q3x.ExpertLinear(dev(dn_h), E, H, I, type_)
    ws = torch.empty(q3x.moe_workspace_bytes(1, E, k, H, I), dtype=torch.uint8, device="cuda:0")
    for t in range(4):
        logits_h = rng.normal(0, 1, (1, E)).astype(np.float32)
        X_h = rng.normal(0, 1, (1, H)).astype(np.float32)
        ids = torch.empty((1, k), dtype=torch.int32, device="cuda:0")
        w = torch.empty((1, k), dtype=torch.float32, device="cuda:0")
        Y = torch.empty((1, H), dtype=torch.float32, device="cuda:0")
        say(f"routed_logits config 4 token {t}")
        q3x.moe_routed_logits(gul, dnl, dev(X_h), 1, dev(logits_h), k, ids, w, Y, workspace=ws)
        torch.cuda.synchronize()
        ids_o, w_o, _ = oracle.router_top_k(logits_h, k)
        assert np.array_equal(host(ids), ids_o)
        want = oracle.moe_routed(gu_h, dn_h, type_, E, H, I, X_h, ids_o, w_o)
        bound = moe_bound(gu_h, dn_h, type_, E, H, I, X_h, ids_o, w_o)
        assert np.all(np.abs(host(Y).astype(np.float64) - want) <= bound)


@pytest.mark.parametrize("case", ["ulp_top", "ulp_boundary", "tie_boundary", "wide"])
def test_routed_logits_decode_near_ties(case):
    """One-token routing inside the gate_up launch with logits one ulp apart
    at the top or at the top-8 boundary (workgroups other than the first
    cannot order those by exp alone and take the full router), exact ties at
    the boundary, and a wide spread (tiny exp values): the ids every
    workgroup used -- seen through the output -- and the ids and weights
    returned equal the two-call path and the oracle."""
    torch = _torch()
    type_, E, H, I, k = Q4_0, 256, 2048, 512, 8
    rng = np.random.default_rng(77)
    gu = dev(random_blocks(rng, type_, E * 2 * I, H))
    dn = dev(random_blocks(rng, type_, E * H, I))
    gul, dnl = q3x.ExpertLinear(gu, E, 2 * I, H, type_), q3x.ExpertLinear(dn, E, H, I, type_)
    lg = rng.normal(0, 1, (1, E)).astype(np.float32)
    order = np.argsort(-lg[0], kind="stable")
    down = np.float32(-np.inf)
    if case == "ulp_top":
        lg[0, order[1]] = np.nextafter(lg[0, order[0]], down)
    elif case == "ulp_boundary":
        lg[0, order[k]] = np.nextafter(lg[0, order[k - 1]], down)
    elif case == "tie_boundary":
        lg[0, order[k]] = lg[0, order[k - 1]]
    else:
        lg *= np.float32(40)
    X = dev(rng.normal(0, 1, (1, H)).astype(np.float32))
    logits = dev(lg)
    ids0 = torch.empty((1, k), dtype=torch.int32, device="cuda:0")
    w0 = torch.empty((1, k), dtype=torch.float32, device="cuda:0")
    Y0 = torch.empty((1, H), dtype=torch.float32, device="cuda:0")
    say(f"routed_logits near ties case={case}")
    q3x.router_top_k(logits, 1, E, k, ids0, w0)
    q3x.moe_routed(gul, dnl, X, 1, ids0, w0, k, Y0)
    ids1 = torch.empty((1, k), dtype=torch.int32, device="cuda:0")
    w1 = torch.empty((1, k), dtype=torch.float32, device="cuda:0")
    Y1 = torch.empty((1, H), dtype=torch.float32, device="cuda:0")
    q3x.moe_routed_logits(gul, dnl, X, 1, logits, k, ids1, w1, Y1)
    torch.cuda.synchronize()
    ids_o, w_o, _ = oracle.router_top_k(lg, k)
    assert np.array_equal(host(ids1), ids_o) and np.array_equal(host(ids0), ids_o)
    assert np.array_equal(host(w1).view(np.uint32), w_o.view(np.uint32))
    assert np.array_equal(host(Y1).view(np.uint32), host(Y0).view(np.uint32))


def _libm_expf():
    import ctypes
    import ctypes.util
    libm = ctypes.CDLL(ctypes.util.find_library("m") or "libm.so.6")
    fn = libm.expf
    fn.restype, fn.argtypes = ctypes.c_float, [ctypes.c_float]
    return lambda v: np.float32(fn(float(v)))


def boundary_tie_logits(E, k, seed0=0, tries=4000):
    """Logits whose e = expf(l - max) tie exactly at positions k-1 and k, with
    an expert of lower index one ulp of e below the tie, such that the
    reference's p = e / total rounds that expert onto the tie and its strict
    '>' scan takes it (engine.cpp:391-398), while ordering by e with the tie
    accepted (the earlier shortcut rule) takes the tied expert.  Searched over
    seeds on the host; the kernel's libm_expf equals the host expf."""
    from tests.test_router_order import by_exp_planted
    expf = _libm_expf()
    for seed in range(seed0, seed0 + tries):
        rng = np.random.default_rng(seed)
        lg = rng.normal(0, 1, E).astype(np.float32)
        mx = lg.max()
        e = np.array([expf(v - mx) for v in lg], np.float32)
        order = np.argsort(-e, kind="stable")
        a, b = sorted(int(i) for i in order[k - 1:k + 1])
        lg[b] = lg[a] = max(lg[a], lg[b])
        cand = [int(i) for i in order[k + 1:] if i < a]
        if not cand or lg[a] == mx:
            continue
        e_a = expf(lg[a] - mx)
        target = np.nextafter(e_a, np.float32(0))
        v = lg[a]
        for _ in range(64):
            v = np.nextafter(v, np.float32(-np.inf))
            if expf(v - mx) < e_a:
                break
        if expf(v - mx) != target:
            continue
        lg[cand[0]] = v
        e = np.array([expf(t - mx) for t in lg], np.float32)
        ids_o, _, _ = oracle.router_top_k(lg[None, :], k)
        old = by_exp_planted(e, k)
        if old is not None and list(ids_o[0]) != old:
            return lg[None, :], seed
    raise AssertionError("no boundary-tie case found")


@pytest.mark.parametrize("type_,E,H,I,k,seed0", [
    (Q4_0, 256, 2048, 512, 8, 0), (Q4_0, 256, 2048, 512, 8, 100), (Q4_0, 256, 2048, 512, 8, 1000),
    (Q8_0, 64, 512, 256, 4, 0), (Q4_0, 8, 256, 128, 2, 0)])
def test_routed_logits_decode_boundary_tie_lower_index(type_, E, H, I, k, seed0):
    """A tie at the top-k boundary with a lower-index expert one ulp below:
    every workgroup of the gate_up launch must route like the reference (the
    ids returned, the weights, and through Y the rows every workgroup used),
    bit for bit against the two-call path and the oracle."""
    torch = _torch()
    lg, seed = boundary_tie_logits(E, k, seed0)
    rng = np.random.default_rng(9000 + seed)
    gu_h = random_blocks(rng, type_, E * 2 * I, H)
    dn_h = random_blocks(rng, type_, E * H, I)
    gul = q3x.ExpertLinear(dev(gu_h), E, 2 * I, H, type_)
    dnl = q3x.ExpertLinear(dev(dn_h), E, H, I, type_)
    X_h = rng.normal(0, 1, (1, H)).astype(np.float32)
    X, logits = dev(X_h), dev(lg)
    say(f"routed_logits boundary tie type={type_} E={E} k={k} seed={seed}")
    ids0 = torch.empty((1, k), dtype=torch.int32, device="cuda:0")
    w0 = torch.empty((1, k), dtype=torch.float32, device="cuda:0")
    Y0 = torch.empty((1, H), dtype=torch.float32, device="cuda:0")
    q3x.router_top_k(logits, 1, E, k, ids0, w0)
    q3x.moe_routed(gul, dnl, X, 1, ids0, w0, k, Y0)
    ids1 = torch.empty((1, k), dtype=torch.int32, device="cuda:0")
    w1 = torch.empty((1, k), dtype=torch.float32, device="cuda:0")
    Y1 = torch.empty((1, H), dtype=torch.float32, device="cuda:0")
    q3x.moe_routed_logits(gul, dnl, X, 1, logits, k, ids1, w1, Y1)
    torch.cuda.synchronize()
    ids_o, w_o, _ = oracle.router_top_k(lg, k)
    assert np.array_equal(host(ids0), ids_o) and np.array_equal(host(ids1), ids_o)
    assert np.array_equal(host(w1).view(np.uint32), w_o.view(np.uint32))
    assert np.array_equal(host(Y1).view(np.uint32), host(Y0).view(np.uint32))
    want = oracle.moe_routed(gu_h, dn_h, type_, E, H, I, X_h, ids_o, w_o)
    bound = moe_bound(gu_h, dn_h, type_, E, H, I, X_h, ids_o, w_o)
    assert np.all(np.abs(host(Y1).astype(np.float64) - want) <= bound)
