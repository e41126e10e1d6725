"""GPU test of q3x_hip_moe_routed_noalloc, the routed-expert matmul on the
library's static per-device scratch (no workspace argument, no allocation),
through the C ABI: its output equals q3x_hip_moe_routed's with a caller
workspace bit for bit, on two calls in a row (the second smaller, so it
reuses the first call's scratch contents), for the grouped prefill path and
the fused decode path; requests larger than the scratch are rejected before
any device work."""
import ctypes

import numpy as np
import pytest

import qwen3x_amd as q3x
from tests.helpers import Q4_0, Q8_0, bits, random_blocks
from tests.test_gpu_parity import _torch, dev, host, say

pytestmark = pytest.mark.gpu

SCRATCH = 32 << 20


def _routed(torch, noalloc, gu, dn, type_, E, H, I, X, tokens, ids, wts, k, Y, accumulate):
    lib = q3x.lib()
    stream = torch.cuda.current_stream().cuda_stream
    args = [gu.data_ptr(), dn.data_ptr(), type_, E, H, I, X.data_ptr(), tokens, ids.data_ptr(), wts.data_ptr(), k,
            Y.data_ptr(), accumulate]
    if noalloc:
        return lib.q3x_hip_moe_routed_noalloc(*args, stream)
    need = q3x.moe_workspace_bytes(tokens, E, k, H, I)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda:0")
    code = lib.q3x_hip_moe_routed(*args, ws.data_ptr(), need, stream)
    torch.cuda.synchronize()
    return code


def _inputs(rng, torch, E, H, k, tokens):
    X = rng.normal(0, 1, (tokens, H)).astype(np.float32)
    logits = rng.normal(0, 1, (tokens, E)).astype(np.float32)
    ids = torch.empty((tokens, k), dtype=torch.int32, device="cuda:0")
    wts = torch.empty((tokens, k), dtype=torch.float32, device="cuda:0")
    q3x.router_top_k(dev(logits), tokens, E, k, ids, wts)
    return dev(X), ids, wts


@pytest.mark.parametrize("type_,E,H,I,k,calls", [
    # 35B-A3B expert shape: 256 tokens (28 MiB of workspace), then 3 tokens,
    # then one token (the fused decode path), then 256 tokens again
    (Q4_0, 64, 2048, 512, 8, (256, 3, 1, 256)),
    (Q8_0, 16, 512, 256, 4, (100, 1, 40))])
def test_noalloc_equals_the_workspace_entry_point(type_, E, H, I, k, calls):
    torch = _torch()
    assert q3x.NOALLOC_SCRATCH_BYTES == SCRATCH
    rng = np.random.default_rng(E + H + k)
    gu = dev(random_blocks(rng, type_, E * 2 * I, H))
    dn = dev(random_blocks(rng, type_, E * H, I))
    for tokens in calls:
        say(f"noalloc type={type_} E={E} H={H} I={I} k={k} tokens={tokens}")
        X, ids, wts = _inputs(rng, torch, E, H, k, tokens)
        for accumulate in (0, 1):
            base = rng.normal(0, 1, (tokens, H)).astype(np.float32)
            want = dev(base)
            got = dev(base)
            assert _routed(torch, False, gu, dn, type_, E, H, I, X, tokens, ids, wts, k, want, accumulate) == q3x.OK
            assert _routed(torch, True, gu, dn, type_, E, H, I, X, tokens, ids, wts, k, got, accumulate) == q3x.OK
            torch.cuda.synchronize()
            assert np.array_equal(bits(host(got)), bits(host(want))), (tokens, accumulate)


def test_noalloc_rejects_requests_beyond_the_scratch():
    torch = _torch()
    E, H, I, k = 64, 2048, 512, 8
    tokens = 300  # 32.8 MiB of workspace
    assert q3x.moe_workspace_bytes(tokens, E, k, H, I) > SCRATCH
    Y = torch.full((tokens, H), 7.0, dtype=torch.float32, device="cuda:0")
    P = ctypes.c_void_p(0x1000)  # never dereferenced: the size check fails first
    code = q3x.lib().q3x_hip_moe_routed_noalloc(P, P, Q4_0, E, H, I, P, tokens, P, P, k, Y.data_ptr(), 0, None)
    assert code == q3x.ESCRATCH
    assert "scratch" in q3x.strerror(code)
    torch.cuda.synchronize()
    assert bool((Y == 7.0).all())
