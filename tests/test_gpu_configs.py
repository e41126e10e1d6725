"""The five BASELINE.json configurations at full size, on the GPU, against the
oracle on the same bytes (weights quantised on the GPU by q3x_hip_quantize,
whose bit-exactness with the reference packer is tested separately).

Tolerance: max|delta| <= 1e-5 * ||w_row||_2 * ||x||_2 per element, every
output of every config against the oracle (the N=4096 prefill included);
the N=4096 prefill is also checked token by token against the GPU matvec
within twice the bound -- a size-independent consistency property."""
import numpy as np
import pytest

import oracle
import qwen3x_amd as q3x
from qwen3x_amd import workloads as wl
from tests.helpers import dequant_numpy, row_bound
from tests.test_gpu_parity import TOL, moe_bound

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    assert torch.cuda.is_available()
    return torch


def host(t):
    _torch().cuda.synchronize()
    return t.cpu().numpy()


def say(msg):
    print(msg, flush=True)


def check(got, want, bound, label):
    diff = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert np.all(np.isfinite(got)), label
    bad = diff > bound
    assert not bad.any(), f"{label}: {bad.sum()} outside; worst {diff[bad].max()} vs {bound[bad].min()}"
    return float((diff / np.maximum(bound, 1e-300)).max())


@pytest.mark.parametrize("index", [0, 1, 3])
def test_decode_matvec_configs(index):
    torch = _torch()
    mats = wl.dense_matrices(index)
    cols_max = max(m.cols for m in mats)
    x_full = wl.activations(index, 1, cols_max)[0].contiguous()
    x_host = host(x_full)
    for m in mats:
        say(f"config {index} {m.name} {m.rows}x{m.cols}")
        y = torch.empty(m.rows, dtype=torch.float32, device="cuda:0")
        q3x.mv(m.linear, x_full, y)
        w = host(m.weight)
        x = x_host[:m.cols]
        want = oracle.mv(w, m.type, m.rows, m.cols, x)
        wd = dequant_numpy(w, m.type, m.rows, m.cols)
        # dequantised rows are bit-exact with the reference's embed
        sample_rows = [0, m.rows // 2, m.rows - 1]
        out = torch.empty((1, m.cols), dtype=torch.float32, device="cuda:0")
        for r in sample_rows:
            q3x.dequant(m.linear, r, 1, out)
            assert np.array_equal(host(out)[0].view(np.uint32), oracle.embed(w, m.type, m.cols, r).view(np.uint32))
        worst = check(host(y), want, row_bound(wd, x, TOL), f"config {index} {m.name}")
        say(f"  worst |delta|/bound = {worst:.3g}")


@pytest.mark.parametrize("index,count,split", [(2, 512, False), (2, 4096, False), (3, 512, False),
                                               (2, 512, True), (3, 512, True)])
def test_prefill_gemm_configs(index, count, split):
    # split: q3x_hip_gemm_ws with the workspace its plan asks for (the down
    # projections at N = 512 split K over workgroups).
    torch = _torch()
    mats = wl.dense_matrices(index)
    for m in mats:
        say(f"config {index} N={count} {m.name} {m.rows}x{m.cols} split={split}")
        X = wl.activations(index, count, m.cols, salt=m.rows)
        Y = torch.empty((count, m.rows), dtype=torch.float32, device="cuda:0")
        if split:
            nbytes = q3x.gemm_workspace_bytes(m.linear, count)
            ws = torch.empty(max(nbytes, 4) // 4, dtype=torch.float32, device="cuda:0")
            q3x.batch_mv_ws(m.linear, X, Y, count, ws if nbytes else None)
            del ws
        else:
            q3x.batch_mv(m.linear, X, Y, count)
        w = host(m.weight)
        Xh = host(X)
        Yh = host(Y)
        wd = dequant_numpy(w, m.type, m.rows, m.cols)
        # Every token against the oracle (row-parallel on the host's cores:
        # about 15 s at N = 4096 on 16 cores).
        toks = np.arange(count)
        want = oracle.gemm(w, m.type, m.rows, m.cols, Xh[toks])
        worst = check(Yh[toks], want, row_bound(wd, Xh[toks], TOL), f"config {index} {m.name} N={count}")
        say(f"  worst |delta|/bound = {worst:.3g} over {toks.size} tokens")
        if count > 512:
            # every token against the GPU matvec
            Ymv = torch.empty_like(Y)
            for t in range(count):
                q3x.mv(m.linear, X[t], Ymv[t])
            check(Yh, host(Ymv), 2 * row_bound(wd, Xh, TOL), f"config {index} {m.name}: GEMM vs matvec")
        del X, Y


@pytest.mark.parametrize("tokens", [1, 2048])
def test_moe_config(tokens):
    torch = _torch()
    moe = wl.moe_weights(4)
    k = wl.CONFIGS[4]["top_k"]
    logits = wl.router_logits(4, tokens, moe.experts)
    X = wl.activations(4, tokens, moe.H)
    ids = torch.empty((tokens, k), dtype=torch.int32, device="cuda:0")
    wts = torch.empty((tokens, k), dtype=torch.float32, device="cuda:0")
    Y = torch.empty((tokens, moe.H), dtype=torch.float32, device="cuda:0")
    say(f"config 4 tokens={tokens}: router + routed experts")
    q3x.router_top_k(logits, tokens, moe.experts, k, ids, wts)
    q3x.moe_routed(moe.gate_up_linear, moe.down_linear, X, tokens, ids, wts, k, Y)
    ids_h, wts_h, lg = host(ids), host(wts), host(logits)
    ids_o, wts_o, _ = oracle.router_top_k(lg, k)
    # the router is exact: same experts, same weights bit for bit
    assert np.array_equal(ids_h, ids_o)
    assert np.array_equal(wts_h.view(np.uint32), wts_o.view(np.uint32))
    gu, dn = host(moe.gate_up), host(moe.down)
    Xh = host(X)
    want = oracle.moe_routed(gu, dn, moe.type, moe.experts, moe.H, moe.I, Xh, ids_h, wts_h)
    bound = moe_bound(gu, dn, moe.type, moe.experts, moe.H, moe.I, Xh, ids_h, wts_h)
    worst = check(host(Y), want, bound, f"config 4 tokens={tokens}")
    say(f"  worst |delta|/bound = {worst:.3g}")
