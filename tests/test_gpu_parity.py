"""GPU parity tests: the HIP library (through its C ABI) against the CPU oracle on
the same seeded inputs.

Bar (north star): dequantised weights bit-exact; outputs within
max|delta| <= 1e-5 * ||w_row||_2 * ||x||_2 per element (norms in double),
because only the FP32 summation order may differ.  Index work (router ids,
grouping) is exact."""
import os
import subprocess
import sys

import numpy as np
import pytest

import oracle
import qwen3x_amd as q3x
from tests.helpers import Q4_0, Q8_0, bits, dequant_numpy, q4_blocks, q8_blocks, random_blocks, row_bound

pytestmark = pytest.mark.gpu
TOL = 1e-5


def _torch():
    import torch
    assert torch.cuda.is_available(), "GPU tests need cuda:0"
    return torch


def dev(a):
    torch = _torch()
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def host(t):
    _torch().cuda.synchronize()
    return t.cpu().numpy()


def say(msg):
    print(msg, flush=True)


def check_bound(got, want, wd, x, label):
    bound = row_bound(wd, x, TOL)
    diff = np.abs(got.astype(np.float64) - want.astype(np.float64))
    bad = diff > bound
    assert np.all(np.isfinite(got)), label
    assert not bad.any(), f"{label}: {bad.sum()} outside bound; worst {diff[bad].max()} vs {bound[bad].min()}"


# ----------------------------------------------------------- host binary ----

def test_reference_unit_cases_through_cpp_host_interface(repo_root):
    exe = os.path.join(repo_root, "qwen3x_amd", "q3x_hip_host_test")
    say(f"running {exe}")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "q3x-hip-host-test: ok" in r.stdout


# --------------------------------------------------------------- dequant ----

SPECIAL = np.array([0x3555, 0x2E66, 0x0400, 0x0001, 0x8001, 0x03FF, 0x7BFF, 0xFBFF, 0x0000, 0x8000], np.uint16)


@pytest.mark.parametrize("type_", [Q8_0, Q4_0])
@pytest.mark.parametrize("rows,cols,special", [(2, 64, False), (37, 96, True), (256, 4096, False),
                                               (64, 5120, True)])
def test_dequant_bit_exact(type_, rows, cols, special):
    torch = _torch()
    rng = np.random.default_rng(rows + cols + type_)
    w = random_blocks(rng, type_, rows, cols, SPECIAL if special else None)
    want = oracle.dequant(w, type_, rows, cols)
    out = torch.empty((rows, cols), dtype=torch.float32, device="cuda:0")
    say(f"dequant type={type_} {rows}x{cols}")
    q3x.dequant(q3x.Linear(dev(w), rows, cols, type_), 0, rows, out)
    got = host(out)
    assert np.array_equal(bits(got), bits(want))
    # a window of the last rows
    n = min(3, rows)
    part = torch.empty((n, cols), dtype=torch.float32, device="cuda:0")
    q3x.dequant(q3x.Linear(dev(w), rows, cols, type_), rows - n, n, part)
    assert np.array_equal(bits(host(part)), bits(want[rows - n:]))


def test_dequant_all_fp16_scales_bit_exact():
    # Every one of the 65536 scale patterns, finite ones bit for bit, NaN as NaN.
    torch = _torch()
    scales = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    vals = np.tile(np.arange(-16, 16, dtype=np.int64), (65536, 1))
    from tests.helpers import q8_blocks
    w = q8_blocks(scales, vals)
    rows, cols = 2048, 1024
    want = oracle.dequant(w, Q8_0, rows, cols)
    out = torch.empty((rows, cols), dtype=torch.float32, device="cuda:0")
    q3x.dequant(q3x.Linear(dev(w), rows, cols, Q8_0), 0, rows, out)
    got = host(out)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(bits(got)[~nan], bits(want)[~nan])


# -------------------------------------------------------------------- mv ----

MV_SHAPES = [
    (1, 32), (2, 64), (3, 96), (5, 160),           # generic path (rows not 256-col multiples)
    (7, 256), (33, 512),                           # 16 lanes per row
    (65, 1024),                                    # 32 lanes per row
    (100, 2048), (1000, 4096), (5, 12288),         # 64 lanes per row, passes
    (17, 5120), (3, 17408), (129, 2304),           # partial last pass
]


@pytest.mark.parametrize("type_", [Q8_0, Q4_0])
@pytest.mark.parametrize("rows,cols", MV_SHAPES)
def test_mv_parity(type_, rows, cols):
    torch = _torch()
    rng = np.random.default_rng(rows * 31 + cols + type_)
    w = random_blocks(rng, type_, rows, cols)
    x = rng.normal(0, 1, cols).astype(np.float32)
    want = oracle.mv(w, type_, rows, cols, x)
    wd = dequant_numpy(w, type_, rows, cols)
    lin = q3x.Linear(dev(w), rows, cols, type_)
    y = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda:0")
    say(f"mv type={type_} {rows}x{cols}")
    q3x.mv(lin, dev(x), y)
    got = host(y)
    check_bound(got, want, wd, x, f"mv {rows}x{cols}")
    # accumulate: y += W x
    q3x.mv_add(lin, dev(x), y)
    check_bound(host(y), 2 * want, wd, 2 * x, f"mv_add {rows}x{cols}")
    # deterministic: identical bits on a second run
    y2 = torch.empty_like(y)
    q3x.mv(lin, dev(x), y2)
    assert np.array_equal(bits(host(y2)), bits(got))


@pytest.mark.parametrize("type_", [Q8_0, Q4_0])
def test_mv_unaligned_pointers_take_the_generic_path(type_):
    torch = _torch()
    rows, cols = 40, 4096
    rng = np.random.default_rng(17)
    w = random_blocks(rng, type_, rows, cols)
    x = rng.normal(0, 1, cols).astype(np.float32)
    want = oracle.mv(w, type_, rows, cols, x)
    wd = dequant_numpy(w, type_, rows, cols)
    wbuf = torch.zeros(w.size + 16, dtype=torch.uint8, device="cuda:0")
    wbuf[2:2 + w.size] = dev(w)
    xbuf = torch.zeros(cols + 1, dtype=torch.float32, device="cuda:0")
    xbuf[1:] = dev(x)
    y = torch.empty(rows, dtype=torch.float32, device="cuda:0")
    q3x.mv(q3x.Linear(wbuf[2:], rows, cols, type_), xbuf[1:], y)
    check_bound(host(y), want, wd, x, "unaligned mv")


def _q4_sparse(rng, rows, cols, live):
    """Q4_0 rows whose nibbles are all 8 (weight zero) except a fraction `live`
    drawn uniformly from 0..15; returns the bytes and the nibbles [rows, cols]."""
    nb = rows * cols // 32
    scales = rng.normal(0.0, 0.02, nb).astype(np.float16).view(np.uint16)
    n = np.full((nb, 32), 8, np.int64)
    m = rng.random((nb, 32)) < live
    n[m] = rng.integers(0, 16, int(m.sum()))
    packed = (n[:, :16] | (n[:, 16:] << 4)).astype(np.uint8)
    return q4_blocks(scales, packed), n.reshape(rows, cols)


def q4_error_bound(w, nib, rows, cols, x):
    """Guaranteed bound on |y - W x| for the Q4_0 matvec kernels.

    The staged kernels (block_dot_q4_exact) multiply each weight n - 8, exact
    in binary16, by its FP32 activation exactly, sum elements 0..15 and
    16..31 in two chains of 16 (the first FMA of each adds to zero, so 15
    roundings), join them with one FMA and multiply by f16(d): at most
    gamma(17) * |d| * sum_i |n_i - 8| |x_i| per block.  The generic kernel
    runs the reference's single chain of 32 (arch/cpu.cpp:91-101) and the
    scale FMA: gamma(33).  A row adds its blocks in per-lane partial sums of
    at most ceil(nb / 16) blocks, then a tree of at most 6 levels, and the
    store may add y: every block value passes through at most
    ceil(nb / 16) + 7 roundings.  With |v_b| <= (1 + gamma(33)) |d_b| sum_i
    |n_i - 8| |x_i| the total is at most gamma(33 + ceil(nb/16) + 8) *
    sum_j |w_j| |x_j| <= that times ||w|| ||x|| (Cauchy-Schwarz), which stays
    inside the north-star 1e-5 * ||w|| ||x|| for rows of up to 64,512 columns."""
    u = 2.0 ** -24

    def gamma(k):
        return k * u / (1 - k * u)

    nb = cols // 32
    blk = w.reshape(rows * nb, 18)
    d = np.abs(blk[:, 0:2].copy().view(np.float16).astype(np.float64)).reshape(rows, nb)
    ax = np.abs(x.astype(np.float64)).reshape(nb, 32)
    n = nib.astype(np.float64).reshape(rows, nb, 32)
    terms = (np.abs(n - 8.0) * ax[None]).sum(axis=2)                # [rows, nb]
    return gamma(33 + -(-nb // 16) + 8) * (d * terms).sum(axis=1)


@pytest.mark.parametrize("rows,cols", [(64, 2048), (64, 4096), (64, 5120), (32, 12288), (16, 17408)])
@pytest.mark.parametrize("live", [0.0, 0.01, 0.05, 0.1, 0.5])
@pytest.mark.parametrize("aligned", [True, False])
def test_mv_q4_sparse_blocks_error_bound(rows, cols, live, aligned):
    # Blocks that are mostly nibble 8 (zero weights) at the production widths,
    # and rows with exactly one live nibble per block: the staged kernel
    # (aligned) and the generic kernel (unaligned) against W x in double,
    # within the guaranteed bound above, which itself lies inside the
    # north-star bound; rows of zero weights give exactly zero.
    torch = _torch()
    rng = np.random.default_rng(int(cols + 1000 * live + rows))
    w, nib = _q4_sparse(rng, rows, cols, live)
    w = w.reshape(rows, cols // 32, 18)
    nib[rows // 2] = 8                                  # one row of zero weights
    w[rows // 2, :, 2:] = 0x88
    one = rows // 2 + 1                                 # one live nibble (7 or 9) per block
    nb = cols // 32
    nib[one] = 8
    pos = rng.integers(0, 32, nb)
    nib[one].reshape(nb, 32)[np.arange(nb), pos] = rng.choice([7, 9], nb)
    row = nib[one].reshape(nb, 32)
    w[one, :, 2:] = (row[:, :16] | (row[:, 16:] << 4)).astype(np.uint8)
    w = w.reshape(-1)
    x = rng.normal(0, 1, cols).astype(np.float32)
    x[::7] *= np.float32(50)                            # a spread of magnitudes
    wd = dequant_numpy(w, Q4_0, rows, cols)
    exact = wd.astype(np.float64) @ x.astype(np.float64)
    want = oracle.mv(w, Q4_0, rows, cols, x)
    say(f"q4 sparse mv {rows}x{cols} live={live} aligned={aligned}")
    if aligned:
        wt, xt = dev(w), dev(x)
    else:
        wt = torch.zeros(w.size + 16, dtype=torch.uint8, device="cuda:0")
        wt[2:2 + w.size] = dev(w)
        wt = wt[2:]
        xbuf = torch.zeros(cols + 1, dtype=torch.float32, device="cuda:0")
        xbuf[1:] = dev(x)
        xt = xbuf[1:]
    y = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda:0")
    q3x.mv(q3x.Linear(wt, rows, cols, Q4_0), xt, y)
    got = host(y)
    assert got[rows // 2] == 0.0 and want[rows // 2] == 0.0
    err = np.abs(got.astype(np.float64) - exact)
    bound = q4_error_bound(w, nib, rows, cols, x)
    assert np.all(err <= bound), f"worst {(err / np.maximum(bound, 1e-300)).max()} of the bound"
    north = row_bound(wd, x, TOL)
    assert np.all(bound <= north)                      # the guarantee is inside the north-star bound
    check_bound(got, want, wd, x, f"q4 sparse {rows}x{cols}")
    ref_err = np.abs(want.astype(np.float64) - exact)
    say(f"  max |err| gpu {err.max():.3e}  reference {ref_err.max():.3e}  bound {bound.max():.3e}")


@pytest.mark.parametrize("type_,rows,cols", [(Q8_0, 70000, 2048), (Q4_0, 70000, 2048), (Q8_0, 20000, 768),
                                             (Q4_0, 300000, 256)])
def test_mv_many_rows_multi_row_waves(type_, rows, cols):
    # Row counts that select 2 and 4 row iterations per wavefront.
    torch = _torch()
    rng = np.random.default_rng(rows + cols)
    w = random_blocks(rng, type_, rows, cols)
    x = rng.normal(0, 1, cols).astype(np.float32)
    want = oracle.mv(w, type_, rows, cols, x)
    wd = dequant_numpy(w, type_, rows, cols)
    y = torch.empty(rows, dtype=torch.float32, device="cuda:0")
    say(f"mv many rows type={type_} {rows}x{cols}")
    q3x.mv(q3x.Linear(dev(w), rows, cols, type_), dev(x), y)
    check_bound(host(y), want, wd, x, f"mv {rows}x{cols}")


def test_mv_zero_rows_are_exactly_zero():
    # ||w_row|| = 0 allows no error at all: zero scales and all-0x88 Q4 blocks.
    torch = _torch()
    rows, cols = 8, 4096
    rng = np.random.default_rng(2)
    x = dev(rng.normal(0, 1, cols).astype(np.float32))
    from tests.helpers import q4_blocks, q8_blocks
    nb = rows * cols // 32
    for type_, w in ((Q8_0, q8_blocks(np.zeros(nb), rng.integers(-128, 128, (nb, 32)))),
                     (Q4_0, q4_blocks(np.full(nb, 0x3C00), np.full((nb, 16), 0x88)))):
        y = torch.full((rows,), 7.0, dtype=torch.float32, device="cuda:0")
        q3x.mv(q3x.Linear(dev(w), rows, cols, type_), x, y)
        assert np.all(host(y) == 0.0)


# -------------------------------------------------------------- mv_multi ----

@pytest.mark.parametrize("type_,cols,rows_list,acc", [
    (Q8_0, 4096, [4096, 1024, 1024], [False, False, True]),    # q, k, v (v accumulates)
    (Q4_0, 5120, [3000, 3000], [False, False]),                # gate, up
    (Q8_0, 2048, [1, 7, 100, 2049, 33, 5, 64, 900], [True, False] * 4),  # 8 matrices
    (Q4_0, 512, [70, 3], [False, True]),                       # 16 lanes per row
    (Q8_0, 96, [5, 3], [False, True]),                         # rows not 16-byte multiples: generic path
    # 21288 rows together take the 64-VGPR build of 16K-64K-row Q8_0 launches,
    # each matrix alone the default build: same arithmetic, same bits
    (Q8_0, 1024, [12288, 9000], [False, True]),
])
def test_mv_multi_equals_separate_mv(type_, cols, rows_list, acc):
    torch = _torch()
    rng = np.random.default_rng(cols + len(rows_list) + type_)
    x = rng.normal(0, 1, cols).astype(np.float32)
    xd = dev(x)
    mats, outs, seps = [], [], []
    for i, rows in enumerate(rows_list):
        w = random_blocks(rng, type_, rows, cols)
        start = rng.normal(0, 1, rows).astype(np.float32)
        mats.append((w, q3x.Linear(dev(w), rows, cols, type_)))
        outs.append(dev(start))
        seps.append(dev(start))
    say(f"mv_multi type={type_} cols={cols} rows={rows_list}")
    q3x.mv_multi([m for _, m in mats], xd, outs, acc)
    for (w, m), y, a in zip(mats, seps, acc):
        q3x.mv(m, xd, y, a)
    for (w, m), got, sep, a, in zip(mats, outs, seps, acc):
        g = host(got)
        assert np.array_equal(bits(g), bits(host(sep))), f"rows={m.rows}: mv_multi differs from mv"
        want = oracle.mv(w, type_, m.rows, cols, x)
        wd = dequant_numpy(w, type_, m.rows, cols)
        if not a:
            check_bound(g, want, wd, x, f"mv_multi {m.rows}x{cols}")


def test_mv_multi_rejects_mixed_or_bad_items():
    torch = _torch()
    w = torch.zeros(34 * 4, dtype=torch.uint8, device="cuda:0")
    x = torch.zeros(128, dtype=torch.float32, device="cuda:0")
    y = torch.zeros(4, dtype=torch.float32, device="cuda:0")
    with pytest.raises(ValueError):
        q3x.mv_multi([q3x.Linear(w, 1, 128, Q8_0), q3x.Linear(w, 1, 64, Q8_0)], x, [y, y])
    with pytest.raises(ValueError):
        q3x.mv_multi([q3x.Linear(w, 1, 128, Q8_0)] * 9, x, [y] * 9)
    with pytest.raises(q3x.Q3xHipError):
        q3x.mv_multi([q3x.Linear(w, 0, 128, Q8_0)], x, [y])


# ------------------------------------------------------------------ GEMM ----

GEMM_CASES = [(Q8_0, 64, 128, 1), (Q8_0, 130, 256, 5), (Q8_0, 300, 512, 129), (Q4_0, 256, 1024, 37),
              (Q4_0, 129, 4096, 300), (Q8_0, 1000, 2048, 128), (Q4_0, 77, 96, 3), (Q8_0, 3, 64, 200),
              # 128x128-tile path (>= 512 workgroups), partial tiles on both edges
              (Q8_0, 4096, 512, 2048), (Q4_0, 4000, 256, 2100),
              # 128x192 tiles (one per CU), whole and partial on both edges
              (Q8_0, 12288, 256, 512), (Q4_0, 12000, 128, 500),
              # 64x128 tiles with the K blocks in two halves (long K, <= 256 tiles), odd block count
              (Q8_0, 3300, 8224, 300)]


@pytest.mark.parametrize("type_,rows,cols,count", GEMM_CASES)
def test_gemm_parity(type_, rows, cols, count):
    torch = _torch()
    rng = np.random.default_rng(rows + cols + count + type_)
    w = random_blocks(rng, type_, rows, cols)
    X = rng.normal(0, 1, (count, cols)).astype(np.float32)
    want = oracle.gemm(w, type_, rows, cols, X)
    wd = dequant_numpy(w, type_, rows, cols)
    lin = q3x.Linear(dev(w), rows, cols, type_)
    Y = torch.full((count, rows), float("nan"), dtype=torch.float32, device="cuda:0")
    say(f"gemm type={type_} {rows}x{cols} count={count}")
    q3x.batch_mv(lin, dev(X), Y, count)
    got = host(Y)
    check_bound(got, want, wd, X, f"gemm {rows}x{cols}x{count}")
    q3x.batch_mv(lin, dev(X), Y, count, add=True)
    check_bound(host(Y), 2 * want, wd, 2 * X, "gemm add")


# One nonzero weight per row: every block sum is a single product q * x, so
# the GEMM must return fl(d * fl(q * x)) up to the matrix cores' own
# rounding (the reference's loop, arch/cpu.cpp:64-73 / 91-101, computes
# exactly that: inner = q * x, then sum = d * inner from zero).  The prefill
# kernel splits x into three bf16 parts and sums q * a3 + q * a2 + q * a1;
# the products and the first partial sum are exact, and the matrix cores'
# FP32 accumulation is not rounded like IEEE round-to-nearest (measured: one
# ulp off in about 14% of single-product sums), so the bar is 2 ulp -- where a
# dropped split part errs by 2^8 ulp or more, and a mispaired activation and
# weight chunk or a misplaced tile by an unrelated value.  x spans 2^-90 ..
# 2^90.  The shapes take each tile shape of the launch (128 x 256, 128 x 192,
# 64 x 128 with one and two stages ahead and with the K blocks in two
# halves -- an even and an odd block count -- and 64 x 64) and partial tiles.
ONE_PRODUCT_CASES = [(Q8_0, 4096, 256, 2048), (Q4_0, 4096, 320, 2048), (Q8_0, 4096, 8192, 512),
                     (Q4_0, 2048, 1024, 1024), (Q8_0, 257, 512, 300), (Q4_0, 100, 96, 7),
                     (Q8_0, 12288, 128, 512), (Q4_0, 11999, 96, 500), (Q4_0, 4096, 8192, 1024),
                     (Q4_0, 4096, 8224, 500)]


def _one_product_matrix(rng, type_, rows, cols):
    nbr = cols // 32
    scales = rng.normal(0.0, 0.05, rows * nbr).astype(np.float16)
    scales[scales == 0] = np.float16(0.01)
    col = rng.integers(0, cols, rows)
    if type_ == Q8_0:
        q = rng.integers(1, 128, rows) * rng.choice([-1, 1], rows)
        values = np.zeros((rows, cols), np.int64)
        values[np.arange(rows), col] = q
        w = q8_blocks(scales.view(np.uint16), values.reshape(-1, 32))
    else:
        nib = rng.integers(0, 15, rows)
        nib[nib >= 8] += 1  # 0..15 without 8
        q = nib - 8
        full = np.full((rows, cols), 8, np.uint8)
        full[np.arange(rows), col] = nib
        blocks = full.reshape(-1, 32)
        w = q4_blocks(scales.view(np.uint16), blocks[:, :16] | (blocks[:, 16:] << 4))
    d = scales.reshape(rows, nbr)[np.arange(rows), col // 32].astype(np.float32)
    return w, col, q.astype(np.float32), d


@pytest.mark.parametrize("type_,rows,cols,count", ONE_PRODUCT_CASES)
def test_gemm_one_product_per_row(type_, rows, cols, count):
    torch = _torch()
    rng = np.random.default_rng(rows * 7 + cols + count + type_)
    w, col, q, d = _one_product_matrix(rng, type_, rows, cols)
    mant = rng.uniform(1.0, 2.0, (count, cols)) * rng.choice([-1.0, 1.0], (count, cols))
    X = np.ldexp(mant, rng.integers(-90, 91, (count, cols))).astype(np.float32)
    want = d[None, :] * (q[None, :] * X[:, col])  # float32: rounded after each product
    toks = np.array([0, count // 2, count - 1])
    assert np.array_equal(bits(oracle.gemm(w, type_, rows, cols, X[toks])), bits(want[toks]))
    lin = q3x.Linear(dev(w), rows, cols, type_)
    Y = torch.full((count, rows), float("nan"), dtype=torch.float32, device="cuda:0")
    say(f"gemm one product per row: type={type_} {rows}x{cols} count={count}")
    q3x.batch_mv(lin, dev(X), Y, count)
    got = host(Y)
    assert np.all(np.sign(got) == np.sign(want))
    ulps = np.abs(bits(got).astype(np.int64) - bits(want).astype(np.int64))
    say(f"  exact {np.mean(ulps == 0):.3f}, worst {ulps.max()} ulp")
    assert ulps.max() <= 2, f"{np.count_nonzero(ulps > 2)} outputs beyond 2 ulp; first at {np.argwhere(ulps > 2)[0]}"
    q3x.batch_mv(lin, dev(X), Y, count, add=True)  # the same sums again, added: exactly twice
    assert np.array_equal(bits(host(Y)), bits(got + got))


# Split K (q3x_hip_gemm_ws): shapes whose plan splits (few output tiles over
# a long K), against the oracle's bound, with accumulate, twice in a row bit
# for bit (deterministic), and with a workspace one byte short (the unsplit
# launch, equal to q3x_hip_gemm bit for bit).  Odd and uneven K block counts
# give units of unequal length; partial tiles on both edges.
SPLIT_CASES = [(Q8_0, 256, 8192, 64), (Q4_0, 300, 8224, 70), (Q8_0, 1000, 12288, 130), (Q4_0, 640, 17408, 40),
               (Q8_0, 77, 16416, 3)]


def _workspace(linear, count):
    torch = _torch()
    nbytes = q3x.gemm_workspace_bytes(linear, count)
    assert nbytes > 0, "the plan must split this shape"
    return torch.empty(nbytes // 4, dtype=torch.float32, device="cuda:0"), nbytes


@pytest.mark.parametrize("type_,rows,cols,count", SPLIT_CASES)
def test_gemm_split_parity(type_, rows, cols, count):
    torch = _torch()
    rng = np.random.default_rng(rows + 3 * cols + count + type_)
    w = random_blocks(rng, type_, rows, cols)
    X = rng.normal(0, 1, (count, cols)).astype(np.float32)
    want = oracle.gemm(w, type_, rows, cols, X)
    wd = dequant_numpy(w, type_, rows, cols)
    lin = q3x.Linear(dev(w), rows, cols, type_)
    ws, nbytes = _workspace(lin, count)
    say(f"gemm split type={type_} {rows}x{cols} count={count} workspace={nbytes}")
    Xd = dev(X)
    Y = torch.full((count, rows), float("nan"), dtype=torch.float32, device="cuda:0")
    q3x.batch_mv_ws(lin, Xd, Y, count, ws)
    got = host(Y)
    check_bound(got, want, wd, X, f"gemm split {rows}x{cols}x{count}")
    Y2 = torch.full_like(Y, float("nan"))
    q3x.batch_mv_ws(lin, Xd, Y2, count, ws)
    assert np.array_equal(bits(host(Y2)), bits(got))
    q3x.batch_mv_ws(lin, Xd, Y, count, ws, add=True)
    check_bound(host(Y), 2 * want, wd, 2 * X, "gemm split add")
    # one byte short: the unsplit launch, q3x_hip_gemm's result
    short = ws.view(torch.uint8)[: nbytes - 1]
    Y3 = torch.full_like(Y, float("nan"))
    q3x.batch_mv_ws(lin, Xd, Y3, count, short)
    Y4 = torch.full_like(Y, float("nan"))
    q3x.batch_mv(lin, Xd, Y4, count)
    assert np.array_equal(bits(host(Y3)), bits(host(Y4)))


# The one-product matrices through the split launch: a block's product lands
# in one unit, the others add exact zeros, so the same 2-ulp bar holds; a
# unit summed into the wrong tile or slot gives unrelated values.
@pytest.mark.parametrize("type_,rows,cols,count", [(Q8_0, 256, 8192, 64), (Q4_0, 300, 8224, 70),
                                                   (Q8_0, 5120, 17408, 512)])
def test_gemm_split_one_product_per_row(type_, rows, cols, count):
    torch = _torch()
    rng = np.random.default_rng(rows * 11 + cols + count + type_)
    w, col, q, d = _one_product_matrix(rng, type_, rows, cols)
    mant = rng.uniform(1.0, 2.0, (count, cols)) * rng.choice([-1.0, 1.0], (count, cols))
    X = np.ldexp(mant, rng.integers(-90, 91, (count, cols))).astype(np.float32)
    want = d[None, :] * (q[None, :] * X[:, col])
    lin = q3x.Linear(dev(w), rows, cols, type_)
    ws, nbytes = _workspace(lin, count)
    Y = torch.full((count, rows), float("nan"), dtype=torch.float32, device="cuda:0")
    say(f"gemm split one product per row: type={type_} {rows}x{cols} count={count} workspace={nbytes}")
    q3x.batch_mv_ws(lin, dev(X), Y, count, ws)
    got = host(Y)
    assert np.all(np.sign(got) == np.sign(want))
    ulps = np.abs(bits(got).astype(np.int64) - bits(want).astype(np.int64))
    say(f"  exact {np.mean(ulps == 0):.3f}, worst {ulps.max()} ulp")
    assert ulps.max() <= 2, f"{np.count_nonzero(ulps > 2)} outputs beyond 2 ulp; first at {np.argwhere(ulps > 2)[0]}"


# ---------------------------------------------------------------- router ----

def _router_logits(rng, tokens, experts, kind):
    if kind == "normal":
        logits = rng.normal(0, 1, (tokens, experts)).astype(np.float32)
        logits[::7, 3] = logits[::7, 5]  # exact ties
    elif kind == "grid":
        # values on a coarse grid: many equal probabilities, and distinct ones
        # that the division by the total can round together
        logits = (rng.integers(-6, 7, (tokens, experts)) * 0.125).astype(np.float32)
    else:
        # a wide spread: exp underflows to subnormals and to zero, -inf logits
        logits = rng.normal(0, 40, (tokens, experts)).astype(np.float32)
        logits[::5, 0] = -np.inf
        logits[::3, 1] = -120.0
    return logits


@pytest.mark.parametrize("tokens,experts,top_k,kind", [
    (1, 256, 8, "normal"), (2048, 256, 8, "normal"), (37, 6, 3, "normal"), (100, 1024, 8, "normal"),
    (5, 64, 1, "normal"), (513, 256, 8, "grid"), (64, 130, 8, "grid"), (300, 256, 8, "wide"),
    (9, 1000, 5, "wide")])
def test_router_parity(tokens, experts, top_k, kind):
    # The GPU softmax is the reference's operation for operation (libm's expf
    # arithmetic, the total in expert order, correctly rounded divisions), so
    # ids and weights are exact.
    torch = _torch()
    rng = np.random.default_rng(tokens + experts)
    logits = _router_logits(rng, tokens, experts, kind)
    ids_o, w_o, _ = oracle.router_top_k(logits, top_k)
    ids = torch.empty((tokens, top_k), dtype=torch.int32, device="cuda:0")
    w = torch.empty((tokens, top_k), dtype=torch.float32, device="cuda:0")
    say(f"router tokens={tokens} experts={experts} top_k={top_k} {kind}")
    q3x.router_top_k(dev(logits), tokens, experts, top_k, ids, w)
    ids_g, w_g = host(ids), host(w)
    bad = np.nonzero(~np.all(ids_g == ids_o, axis=1))[0]
    assert bad.size == 0, f"{bad.size} tokens select other experts, first {bad[:4]}"
    assert np.array_equal(bits(w_g), bits(w_o))


# ------------------------------------------------------------------- MoE ----

def moe_bound(gu, dn, type_, E, H, I, X, ids, wts):
    """Per-element bound for the routed sum: each slot's down product within
    TOL * ||down_row|| * ||h||, plus the first-order effect of the gate/up
    products' own TOL * ||row|| * ||x|| errors on h (double precision)."""
    gdq = dequant_numpy(gu, type_, E * 2 * I, H).reshape(E, 2 * I, H)
    ddq = dequant_numpy(dn, type_, E * H, I).reshape(E, H, I)
    T, k = ids.shape
    Xd = X.astype(np.float64)
    xn = np.linalg.norm(Xd, axis=1)
    coef = np.zeros((T, k))                      # TOL*||h|| + ||dh|| per (token, slot)
    for e in np.unique(ids):
        if e < 0 or e >= E:
            continue
        ts, ss = np.nonzero(ids == e)
        G = gdq[e].astype(np.float64)
        gu_v = Xd[ts] @ G.T
        g, u = gu_v[:, :I], gu_v[:, I:]
        sig = 1 / (1 + np.exp(-g))
        h = g * sig * u
        dg = TOL * np.linalg.norm(G[:I], axis=1)[None, :] * xn[ts, None]
        du = TOL * np.linalg.norm(G[I:], axis=1)[None, :] * xn[ts, None]
        dsilu = sig * (1 + g * (1 - sig))
        dh = np.abs(dsilu * u) * dg + np.abs(g * sig) * du + 1e-6 * np.abs(h)
        coef[ts, ss] = TOL * np.linalg.norm(h, axis=1) + np.linalg.norm(dh, axis=1)
    rown = np.linalg.norm(ddq.astype(np.float64), axis=2)          # [E, H]
    valid = (ids >= 0) & (ids < E)
    safe = np.where(valid, ids, 0)
    contrib = (np.abs(wts) * coef * valid)[:, :, None] * rown[safe]  # [T, k, H]
    return contrib.sum(axis=1)


@pytest.mark.parametrize("type_,E,H,I,top_k,tokens", [
    (Q4_0, 4, 32, 32, 2, 1), (Q4_0, 4, 32, 32, 2, 3), (Q4_0, 16, 256, 64, 4, 1), (Q4_0, 16, 256, 64, 4, 50),
    (Q8_0, 8, 512, 256, 2, 1), (Q8_0, 8, 512, 256, 2, 70), (Q4_0, 64, 2048, 512, 8, 1),
    (Q4_0, 64, 2048, 512, 8, 40),
    # 100 and 150 pairs per expert: two and three 80-pair tiles per expert,
    # the last one short
    (Q4_0, 8, 256, 64, 4, 200), (Q8_0, 4, 512, 128, 2, 300)])
def test_moe_routed_parity(type_, E, H, I, top_k, tokens):
    torch = _torch()
    rng = np.random.default_rng(E + H + I + tokens)
    gu = random_blocks(rng, type_, E * 2 * I, H)
    dn = random_blocks(rng, type_, E * H, I)
    X = rng.normal(0, 1, (tokens, H)).astype(np.float32)
    ids = np.stack([rng.choice(E, top_k, replace=False) for _ in range(tokens)]).astype(np.int32)
    wts = rng.random((tokens, top_k)).astype(np.float32)
    wts /= wts.sum(1, keepdims=True)
    want = oracle.moe_routed(gu, dn, type_, E, H, I, X, ids, wts)
    Y = torch.full((tokens, H), float("nan"), dtype=torch.float32, device="cuda:0")
    say(f"moe type={type_} E={E} H={H} I={I} k={top_k} tokens={tokens}")
    q3x.moe_routed(q3x.ExpertLinear(dev(gu), E, 2 * I, H, type_), q3x.ExpertLinear(dev(dn), E, H, I, type_),
                   dev(X), tokens, dev(ids), dev(wts), top_k, Y)
    got = host(Y)
    bound = moe_bound(gu, dn, type_, E, H, I, X, ids, wts)
    diff = np.abs(got.astype(np.float64) - want)
    assert np.all(np.isfinite(got))
    assert np.all(diff <= bound), f"{(diff > bound).sum()} outside; worst {diff.max()}"
    # accumulate
    q3x.moe_routed(q3x.ExpertLinear(dev(gu), E, 2 * I, H, type_), q3x.ExpertLinear(dev(dn), E, H, I, type_),
                   dev(X), tokens, dev(ids), dev(wts), top_k, Y, accumulate=True)
    assert np.all(np.abs(host(Y).astype(np.float64) - 2 * want) <= 2 * bound)


@pytest.mark.parametrize("type_,H,I", [(Q4_0, 256, 64),    # unaligned down rows: grouped path at 1 token
                                       (Q8_0, 256, 256)])  # aligned: fused decode kernel at 1 token
def test_moe_invalid_ids_contribute_nothing(type_, H, I):
    torch = _torch()
    E, k = 4, 3
    rng = np.random.default_rng(99 + I)
    gu = random_blocks(rng, type_, E * 2 * I, H)
    dn = random_blocks(rng, type_, E * H, I)
    for tokens in (1, 6):
        X = rng.normal(0, 1, (tokens, H)).astype(np.float32)
        ids = np.tile(np.array([2, -1, 7], np.int32), (tokens, 1))
        wts = np.tile(np.array([0.5, 0.3, 0.2], np.float32), (tokens, 1))
        want = oracle.moe_routed(gu, dn, type_, E, H, I, X, ids[:, :1], wts[:, :1])
        Y = torch.empty((tokens, H), dtype=torch.float32, device="cuda:0")
        say(f"moe invalid ids type={type_} H={H} I={I} tokens={tokens}")
        q3x.moe_routed(q3x.ExpertLinear(dev(gu), E, 2 * I, H, type_), q3x.ExpertLinear(dev(dn), E, H, I, type_),
                       dev(X), tokens, dev(ids), dev(wts), k, Y)
        bound = moe_bound(gu, dn, type_, E, H, I, X, ids[:, :1], wts[:, :1])
        assert np.all(np.abs(host(Y) - want) <= bound)


# -------------------------------------------------------------- quantize ----

@pytest.mark.parametrize("type_", [Q8_0, Q4_0])
def test_quantize_bit_exact(type_):
    torch = _torch()
    rng = np.random.default_rng(type_)
    vals = rng.normal(0, 0.02, (512, 4096)).astype(np.float32)
    vals[0, :32] = 0
    vals[1, :32] = [127.0, -127.0, 126.5, -126.5, 0.5, -0.5] + [0.0] * 26
    vals[2, :32] = np.linspace(-8, 7.5, 32)
    vals[3, :32] = 1e-30
    vals[4, :32] *= 1e4
    want = oracle.quantize(type_, vals)
    out = torch.empty(want.size, dtype=torch.uint8, device="cuda:0")
    q3x.quantize(type_, dev(vals), 512, 4096, out)
    assert np.array_equal(host(out), want)


@pytest.mark.parametrize("type_,key", [(Q8_0, "q8_0"), (Q4_0, "q4_0")])
def test_quantize_matches_reference_packer_fixture(type_, key):
    torch = _torch()
    f = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "quantizer.npz"),
                allow_pickle=False)
    vals = (f["bf16"].astype(np.uint32) << 16).view(np.float32)
    say(f"quantize fixture type={type_} blocks={vals.size // 32}")
    out = torch.empty(f[key].size, dtype=torch.uint8, device="cuda:0")
    q3x.quantize(type_, dev(vals), vals.size // 32, 32, out)
    assert np.array_equal(host(out), f[key])
