"""The routing shortcut of the decode MoE gate_up launch, checked on the CPU.

Workgroups other than the first pick the experts by e = exp(l - max) instead
of by p = e / total (the reference's order, engine.cpp:383-404) when the rule
of router_select_by_exp holds: among the top_k + 1 largest e, neighbours
inside the first top_k are equal or more than 2^-21 apart (relative), the
pair at the boundary (positions top_k - 1 and top_k) is more than 2^-21 apart
and never equal, and the smallest is at least 2^-100.  Dividing by one
positive total keeps that order, equal e stay equal, and a gap of 2^-21
survives the division's rounding (at most 2^-24 of each quotient).  A tie at
the boundary is refused because it hides the next smaller e, which can sit
one ulp below with a lower index, round to the same p and win the
reference's strict '>' scan.

This test restates the rule and the reference's selection on float32 values,
with adversarial near-ties, and requires the two selections to agree
whenever the rule holds.  The earlier rule (equality allowed at the boundary)
is kept as a planted mistake: the boundary cases below must catch it.
"""
import numpy as np

F32 = np.float32


def reference_ids(e, k):
    """engine.cpp:383-404 on given e: sequential float32 total, correctly
    rounded p = e / total, k passes of a strict '>' scan (lowest index wins)."""
    e = np.asarray(e, F32)
    total = F32(0)
    for v in e:
        total = F32(total + v)
    p = (e / total).astype(F32)
    taken = np.zeros(len(e), bool)
    ids = []
    for _ in range(k):
        best, best_i = F32(-1), -1
        for i, v in enumerate(p):
            if not taken[i] and v > best:
                best, best_i = v, i
        taken[best_i] = True
        ids.append(best_i)
    return ids


def _by_exp(e, k, boundary_tie_allowed):
    order = sorted(range(len(e)), key=lambda i: (-float(e[i]), i))[:min(k + 1, len(e))]
    vals = [float(e[i]) for i in order]
    for s, (a, b) in enumerate(zip(vals, vals[1:])):
        gap = a >= b * (1 + 2.0 ** -21)
        tie_ok = a == b and (s + 1 < k or boundary_tie_allowed)
        if not (gap or tie_ok):
            return None
    if vals[-1] < 2.0 ** -100:
        return None
    return order[:k]


def by_exp(e, k):
    """The shortcut (router_select_by_exp): k + 1 passes by e (lowest index
    among equals), the rule, and the first k ids; None where it does not hold."""
    return _by_exp(e, k, boundary_tie_allowed=False)


def by_exp_planted(e, k):
    """The same with the earlier, wrong rule: an exact tie at the boundary
    pair accepted."""
    return _by_exp(e, k, boundary_tie_allowed=True)


def test_minimal_boundary_tie_with_a_lower_index_neighbour():
    # E = 8, k = 2: e[3] = 1, e[5] = e[6] = t, e[0] = t one ulp down.  p[0]
    # rounds to p[5], and the reference takes expert 0 for the second slot.
    for t in np.linspace(0.5, 0.99, 491).astype(F32):
        e = np.full(8, F32(0.01), F32)
        e[3] = 1
        e[5] = e[6] = t
        e[0] = np.nextafter(t, F32(0))
        want = reference_ids(e, 2)
        if want[1] != 0:
            continue                       # this t's quotients stayed apart
        assert want == [3, 0]
        assert by_exp_planted(e, 2) == [3, 5]   # the earlier rule is wrong here
        assert by_exp(e, 2) is None             # the rule refuses it
        return
    raise AssertionError("no t made p[0] round to p[5]")


def test_advisor_case_k1():
    # e[5] = e[7] = 1, e[2] = nextafter(1, 0), the rest 0.1 / E; k = 1.
    E = 8
    e = np.full(E, F32(0.1 / E), F32)
    e[5] = e[7] = 1
    e[2] = np.nextafter(F32(1), F32(0))
    assert reference_ids(e, 1) == [2]
    assert by_exp_planted(e, 1) == [5]
    assert by_exp(e, 1) is None


def test_planted_boundary_sweep():
    """Ties across the top_k boundary with a lower-index expert one to a few
    ulps below: the rule never gives a wrong id, and the earlier rule does
    (so these cases bite)."""
    rng = np.random.default_rng(7)
    planted_wrong = 0
    for trial in range(4000):
        E = int(rng.choice([8, 64, 256]))
        k = int(rng.integers(1, 9))
        if k + 2 > E:
            continue
        e = np.exp(rng.normal(0, 1, E).astype(F32)).astype(F32)
        e /= F32(e.max())
        order = np.argsort(-e, kind="stable")
        # the tie spans positions k-1 and k; a lower index joins one ulp below
        a = int(min(order[k - 1], order[k]))
        b = int(max(order[k - 1], order[k]))
        e[b] = e[a]
        below = [int(i) for i in order[k + 1:] if i < a]
        if not below:
            continue
        j = below[0]
        steps = int(rng.integers(1, 4))
        v = e[a]
        for _ in range(steps):
            v = np.nextafter(v, F32(0))
        if not float(v) < float(e[order[k - 2]] if k >= 2 else np.inf):
            continue
        e[j] = v
        want = reference_ids(e, k)
        got = by_exp(e, k)
        assert got is None or got == want, (E, k)
        old = by_exp_planted(e, k)
        if old is not None and old != want:
            planted_wrong += 1
    assert planted_wrong > 50


def test_shortcut_agrees_with_the_reference_wherever_it_applies():
    rng = np.random.default_rng(2026)
    applied = rejected = 0
    for trial in range(3000):
        E = int(rng.choice([8, 64, 256]))
        k = int(rng.integers(1, 9))
        logits = rng.normal(0, rng.choice([0.5, 2.0, 8.0]), E).astype(F32)
        e = np.exp(logits - logits.max()).astype(F32)
        top = np.argsort(-e, kind="stable")[:k + 1]
        kind = trial % 6
        if kind == 1:    # exact ties around the boundary
            e[top[-1]] = e[top[-2]]
        elif kind == 2:  # neighbours one ulp apart
            e[top[1]] = np.nextafter(e[top[0]], F32(0))
        elif kind == 3:  # a few ulps apart
            e[top[-1]] = e[top[-2]] * F32(1 - 3 * 2.0 ** -24)
        elif kind == 4:  # just past the rule's gap
            e[top[1]] = F32(float(e[top[0]]) / (1 + 2.0 ** -20))
        elif kind == 5 and k >= 2:  # exact ties inside the first k (allowed)
            e[top[1]] = e[top[0]]
        want = reference_ids(e, k)
        got = by_exp(e, k)
        if got is None:
            rejected += 1
            continue
        applied += 1
        assert got == want, (E, k, kind)
    assert applied > 1500 and rejected > 300
