"""The routing shortcut of the decode MoE gate_up launch, checked on the CPU.

Workgroups other than the first pick the experts by e = exp(l - max) instead
of by p = e / total (the reference's order, engine.cpp:383-404) when every two
neighbours among the top_k + 1 largest e are equal or more than 2^-21 apart
(relative) and the smallest is at least 2^-100: dividing by one positive total
keeps that order, equal e stay equal, and a gap of 2^-21 survives the
division's rounding (at most 2^-24 of each quotient).  This test restates the
rule and the reference's selection on float32 values, with adversarial
near-ties, and requires the two selections to agree whenever the rule holds.
"""
import numpy as np

F32 = np.float32


def reference_ids(e, k):
    """engine.cpp:383-404 on given e: sequential float32 total, correctly
    rounded p = e / total, k passes of a strict '>' scan (lowest index wins)."""
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


def by_exp(e, k):
    """The shortcut: k + 1 passes by e (lowest index among equals), the rule,
    and the first k ids; None where the rule does not hold."""
    order = sorted(range(len(e)), key=lambda i: (-float(e[i]), i))[:min(k + 1, len(e))]
    vals = [float(e[i]) for i in order]
    for a, b in zip(vals, vals[1:]):
        if not (a == b or a >= b * (1 + 2.0 ** -21)):
            return None
    if vals[-1] < 2.0 ** -100:
        return None
    return order[:k]


def test_shortcut_agrees_with_the_reference_wherever_it_applies():
    rng = np.random.default_rng(2026)
    applied = rejected = 0
    for trial in range(3000):
        E = int(rng.choice([8, 64, 256]))
        k = int(rng.integers(1, 9))
        logits = rng.normal(0, rng.choice([0.5, 2.0, 8.0]), E).astype(F32)
        e = np.exp(logits - logits.max()).astype(F32)
        top = np.argsort(-e, kind="stable")[:k + 1]
        kind = trial % 5
        if kind == 1:    # exact ties around the boundary
            e[top[-1]] = e[top[-2]]
        elif kind == 2:  # neighbours one ulp apart
            e[top[1]] = np.nextafter(e[top[0]], F32(0))
        elif kind == 3:  # a few ulps apart
            e[top[-1]] = e[top[-2]] * F32(1 - 3 * 2.0 ** -24)
        elif kind == 4:  # just past the rule's gap
            e[top[1]] = F32(float(e[top[0]]) / (1 + 2.0 ** -20))
        want = reference_ids(e, k)
        got = by_exp(e, k)
        if got is None:
            rejected += 1
            continue
        applied += 1
        assert got == want, (E, k, kind)
    assert applied > 1500 and rejected > 300
