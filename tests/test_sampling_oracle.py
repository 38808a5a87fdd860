"""CPU pins of the sampling oracle (oracle/sampling.py).

* The literal cases of the reference's own tests
  (tests/test_tensor_sampling.py:73-113).
* Exact rational enumeration: every accept / reject / residual / bonus /
  EOS / budget branch of a verification, each with the probability of its
  uniform interval, enumerated with Fractions independently of the oracle.
  The oracle, driven by an interior point of each branch's intervals, must
  return exactly that branch; and the emitted law must be the target's
  (speculative sampling's defining property: one verified token is
  distributed as p whatever q is).
"""
import itertools
from collections import defaultdict
from fractions import Fraction as F

import numpy as np
import pytest
import torch

from oracle import sampling


def branches(row):
    """(token, mass, interior point) of a categorical draw from `row`."""
    start = F(0)
    for token, mass in enumerate(row):
        if mass:
            yield token, mass, start + mass / 2
        start += mass


def expected_rounds(tokens, q, p, budget, stops):
    """(round tuple, mass, tape) for every verification branch."""
    tokens = tuple(tokens)
    if budget == 0:
        yield ((), 0, None, None, 'budget'), F(1), ()
        return

    def reason(out, token):
        return 'eos' if token in stops else ('budget' if len(out) == budget else 'round_complete')

    def walk(j, tape, mass):
        if j == len(tokens):
            for v, m, mid in branches(p[j]):
                out = tokens[:j] + (v,)
                yield (out, j, None, 'bonus', reason(out, v)), mass * m, tape + (mid,)
            return
        t = tokens[j]
        alpha = min(F(1), p[j][t] / q[j][t])
        if alpha > 0:
            out = tokens[:j + 1]
            if t in stops or len(out) == budget:
                yield (out, j + 1, None, None, 'eos' if t in stops else 'budget'), mass * alpha, tape + (alpha / 2,)
            else:
                yield from walk(j + 1, tape + (alpha / 2,), mass * alpha)
        if alpha < 1:
            positive = [max(a - b, F(0)) for a, b in zip(p[j], q[j])]
            total = sum(positive)
            for v, m, mid in branches([x / total for x in positive]):
                out = tokens[:j] + (v,)
                yield (out, j, j, 'residual', reason(out, v)), mass * (1 - alpha) * m, tape + ((1 + alpha) / 2, mid)

    yield from walk(0, (), F(1))


def run_oracle(tokens, q, p, tape, budget, stops):
    r = sampling.verify_proposal(tokens, [[float(x) for x in row] for row in q], [[float(x) for x in row] for row in p],
                                 [float(u) for u in tape], max_new_tokens=budget, eos_ids=stops)
    assert r.draws == len(tape)
    return (r.tokens, r.accepted_draft_tokens, r.rejected_index, r.extra_token_kind, r.stop_reason)


def test_reference_literal_cases():
    # tests/test_tensor_sampling.py:90-113
    assert sampling.sample_categorical([0.5, 0, 0.5], 0.5) == 2
    r = sampling.verify_proposal([0], [[1, 0]], [[0.5, 0.5], [1, 0]], [0.5, 0], max_new_tokens=2)
    assert r.rejected_index == 0 and r.tokens == (1,)
    with pytest.raises(ValueError):
        sampling.verify_proposal([1], [[1, 0]], [[0, 1], [1, 0]], [], max_new_tokens=2)
    for bad in (-1.0, 1.0, np.inf, np.nan):
        with pytest.raises(ValueError):
            sampling.sample_categorical([1, 0], bad)
    for value in (np.nan, np.inf, -np.inf):
        with pytest.raises(ValueError):
            sampling.logits_to_probabilities([value, 1], 1)
    # :73-88 probability adapter, tiny residual, underflowed support
    for dtype in (torch.bfloat16, torch.float32, torch.float64):
        logits = torch.tensor([[0.25, -0.75, 1.5]], dtype=dtype)
        expect = (logits.double() / 0.7).softmax(-1)
        expect /= expect.sum(-1, keepdim=True)
        np.testing.assert_allclose(sampling.logits_to_probabilities(logits.double().numpy(), 0.7), expect.numpy(),
                                   rtol=1e-15, atol=0)
    delta = 2 ** -40
    assert np.array_equal(sampling.residual_distribution([0.5 + delta, 0.5 - delta], [0.5, 0.5]), [1.0, 0.0])
    with pytest.raises(ValueError):
        sampling.residual_distribution([0.5, 0.5], [0.5, 0.5])
    assert np.array_equal(sampling.logits_to_probabilities([1000, -1000], 1), [1.0, 0.0])


def test_every_branch_and_the_target_law_on_the_quarter_simplex():
    """Vocabulary 3, all (p, q) on the quarter simplex, one proposed token
    drawn from q, budgets 1 and 2, with and without EOS."""
    simplex = [tuple(F(x, 4) for x in r) for r in itertools.product(range(5), repeat=3) if sum(r) == 4]
    cases = 0
    for p0, q0 in itertools.product(simplex, repeat=2):
        for budget, stops in ((1, ()), (2, ()), (2, (1,))):
            law = defaultdict(F)
            for t, qm, qmid in branches(q0):
                # the proposal draw itself, as the oracle's categorical sampler sees it
                assert sampling.sample_categorical([float(x) for x in q0], float(qmid)) == t
                total = F(0)
                for expect, mass, tape in expected_rounds((t,), (q0,), (p0, p0), budget, stops):
                    assert run_oracle((t,), (q0,), (p0, p0), tape, budget, stops) == expect
                    law[expect[0][0]] += qm * mass
                    total += mass
                    cases += 1
                assert total == 1
            assert dict(law) == {i: v for i, v in enumerate(p0) if v}
    assert cases > 1000


def test_multitoken_prefix_dependent_laws_with_eos_and_budget():
    p = lambda prefix: (F(1, 4), F(3, 4)) if not prefix or prefix[-1] else (F(3, 4), F(1, 4))
    q = lambda prefix: (F(1, 2), F(1, 2)) if not prefix else (F(3, 4), F(1, 4))
    for length, budget, stops in itertools.product((0, 1, 2), (0, 1, 2, 3), ((), (1,))):
        for tokens in itertools.product(range(2), repeat=length):
            rows_q = tuple(q(tokens[:j]) for j in range(length))
            rows_p = tuple(p(tokens[:j]) for j in range(length + 1))
            total = F(0)
            for expect, mass, tape in expected_rounds(tokens, rows_q, rows_p, budget, stops):
                assert run_oracle(tokens, rows_q, rows_p, tape, budget, stops) == expect
                total += mass
            assert total == 1


def test_planted_mistake_fails_the_law():
    """A residual that forgets to subtract q (drawing from p on rejection)
    breaks the emitted law, so the law check above pins that term."""
    p0, q0 = (F(1, 4), F(1, 4), F(1, 2)), (F(1, 2), F(1, 4), F(1, 4))
    law = defaultdict(F)
    for t, qm, _ in branches(q0):
        alpha = min(F(1), p0[t] / q0[t])
        law[t] += qm * alpha
        for v, m, _ in branches(p0):          # wrong: p instead of (p - q)+
            law[v] += qm * (1 - alpha) * m
    assert dict(law) != {i: v for i, v in enumerate(p0) if v}
