"""Float64 sampling law and speculative verification on the GPU
(qwen3_dspark_amd.sampling: dspark_logit_row_stats, dspark_spec_verify,
dspark_logits_to_probs, dspark_sample_rows) against the oracle
(oracle/sampling.py, pinned by exact rational branch enumeration in
tests/test_sampling_oracle.py): integer outcomes must be identical."""
import itertools
import math
from fractions import Fraction as F

import numpy as np
import pytest
import torch

from helpers import SEED
from oracle import sampling as oracle
from test_sampling_oracle import branches, expected_rounds

pytestmark = pytest.mark.gpu
DEV = torch.device('cuda:0')


def say(*a):
    print(*a, flush=True)


def as_tuple(r):
    return (tuple(int(t) for t in r.tokens.tolist()), r.accepted_draft_tokens, r.rejected_index, r.extra_token_kind,
            r.stop_reason)


def logit_row(p):
    """float64 logits whose law is p: log p, with -1000 (exp underflows to
    exactly 0) for zero mass."""
    return [math.log(float(x)) if x else -1000.0 for x in p]


def run_batch(cases, stops):
    """cases: [(tokens, q_rows, p_rows, tape, budget)] -> device rounds."""
    from qwen3_dspark_amd.sampling import verify_proposals
    vocab = len(cases[0][2][0])
    logits = torch.tensor([logit_row(row) for _, _, p, _, _ in cases for row in p], dtype=torch.float32)
    toks = torch.tensor([t for c in cases for t in c[0]], dtype=torch.long)
    q = torch.tensor([[float(x) for x in row] for c in cases for row in c[1]], dtype=torch.float64).reshape(-1, vocab)
    uni = []
    for tokens, _, _, tape, _ in cases:
        row = [float(u) for u in tape] + [0.0] * (len(tokens) + 1 - len(tape))
        uni += row
    return verify_proposals(logits.to(DEV), toks.to(DEV), q.to(DEV), torch.tensor(uni, dtype=torch.float64).to(DEV),
                            counts=[len(c[0]) for c in cases], temperature=1.0,
                            max_new_tokens=[c[4] for c in cases], eos_ids=stops)


def test_every_branch_on_the_device():
    """Vocabulary 3: p on the quarter simplex given as logits log p, q on the
    quarter simplex, one or two proposed tokens, budgets 0-2, with and
    without EOS; one request per branch, each driven by an interior point of
    its uniform intervals, must land on exactly its branch."""
    simplex = [tuple(F(x, 4) for x in r) for r in itertools.product(range(5), repeat=3) if sum(r) == 4]
    for stops in ((), (1,)):
        cases, expect = [], []
        for p0, q0 in itertools.product(simplex, repeat=2):
            for t, _, _ in branches(q0):
                for budget in (0, 1, 2):
                    for exp, _, tape in expected_rounds((t,), (q0,), (p0, p0), budget, stops):
                        cases.append(((t,), (q0,), (p0, p0), tape, budget))
                        expect.append(exp)
        # two-token proposals over a prefix-dependent target
        p = lambda prefix: (F(1, 4), F(1, 2), F(1, 4)) if not prefix or prefix[-1] else (F(1, 2), F(1, 4), F(1, 4))
        q = lambda prefix: (F(1, 3), F(1, 3), F(1, 3)) if not prefix else (F(1, 2), F(1, 4), F(1, 4))
        for tokens in itertools.product(range(3), repeat=2):
            rows_q = tuple(q(tokens[:j]) for j in range(2))
            rows_p = tuple(p(tokens[:j]) for j in range(3))
            for budget in (1, 2, 3):
                for exp, _, tape in expected_rounds(tokens, rows_q, rows_p, budget, stops):
                    cases.append((tokens, rows_q, rows_p, tape, budget))
                    expect.append(exp)
        got = run_batch(cases, stops)
        assert [as_tuple(r) for r in got] == expect
        assert [r.draws for r in got] == [len(c[3]) for c in cases]
        say(f'[sampling] {len(cases)} branches (stops {stops}) identical to the enumeration')


def test_full_vocabulary_batch_against_oracle():
    """64 requests x 7 proposed tokens over the 151,936-token vocabulary:
    draft laws from draft logits (target logits + noise), tokens drawn on
    the device, target bf16 logits, temperature 0.8; every integer outcome
    and draw count against the oracle on the same logits and uniforms."""
    from qwen3_dspark_amd.sampling import logits_to_probabilities, sample_categorical, verify_proposals
    V, R, N, T = 151936, 64, 7, 0.8
    gen = torch.Generator(device=DEV).manual_seed(SEED)
    target = (torch.randn(R * (N + 1), V, generator=gen, device=DEV) * 2.0).to(torch.bfloat16)
    rows = torch.arange(R * (N + 1), device=DEV).reshape(R, N + 1)[:, :N].reshape(-1)
    noise = torch.randn(R * N, V, generator=gen, device=DEV) * torch.rand(R * N, 1, generator=gen, device=DEV)
    draft_logits = target[rows].float() + noise
    q = logits_to_probabilities(draft_logits, T)
    tokens = sample_categorical(q, torch.rand(R * N, generator=gen, device=DEV, dtype=torch.float64))
    uniforms = torch.rand(R * (N + 1), generator=gen, device=DEV, dtype=torch.float64)
    budgets = [int(b) for b in torch.randint(0, 10, (R,), generator=torch.Generator().manual_seed(SEED))]
    stops = (5, 151935)
    got = verify_proposals(target, tokens, q, uniforms, counts=[N] * R, temperature=T, max_new_tokens=budgets,
                           eos_ids=stops)
    torch.cuda.synchronize()
    p_h = oracle.logits_to_probabilities(target.float().cpu().numpy(), T)
    q_h, t_h, u_h = q.cpu().numpy(), tokens.cpu().numpy(), uniforms.cpu().numpy()
    kinds = {}
    for r in range(R):
        ref = oracle.verify_proposal(t_h[N * r:N * r + N], q_h[N * r:N * r + N], p_h[(N + 1) * r:(N + 1) * (r + 1)],
                                     u_h[(N + 1) * r:(N + 1) * (r + 1)], max_new_tokens=budgets[r], eos_ids=stops)
        assert as_tuple(got[r]) == (ref.tokens, ref.accepted_draft_tokens, ref.rejected_index, ref.extra_token_kind,
                                    ref.stop_reason), r
        assert got[r].draws == ref.draws
        kinds[got[r].extra_token_kind] = kinds.get(got[r].extra_token_kind, 0) + 1
    say(f'[sampling] 64 requests identical to the oracle; outcomes {kinds}, '
        f'accepted {sum(r.accepted_draft_tokens for r in got)}')
    assert kinds.get('residual', 0) and kinds.get('bonus', 0)


def test_laws_and_row_draws_against_oracle():
    from qwen3_dspark_amd.sampling import logits_to_probabilities, sample_categorical
    gen = torch.Generator(device=DEV).manual_seed(SEED + 1)
    for V, T in ((151936, 1.0), (1000, 0.3), (7, 2.5)):
        logits = (torch.randn(9, V, generator=gen, device=DEV) * 3).to(torch.bfloat16)
        probs = logits_to_probabilities(logits, T)
        ref = oracle.logits_to_probabilities(logits.float().cpu().numpy(), T)
        np.testing.assert_allclose(probs.cpu().numpy(), ref, rtol=1e-12, atol=1e-300)
        assert np.abs(probs.sum(-1).cpu().numpy() - 1).max() <= 1e-12
        u = torch.rand(9, generator=gen, device=DEV, dtype=torch.float64)
        got = sample_categorical(probs, u).cpu().tolist()
        assert got == [oracle.sample_categorical(row, x) for row, x in zip(ref, u.cpu().tolist())]
    # zero-mass entries are never drawn; u beyond the running sum takes the last positive index
    probs = torch.tensor([[0.5, 0.0, 0.5, 0.0], [0.0, 1.0, 0.0, 0.0]], dtype=torch.float64, device=DEV)
    u = torch.tensor([0.5, 0.999999], dtype=torch.float64, device=DEV)
    assert sample_categorical(probs, u).tolist() == [2, 1]
    bad = torch.zeros(2, 8, device=DEV)
    bad[1, 3] = float('inf')
    with pytest.raises(ValueError, match='finite'):
        logits_to_probabilities(bad, 1.0)


def test_verification_errors_and_stops():
    from qwen3_dspark_amd.sampling import verify_proposals
    V = 4
    logits = torch.tensor([[0.0, 1.0, 2.0, 3.0]] * 2, device=DEV)
    q = torch.tensor([[0.25] * 4], dtype=torch.float64, device=DEV)
    u = torch.tensor([0.1, 0.2], dtype=torch.float64, device=DEV)

    def call(tok, q_=q, u_=u, budget=2, stops=(), lg=logits):
        return verify_proposals(lg, torch.tensor([tok], device=DEV), q_, u_, counts=[1], temperature=1.0,
                                max_new_tokens=[budget], eos_ids=stops)[0]
    with pytest.raises(ValueError, match='outside vocabulary'):
        call(4)
    with pytest.raises(ValueError, match='zero mass'):
        call(1, q_=torch.tensor([[0.5, 0.0, 0.5, 0.0]], dtype=torch.float64, device=DEV))
    with pytest.raises(ValueError, match=r'\[0,1\)'):
        call(3, u_=torch.tensor([1.0, 0.2], dtype=torch.float64, device=DEV))
    bad = logits.clone()
    bad[1, 0] = float('nan')
    with pytest.raises(ValueError, match='finite'):
        call(3, lg=bad)
    with pytest.raises(ValueError, match='temperature'):
        verify_proposals(logits, torch.tensor([3], device=DEV), q, u, counts=[1], temperature=0.0, max_new_tokens=[2])
    r = call(3, budget=0)
    assert (r.tokens.tolist(), r.stop_reason, r.draws) == ([], 'budget', 0)
    r = call(3, stops=(3,))                  # p[3] > q[3]: accepted, then EOS stops without a bonus draw
    assert (r.tokens.tolist(), r.accepted_draft_tokens, r.stop_reason, r.draws) == ([3], 1, 'eos', 1)
    r = call(3, budget=1)
    assert (r.tokens.tolist(), r.stop_reason, r.draws) == ([3], 'budget', 1)


def test_laws_and_verification_outside_the_corrected_quotient_range():
    """The sampling kernels divide by T through a corrected reciprocal
    product for T in [2^-100, 2^100] and by IEEE division outside it: at
    temperatures on both sides of each bound, the laws against the oracle
    to 1e-12 and every integer outcome of a verification batch identical.
    The fp32 logits are scaled by T so that the laws stay spread."""
    from qwen3_dspark_amd.sampling import logits_to_probabilities, sample_categorical, verify_proposals
    V, R, N = 2000, 8, 3
    gen = torch.Generator(device=DEV).manual_seed(SEED + 7)
    rows = torch.arange(R * (N + 1), device=DEV).reshape(R, N + 1)[:, :N].reshape(-1)
    for T in (2.0 ** -101, 2.0 ** -99, 2.0 ** 99, 3 * 2.0 ** 100, 2.0 ** 101):
        say(f'[sampling] temperature {T!r}')
        base = torch.randn(R * (N + 1), V, generator=gen, device=DEV, dtype=torch.float64) * 2.0
        target = (base * T).float()
        draft_logits = (target[rows].double() + torch.randn(R * N, V, generator=gen, device=DEV,
                                                            dtype=torch.float64) * T).float()
        q = logits_to_probabilities(draft_logits, T)
        np.testing.assert_allclose(q.cpu().numpy(), oracle.logits_to_probabilities(draft_logits.cpu().numpy(), T),
                                   rtol=1e-12, atol=1e-300)
        tokens = sample_categorical(q, torch.rand(R * N, generator=gen, device=DEV, dtype=torch.float64))
        uniforms = torch.rand(R * (N + 1), generator=gen, device=DEV, dtype=torch.float64)
        got = verify_proposals(target, tokens, q, uniforms, counts=[N] * R, temperature=T,
                               max_new_tokens=[N + 1] * R)
        p_h = oracle.logits_to_probabilities(target.cpu().numpy(), T)
        q_h, t_h, u_h = q.cpu().numpy(), tokens.cpu().numpy(), uniforms.cpu().numpy()
        for r in range(R):
            ref = oracle.verify_proposal(t_h[N * r:N * r + N], q_h[N * r:N * r + N],
                                         p_h[(N + 1) * r:(N + 1) * (r + 1)], u_h[(N + 1) * r:(N + 1) * (r + 1)],
                                         max_new_tokens=N + 1)
            assert as_tuple(got[r]) == (ref.tokens, ref.accepted_draft_tokens, ref.rejected_index,
                                        ref.extra_token_kind, ref.stop_reason), (T, r)
            assert got[r].draws == ref.draws
