"""Float64 sampling law and speculative verification, restated for the CPU
oracle (test infrastructure only).

Follows dspark_qwen/tensor_sampling.py:
  logits_to_probabilities (:37-48)  law = softmax(logits / T) in float64,
                                     normalised once more by its own sum
  sample_categorical (:69-76)        searchsorted(cumsum(law), u, right=True),
                                     else the last index of positive mass
  residual_distribution (:79-89)     (p - q)+ / sum, zero mass is an error
  verify_proposal (:114-162)         accept draft token t_j iff u < min(1, p_j[t_j] / q_j[t_j]);
                                     first rejection -> residual draw,
                                     all accepted -> bonus draw from the last
                                     row; EOS / budget stop after a token
The random source is a tape: draws are taken from `uniforms` in order, as
the reference takes them from its rng; `draws` counts how many were used.
"""
from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class Round:
    tokens: tuple
    accepted_draft_tokens: int
    rejected_index: object
    extra_token_kind: object
    stop_reason: str
    draws: int


def logits_to_probabilities(logits, temperature):
    x = np.asarray(logits, np.float64)
    if not np.isfinite(x).all():
        raise ValueError('Expected finite floating logits and a nonempty vocabulary')
    scaled = x / float(temperature)
    if not np.isfinite(scaled).all():
        raise ValueError('Temperature scaling overflowed')
    e = np.exp(scaled - scaled.max(axis=-1, keepdims=True))
    w = e / e.sum(axis=-1, keepdims=True)
    return w / w.sum(axis=-1, keepdims=True)


def sample_categorical(probs, u):
    probs = np.asarray(probs, np.float64)
    if not 0 <= u < 1:
        raise ValueError('RNG must yield a float64 scalar in [0,1)')
    index = int(np.searchsorted(np.cumsum(probs), u, side='right'))
    return index if index < probs.size else int(np.nonzero(probs > 0)[0][-1])


def residual_distribution(p, q):
    positive = np.maximum(np.asarray(p, np.float64) - np.asarray(q, np.float64), 0.0)
    mass = positive.sum()
    if not mass > 0:
        raise ValueError('Zero residual mass: rejection is impossible for identical laws')
    return positive / mass


def verify_proposal(tokens, q, p, uniforms, *, max_new_tokens, eos_ids=()):
    """tokens [n]; q [n, V] draft laws; p [n+1, V] target laws; uniforms: the
    tape of draws (at least as many as are used)."""
    tokens = [int(t) for t in tokens]
    q = np.asarray(q, np.float64).reshape(len(tokens), -1) if tokens else np.zeros((0, np.shape(p)[-1]))
    p = np.asarray(p, np.float64)
    if p.shape[0] != len(tokens) + 1:
        raise ValueError('Require [n] long tokens, [n,V] q and [n+1,V] p on one device')
    vocab = p.shape[-1]
    if any(not 0 <= t < vocab for t in tokens):
        raise ValueError('Proposal token outside vocabulary')
    if any(q[j, t] == 0 for j, t in enumerate(tokens)):
        raise ValueError('Proposal token has zero mass under its actual sampling law')
    stops = frozenset(int(e) for e in eos_ids)
    tape = iter(uniforms)
    used = 0

    def draw():
        nonlocal used
        used += 1
        u = float(next(tape))
        if not 0 <= u < 1:
            raise ValueError('RNG must yield a float64 scalar in [0,1)')
        return u

    emitted = []

    def reason(token):
        if token in stops:
            return 'eos'
        return 'budget' if len(emitted) == max_new_tokens else 'round_complete'

    if max_new_tokens == 0:
        return Round((), 0, None, None, 'budget', 0)
    for j, token in enumerate(tokens):
        alpha = min(p[j, token] / q[j, token], 1.0)
        if draw() >= alpha:
            replacement = sample_categorical(residual_distribution(p[j], q[j]), draw())
            emitted.append(replacement)
            return Round(tuple(emitted), j, j, 'residual', reason(replacement), used)
        emitted.append(token)
        stop = reason(token)
        if stop != 'round_complete':
            return Round(tuple(emitted), j + 1, None, None, stop, used)
    bonus = sample_categorical(p[-1], draw())
    emitted.append(bonus)
    return Round(tuple(emitted), len(tokens), None, 'bonus', reason(bonus), used)
