"""Float64 sampling law and speculative verification on MI355X: the consumer
of the verification round's output (dspark_qwen/tensor_sampling.py and the
per-request loop of packed_sampling.py:250-259).

    logits = lm_head(hidden)                   TargetHead: hipBLASLt, bf16
    p = softmax(logits / T)  (float64)         never materialised for verification
    verify_proposals(...)                      every request of the batch at once:
        accept t_j iff u < min(1, p_j[t_j] / q_j[t_j]); first rejection emits a
        draw from (p_j - q_j)+, a fully accepted block a bonus draw from the
        last row; EOS and the budget stop early

Four launches for the whole batch: per-(row, chunk) max / sum-of-exp
statistics of the logits; one lane per request for the accept / reject
decisions; then the final categorical draws (a float64 CDF over the
vocabulary as 256 segment sums per draw from a wide grid, and one workgroup
per draw that scans them and walks the segment holding u).

Random numbers: the reference draws float64 uniforms one by one from a
per-request rng (TensorRandom.uniform).  Here the caller passes them: request
r's draws, in the reference's order, as a row of at least n_r + 1 values
(n_r accept tests at most, then one categorical draw).  Each result reports
how many it used, so a caller replaying a reference rng advances it by
exactly that many.  Given the same draws the integer outcomes are the
reference's; its probabilities are float64 sums taken in another order, so a
draw within about 1e-16 of a decision boundary may fall the other way.

Checks that would read every q row (the draft laws' sums) are the draft's
responsibility here; the token ranges, q at each proposed token, finite
logits (and temperature overflow) and the uniforms are checked on the device
and raise ValueError with the reference's messages after one device read.
"""
import math
from dataclasses import dataclass
from numbers import Real

import torch

from . import _native
from ._device import Workspace, require_gfx950, upload

PROBABILITY_POLICY = 'float64_softmax_normalize_cdf_v1'
_EXTRA = {0: None, 1: 'residual', 2: 'bonus'}
_STOP = {0: 'round_complete', 1: 'eos', 2: 'budget'}
_ERRORS = {
    1: 'Proposal token outside vocabulary',
    2: 'Proposal token has zero mass under its actual sampling law',
    3: 'Expected finite floating logits and a nonempty vocabulary',
    4: 'Zero residual mass: rejection is impossible for identical laws',
    5: 'RNG must yield a float64 scalar in [0,1)',
    6: 'At most 255 proposed tokens per request',
}
MAX_PROPOSAL = 255


def validate_temperature(temperature):
    """tensor_sampling.py:18-22."""
    if (isinstance(temperature, bool) or not isinstance(temperature, Real) or not math.isfinite(temperature)
            or temperature <= 0):
        raise ValueError('temperature must be finite and strictly positive')
    return float(temperature)


@dataclass(frozen=True)
class VerifiedRound:
    """tensor_sampling.TensorRound plus the number of uniforms used."""
    tokens: torch.Tensor
    accepted_draft_tokens: int
    rejected_index: object
    extra_token_kind: object
    stop_reason: str
    draws: int


class TargetHead:
    """The target's LM head [vocab, hidden] (bf16): a plain GEMM on hipBLASLt."""

    def __init__(self, weight):
        self.device = require_gfx950(weight.device)
        if weight.ndim != 2 or weight.dtype != torch.bfloat16:
            raise ValueError('LM head weight must be bf16 [vocab, hidden]')
        self.weight = weight.detach().contiguous()
        self.vocab, self.hidden = self.weight.shape

    def __call__(self, hidden):
        if hidden.ndim != 2 or hidden.shape[1] != self.hidden or hidden.device != self.device:
            raise ValueError('Expected [rows, hidden] hidden states on the head device')
        return torch.nn.functional.linear(hidden.to(torch.bfloat16), self.weight)


_WORKSPACES = {}


def _draw_workspace(device, jobs):
    ws = _WORKSPACES.get(device)
    if ws is None:
        ws = _WORKSPACES[device] = Workspace(device)
    return ws.get(_native.load().dspark_draw_workspace_bytes(jobs))


def _logits(logits):
    if (not isinstance(logits, torch.Tensor) or logits.ndim != 2 or logits.shape[0] < 1 or logits.shape[1] < 1
            or logits.dtype not in (torch.bfloat16, torch.float32) or logits.stride(1) != 1):
        raise ValueError('Expected bf16 or fp32 logits [rows, vocab] with contiguous rows')
    return 0 if logits.dtype == torch.bfloat16 else 1


def _row_stats(logits, temperature):
    dev = require_gfx950(logits.device)
    dtype = _logits(logits)
    rows, vocab = logits.shape
    lib = _native.load()
    stats = torch.empty(lib.dspark_row_stats_bytes(rows, vocab) // 8, dtype=torch.float64, device=dev)
    bad = torch.zeros(rows, dtype=torch.int32, device=dev)
    _native.call('dspark_logit_row_stats', logits.data_ptr(), dtype, rows, vocab, logits.stride(0), temperature,
                 stats.data_ptr(), bad.data_ptr(), _native.stream_handle(dev))
    return stats, bad


@torch.no_grad()
def logits_to_probabilities(logits, temperature):
    """The float64 law of every row (tensor_sampling.py:37-48), materialised."""
    temperature = validate_temperature(temperature)
    stats, bad = _row_stats(logits, temperature)
    rows, vocab = logits.shape
    if rows > 65535:
        raise ValueError('At most 65535 rows per call')
    probs = torch.empty((rows, vocab), dtype=torch.float64, device=logits.device)
    _native.call('dspark_logits_to_probs', logits.data_ptr(), _logits(logits), rows, vocab, logits.stride(0),
                 temperature, stats.data_ptr(), probs.data_ptr(), _native.stream_handle(logits.device))
    if int(bad.max().item()):
        raise ValueError(_ERRORS[3])
    return probs


@torch.no_grad()
def sample_categorical(probs, uniforms):
    """One draw per row of float64 laws probs [rows, V] with uniforms [rows]
    (tensor_sampling.py:69-76): the first index whose running sum exceeds u,
    else the last index of positive mass.  Laws and uniforms are the caller's
    (valid laws, u in [0, 1))."""
    dev = require_gfx950(probs.device)
    if (probs.dtype != torch.float64 or probs.ndim != 2 or not probs.is_contiguous() or uniforms.dtype != torch.float64
            or uniforms.shape != (probs.shape[0],) or uniforms.device != dev):
        raise ValueError('Expected contiguous float64 laws [rows, V] and float64 uniforms [rows] on one device')
    out = torch.empty(probs.shape[0], dtype=torch.long, device=dev)
    ws = _draw_workspace(dev, probs.shape[0])
    _native.call('dspark_sample_rows', probs.data_ptr(), probs.shape[0], probs.shape[1],
                 uniforms.contiguous().data_ptr(), out.data_ptr(), ws.data_ptr(), ws.numel(), _native.stream_handle(dev))
    return out


@torch.no_grad()
def verify_proposals(logits, tokens, draft_probs, uniforms, *, counts, temperature, max_new_tokens, eos_ids=()):
    """Verify every request's proposal in one pass (tensor_sampling.py:114-162
    per request).

    logits: [sum(n_r + 1), V] target logits, request-major (row j of request r
        predicts the token after its context plus tokens[:j]);
    tokens: [sum n_r] int64 proposed tokens, request-major;
    draft_probs: [sum n_r, V] float64, the laws each token was drawn from;
    uniforms: [sum(n_r + 1)] float64, request r's draws in the reference's
        order starting at row offset sum_{i<r}(n_i + 1);
    counts: n_r per request; max_new_tokens: remaining budget per request.
    Returns one VerifiedRound per request."""
    temperature = validate_temperature(temperature)
    dev = require_gfx950(logits.device)
    dtype = _logits(logits)
    counts = [int(n) for n in counts]
    budgets = [int(b) for b in max_new_tokens]
    if not counts or len(budgets) != len(counts) or any(n < 0 for n in counts):
        raise ValueError('One nonnegative proposal length and budget per request required')
    if max(counts) > MAX_PROPOSAL:
        raise ValueError(_ERRORS[6])
    if any(type(b) is not int or b < 0 for b in max_new_tokens):
        raise ValueError('max_new_tokens must be a nonnegative integer')
    rows, vocab = logits.shape
    n_draft = sum(counts)
    if rows != n_draft + len(counts):
        raise ValueError('Require [n] long tokens, [n,V] q and [n+1,V] p on one device')
    if (not isinstance(tokens, torch.Tensor) or tokens.dtype != torch.long or tokens.shape != (n_draft,)
            or tokens.device != dev):
        raise ValueError('Require [n] long tokens, [n,V] q and [n+1,V] p on one device')
    if (not isinstance(draft_probs, torch.Tensor) or draft_probs.dtype != torch.float64
            or draft_probs.shape != (n_draft, vocab) or draft_probs.device != dev or not draft_probs.is_contiguous()):
        raise ValueError('Require [n] long tokens, [n,V] q and [n+1,V] p on one device')
    if (not isinstance(uniforms, torch.Tensor) or uniforms.dtype != torch.float64 or uniforms.shape != (rows,)
            or uniforms.device != dev):
        raise ValueError('RNG must yield a float64 scalar in [0,1)')
    stops = [int(e) for e in eos_ids]
    if any(not 0 <= e < vocab for e in stops):
        raise ValueError('EOS IDs must be integers in the vocabulary')
    cu = [0]
    for n in counts:
        cu.append(cu[-1] + n + 1)
    head = upload(dev, cu + budgets + (stops or [0]))
    cu_rows, budget, stop_ids = head[:len(cu)], head[len(cu):len(cu) + len(budgets)], head[len(cu) + len(budgets):]
    stats, bad = _row_stats(logits, temperature)
    out_tokens = torch.empty(rows, dtype=torch.long, device=dev)
    meta = torch.empty((len(counts), 8), dtype=torch.int32, device=dev)
    ws = _draw_workspace(dev, len(counts))
    _native.call('dspark_spec_verify', logits.data_ptr(), dtype, logits.stride(0), vocab, temperature,
                 stats.data_ptr(), bad.data_ptr(), cu_rows.data_ptr(), len(counts), tokens.data_ptr(),
                 draft_probs.data_ptr(), uniforms.contiguous().data_ptr(), budget.data_ptr(), stop_ids.data_ptr(),
                 len(stops), out_tokens.data_ptr(), meta.data_ptr(), ws.data_ptr(), ws.numel(),
                 _native.stream_handle(dev))
    meta_h = meta.cpu().tolist()
    for m in meta_h:
        if m[6]:
            raise ValueError(_ERRORS[m[6]])
    results = []
    for r, m in enumerate(meta_h):
        emitted, accepted, rejected, extra, stop, draws = m[:6]
        results.append(VerifiedRound(out_tokens[cu[r]:cu[r] + emitted], accepted, rejected if rejected >= 0 else None,
                                     _EXTRA[extra], _STOP[stop], draws))
    return results
