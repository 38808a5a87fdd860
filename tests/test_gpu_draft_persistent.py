"""The draft attention's persistent scheduling (HipDraftAttention(persistent=1
or 8): one workgroup per CU taking (chunk, KV head) items from device ticket
counters) against the hardware-dispatched grid: outputs must be bitwise
equal (the arithmetic per item is the same, only which workgroup runs it
changes), in every kernel instance (bf16 row store, fp32-K AMP pool,
indexed append-order pool), on back-to-back launches of different batches
(the counters reset themselves), and the outputs meet the oracle gate."""
import numpy as np
import pytest
import torch

from helpers import SCALE, SEED, attention_gate, f64
from test_gpu_draft import dev, draft_case, oracle, run  # noqa: F401

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


@pytest.mark.parametrize('form', ['bf16', 'kf32', 'indexed'])
def test_persistent_modes_bitwise_equal_to_hardware_dispatch(dev, form):
    from qwen3_dspark_amd.draft import HipDraftAttention
    gen = torch.Generator().manual_seed(SEED + 31)
    rng = np.random.default_rng(SEED + 31)
    kernels = {m: HipDraftAttention(dev, chunk=1024, persistent=m) for m in (None, 1, 8)}
    # three batches of different sizes back to back: each launch must find
    # the ticket counters zero again
    for case, (contexts, blocks) in enumerate((([3000, 5, 900, 0, 4100], [1, 8, 3, 2, 5]),
                                               ([17, 2048], [8, 1]),
                                               ([int(x) for x in rng.integers(0, 6000, size=40)],
                                                [int(x) for x in rng.integers(1, 9, size=40)]))):
        c = draft_case(gen, rng, contexts, blocks)
        want, cu_b = oracle(c)           # on the bf16 values (fp32 K below holds exactly these)
        kw = {}
        if form == 'kf32':
            c['ctx_k'] = c['ctx_k'].float()
            c['bk'] = c['bk'].float()
        if form == 'indexed':
            n = c['ctx_k'].shape[0]
            perm = torch.from_numpy(rng.permutation(n)).long()
            kw = dict(ctx_k=c['ctx_k'][perm], ctx_v=c['ctx_v'][perm],
                      indices=torch.argsort(perm).to(dev))
        outs = {m: [run(dev, k, c, **kw) for _ in range(2)] for m, k in kernels.items()}
        ref = outs[None][0]
        for m, pair in outs.items():
            for out in pair:
                assert torch.equal(out, ref), (form, case, m)
        rows = [(7 * cu_b[i], 7 * cu_b[i + 1]) for i in range(len(cu_b) - 1)]
        stats = attention_gate(f64(ref), want, rows)
        say(f'[persistent {form}] case {case}: {len(contexts)} requests, max |d| {stats[0]["max_abs"]:.2e}')
    for m in (1, 8):
        assert int(kernels[m]._queue.abs().sum()) == 0, 'the ticket counters must be zero after every launch'
