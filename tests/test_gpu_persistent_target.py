"""PersistentQwenTarget on the GPU: graph buckets and ownership guards
(dspark_qwen/persistent_qwen_target.py:100-472; the reference's tests
tests/test_persistent_qwen_graph.py and tests/test_query_family.py).

A registered graph bucket is verified by replaying the captured full-model
forward (embedding, both decoder layers with the fused stage + attention,
final norm).  Every replay's hidden states, captured features and logits
are compared with the eager forward of the same transaction (run after an
abort), and with the CPU float32 model; commits between replays keep the
resident KV in step.  The guards refuse foreign streams, released or
foreign features and budgets beyond the declared ones."""
import numpy as np
import pytest
import torch

from test_gpu_hf_hooks import close, tiny_qwen3

pytestmark = pytest.mark.gpu
DEV = torch.device('cuda:0')
NEW = 7


def say(*a):
    print(*a, flush=True)


def ids(x):
    return torch.tensor([x], device=DEV)


def make_target(gpu, **kw):
    from qwen3_dspark_amd import backends
    from qwen3_dspark_amd.graph import TorchGraphBackend
    from qwen3_dspark_amd.persistent_target import PersistentQwenTarget
    args = dict(slots=3, context_capacity=256, max_query_tokens=128, graph_backend=TorchGraphBackend(),
                native_backend=backends.CAPACITY_BACKEND,
                max_graph_buckets=1, graph_byte_budget=1 << 30, workspace_byte_budget=1 << 30)
    args.update(kw)
    return PersistentQwenTarget(gpu, layer_ids=(0, 1), **args)


def test_graph_bucket_replays_match_eager_and_cpu_model():
    from qwen3_dspark_amd.persistent_kv import Bucket
    cpu, gpu = tiny_qwen3()
    rng = np.random.default_rng(5)
    target = make_target(gpu)
    names = ['a', 'b', 'c']
    prompts = [rng.integers(0, 512, size=n).tolist() for n in (30, 11, 52)]
    for n in names:
        target.add_request(n)
    pre = Bucket(tuple(len(p) for p in prompts), (0, 0, 0), 'prefill')
    target.register_bucket(pre)
    target.release_features(target.prefill({n: ids(p) for n, p in zip(names, prompts)}, bucket=pre))
    step = Bucket((NEW,) * 3, (256 - NEW,) * 3, 'graph verify')
    target.register_graph_bucket(step, reserve_bytes=256 << 20)
    with pytest.raises(ValueError, match='no capture-on-miss'):
        target.verify({n: ids([1] * NEW) for n in names}, bucket=step)
    say('[graph] capture')
    target.capture_graph({n: ids(rng.integers(0, 512, size=NEW).tolist()) for n in names}, bucket=step)
    assert target.lengths == {n: len(p) for n, p in zip(names, prompts)}
    seqs = [list(p) for p in prompts]
    for rnd, accepted in enumerate(([7, 2, 0], [4, 4, 4], [1, 7, 3], [0, 0, 5])):
        say(f'[graph] replay {rnd}')
        new = [rng.integers(0, 512, size=NEW).tolist() for _ in names]
        chunks = {n: ids(x) for n, x in zip(names, new)}
        g = target.verify(chunks, bucket=step)
        assert g.work['execution_kind'] == 'mi355x_hip_full_model_graph'
        if rnd == 0:
            say(f"[graph] private pool {g.work['graph_retained_bytes']} bytes of a 256 MiB reservation")
        g_last, g_ctx = g.last.clone(), g.context.clone()
        g_logits = {r: x.clone() for r, x in target.predict(g).items()}
        with pytest.raises(RuntimeError, match='existing verification transaction'):
            target.verify_eager(chunks, bucket=step)
        target.abort(g)
        with pytest.raises(RuntimeError, match='feature lease'):
            target.verify_eager(chunks, bucket=step)
        target.release_features(g)
        e = target.verify_eager(chunks, bucket=step)
        e_logits = target.predict(e)
        # replay against eager on the same transaction (the same kernels, so
        # equal up to library algorithm choice under capture)
        assert float((g_last.float() - e.last.float()).abs().max()) <= 2e-2
        assert float((g_ctx.float() - e.context.float()).abs().max()) <= 2e-2
        with torch.no_grad():
            for r, (n, s) in enumerate(zip(names, seqs)):
                ref = cpu(input_ids=torch.tensor([s + new[r]]), use_cache=False).logits[0, -NEW:].numpy()
                close(g_logits[n][0].float().cpu().numpy(), ref, (rnd, n, 'graph logits'))
                close(e_logits[n][0].float().cpu().numpy(), ref, (rnd, n, 'eager logits'))
        target.commit(e, dict(zip(names, accepted)))
        target.release_features(e)
        seqs = [s + x[:a] for s, x, a in zip(seqs, new, accepted)]
        assert target.lengths == {n: len(s) for n, s in zip(names, seqs)}
    # a graph verification committed directly
    new = [rng.integers(0, 512, size=NEW).tolist() for _ in names]
    g = target.verify({n: ids(x) for n, x in zip(names, new)}, bucket=step)
    target.commit(g, dict(zip(names, [3, 3, 3])))
    target.release_features(g)
    seqs = [s + x[:3] for s, x in zip(seqs, new)]
    with torch.no_grad():
        pkv = cpu(input_ids=torch.tensor([seqs[2]]), use_cache=True).past_key_values
    for layer, (k, v) in enumerate(target.request_kv('c')):
        close(k[0].float().cpu().numpy(), pkv.layers[layer].keys[0].numpy(), ('c', layer, 'keys'))


def test_graph_ticket_protocol_and_guards():
    from qwen3_dspark_amd.persistent_kv import Bucket
    _, gpu = tiny_qwen3()
    target = make_target(gpu, workspace_byte_budget=1 << 21, max_buckets=2)
    for n in ('a', 'b'):
        target.add_request(n)
    pre = Bucket((5, 3), (0, 0), 'prefill')
    target.register_bucket(pre)
    f = target.prefill({'a': ids([1, 2, 3, 4, 5]), 'b': ids([6, 7, 8])}, bucket=pre)
    # features: leases checked by identity
    target.predict(f)
    target.release_features(f)
    with pytest.raises(ValueError, match='Foreign or released'):
        target.predict(f)
    with pytest.raises(ValueError, match='already released'):
        target.release_features(f)
    # budgets
    with pytest.raises(ValueError, match='budget'):
        target.register_bucket(Bucket((7, 7), (249, 249), 'too large for 2 MiB'))
    step = Bucket((2, 2), (100, 100), 'graph')
    target.register_graph_bucket(step, reserve_bytes=256 << 20)
    with pytest.raises(ValueError, match='Duplicate graph bucket'):
        target.register_graph_bucket(step, reserve_bytes=256 << 20)
    with pytest.raises(ValueError, match='budget'):
        target.register_bucket(Bucket((1,), (10,), 'third bucket beyond max_buckets'))
    target.capture_graph({'a': ids([9, 9]), 'b': ids([8, 8])}, bucket=step)
    # ticket protocol
    ticket = target.prepare_graph_verify({'a': ids([1, 2]), 'b': ids([3, 4])}, bucket=step)
    with pytest.raises(RuntimeError, match='graph submission'):
        target.prepare_graph_verify({'a': ids([1, 2]), 'b': ids([3, 4])}, bucket=step)
    done = target.submit_graph(ticket)
    with pytest.raises(ValueError, match='unsubmitted'):
        target.submit_graph(ticket)
    feats = target.finish_graph(done)
    with pytest.raises(ValueError, match='submitted graph completion'):
        target.finish_graph(done)
    target.abort(feats)
    target.release_features(feats)
    ticket = target.prepare_graph_verify({'a': ids([1, 2]), 'b': ids([3, 4])}, bucket=step)
    target.cancel_graph(ticket)
    assert target.lengths == {'a': 5, 'b': 3}
    # the owner stream only
    side = torch.cuda.Stream(device=DEV)
    with torch.cuda.stream(side):
        with pytest.raises(RuntimeError, match='owner stream'):
            target.add_request('c')
        with pytest.raises(RuntimeError, match='owner stream'):
            target.verify_eager({'a': ids([1, 2]), 'b': ids([3, 4])}, bucket=step)
    # chunk validation in the reference's order
    with pytest.raises(ValueError, match='explicit bucket'):
        target.verify_eager({}, bucket=step)
    with pytest.raises(ValueError, match='must match the chosen bucket'):
        target.verify_eager({'a': ids([1, 2, 3]), 'b': ids([3, 4])}, bucket=step)
    with pytest.raises(ValueError, match='vocabulary'):
        target.verify_eager({'a': ids([1, 512]), 'b': ids([3, 4])}, bucket=step)
    target.close()
    with pytest.raises(RuntimeError, match='closed'):
        target.add_request('c')
