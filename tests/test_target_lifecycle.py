"""The persistent target's round lifecycle on the CPU
(qwen3_dspark_amd/persistent_target.py; the contract of
dspark_qwen/persistent_qwen_target.py:166-472 and its tests
tests/test_persistent_qwen_target.py / tests/test_persistent_qwen_graph.py).

The target's host half runs over the store's CPU stand-in device
(tests/kv_fake.py); the model forward is replaced by one that stages every
layer into scratch, and a captured program by a stand-in that publishes the
scratch through the store's external-writer receipts.  What is checked is the
stage machine itself: which call each stage admits, the error class and
message of every refusal (the reference's), that a refused call changes
nothing, and that the store is idle again whenever the target is READY.
"""
from types import SimpleNamespace

import pytest
import torch

import kv_fake
from qwen3_dspark_amd.hf_hooks import FusedVerifier
from qwen3_dspark_amd.persistent_kv import Bucket
from qwen3_dspark_amd.persistent_target import (
    _NOT_READY, _REFUSED, _TABLE, PersistentQwenTarget, Stage, _Budget)

HIDDEN, VOCAB = 6, 50


class _Backend:
    kind = 'stand-in program'

    def wait(self, event):
        pass


class _Program:
    """A captured bucket's stand-in: submit 'replays' by returning an event
    object; the store publishes the scratch once complete() says so."""

    def __init__(self, target, bucket):
        self.backend = _Backend()
        self.graph = 'captured'
        self.writer = target.store.register_external_writer(bucket, range(target.store.layers), self.complete)
        self.last = torch.zeros(1, bucket.query_tokens, HIDDEN)
        self.context = torch.zeros(1, bucket.query_tokens, HIDDEN)
        self.retained_bytes, self.memory = 0, None
        self.invalid = False
        self.submitted = None

    def validate(self):
        if self.invalid:
            raise RuntimeError('Captured program invalidated')

    def load(self, chunks):
        pass

    def submit(self, receipt):
        self.submitted = (receipt, object())
        return self.submitted[1]

    def complete(self, event, receipt):
        return self.submitted is not None and self.submitted == (receipt, event)


def make_target(*, fail_forward=False):
    store = kv_fake.store(layers=2, slots=3, context_capacity=24, max_query_tokens=8, heads=2, dim=4)
    head = torch.nn.Linear(HIDDEN, VOCAB, bias=False)
    model = SimpleNamespace(config=SimpleNamespace(vocab_size=VOCAB, hidden_size=HIDDEN, _attn_implementation='x'),
                            get_output_embeddings=lambda: head)
    verifier = FusedVerifier.__new__(FusedVerifier)
    verifier.model, verifier.store, verifier.transaction, verifier.handles = model, store, None, ()
    t = PersistentQwenTarget.__new__(PersistentQwenTarget)
    t.layer_ids = (1,)
    t._setup(store, verifier, 'stand-in', _Backend(), _Budget(4, 1 << 30, 1 << 30, True), 1, 'sdpa')
    t._stream_id = lambda: t.current_stream
    t.current_stream = t._owner_stream = 'owner'

    def forward(ids, positions):
        tx = t.verifier.transaction
        q = ids.shape[1]
        for layer in range(store.layers):
            store.stage_layer(tx, layer, torch.randn(q, 2, 4), torch.randn(q, 2, 4))
            if fail_forward and layer == 0:
                raise RuntimeError('forward failed')
        return torch.randn(1, q, HIDDEN), torch.randn(1, q, HIDDEN)
    t._run_forward = forward
    return t


def ids(*x):
    return torch.tensor([list(x)])


def admitted(t):
    for r in ('a', 'b'):
        t.add_request(r)
    bucket = Bucket((2, 1), (20, 20), 'lifecycle')
    t.register_bucket(bucket)
    return bucket


def test_table_is_total_and_consistent():
    for stage in Stage:
        assert stage in _TABLE
        for event, nxt in _TABLE[stage].items():
            assert isinstance(nxt, Stage)
        if 'admin' not in _TABLE[stage]:
            assert stage in _NOT_READY
    # every round event some stage refuses has the reference's error
    events = {e for row in _TABLE.values() for e in row}
    assert {'commit', 'abort', 'submit', 'finish', 'cancel'} <= events
    assert set(_REFUSED) <= events


def test_eager_round_commit_abort_and_release():
    t = make_target()
    bucket = admitted(t)
    f = t.verify_eager({'a': ids(1, 2), 'b': ids(3)}, bucket=bucket)
    assert t.stage is Stage.VERIFIED and f.spans == {'a': (0, 2, 0), 'b': (2, 1, 0)}
    # a second round, admin calls and release of the pending features are refused
    with pytest.raises(RuntimeError, match='^Finish existing verification transaction first$'):
        t.verify_eager({'a': ids(1, 2), 'b': ids(3)}, bucket=bucket)
    with pytest.raises(RuntimeError, match='^Finish existing verification transaction first$'):
        t.add_request('c')
    with pytest.raises(RuntimeError, match='^Commit or abort before releasing feature lease$'):
        t.release_features(f)
    foreign = SimpleNamespace(spans=f.spans)
    with pytest.raises(ValueError, match='^Only the outstanding verification features can commit$'):
        t.commit(foreign, {'a': 1, 'b': 1})
    with pytest.raises(ValueError, match='^One committed query prefix per verified request required$'):
        t.commit(f, {'a': 1})
    assert t.stage is Stage.VERIFIED
    assert t.commit(f, {'a': 2, 'b': 0})['committed_tokens'] == 2
    assert t.stage is Stage.READY and t.store.open_transaction is None and t.lengths == {'a': 2, 'b': 0}
    with pytest.raises(ValueError, match='^Only outstanding verification features can abort$'):
        t.abort(f)
    # features outlive their round: predict, then release once
    assert set(t.predict(f, last_only=True)) == {'a', 'b'}
    t.release_features(f)
    with pytest.raises(ValueError, match='^Foreign or released features$'):
        t.predict(f)
    with pytest.raises(ValueError, match='^Foreign, copied or already released features$'):
        t.release_features(f)
    # abort rolls every row back
    g = t.verify_eager({'a': ids(4, 5), 'b': ids(6)}, bucket=Bucket((2, 1), (20, 20), 'lifecycle'))
    t.abort(g)
    assert t.stage is Stage.READY and t.lengths == {'a': 2, 'b': 0}


def test_chunk_contract_in_reference_order_changes_nothing():
    t = make_target()
    bucket = admitted(t)
    for chunks, err in (({}, 'explicit bucket required'),
                        ({'a': ids(1, 2, 3), 'b': ids(3)}, 'must match the chosen bucket'),
                        ({'a': ids(1, 2), 'b': ids(VOCAB)}, 'outside vocabulary'),
                        ({'a': ids(1, 2).int(), 'b': ids(3)}, r'\[1,Q\] long')):
        with pytest.raises(ValueError, match=err):
            t.verify_eager(chunks, bucket=bucket)
        assert t.stage is Stage.READY and t.store.open_transaction is None
    with pytest.raises(ValueError, match='explicit bucket required'):
        t.verify_eager({'a': ids(1, 2), 'b': ids(3)}, bucket=(2, 1))


def test_failed_forward_aborts_and_returns_to_ready():
    t = make_target(fail_forward=True)
    bucket = admitted(t)
    with pytest.raises(RuntimeError, match='forward failed'):
        t.verify_eager({'a': ids(1, 2), 'b': ids(3)}, bucket=bucket)
    assert t.stage is Stage.READY and t.store.open_transaction is None and t.verifier.transaction is None
    t.add_request('c')


def graph_target():
    t = make_target()
    bucket = admitted(t)
    t._graphs[bucket] = _Program(t, bucket)
    return t, bucket


def test_graph_round_ticket_completion_lease():
    t, bucket = graph_target()
    chunks = {'a': ids(1, 2), 'b': ids(3)}
    ticket = t.prepare_graph_verify(chunks, bucket=bucket)
    assert t.stage is Stage.TICKETED
    for call in (lambda: t.add_request('c'), lambda: t.prepare_graph_verify(chunks, bucket=bucket),
                 lambda: t.verify_eager(chunks, bucket=bucket)):
        with pytest.raises(RuntimeError, match='^Finish graph submission and release feature lease first$'):
            call()
    with pytest.raises(ValueError, match='^Exact unsubmitted graph ticket required$'):
        t.submit_graph(SimpleNamespace())
    with pytest.raises(ValueError, match='^Exact submitted graph completion required$'):
        t.finish_graph(None)
    done = t.submit_graph(ticket)
    assert t.stage is Stage.IN_FLIGHT
    with pytest.raises(ValueError, match='^Exact unsubmitted graph ticket required$'):
        t.submit_graph(ticket)
    feats = t.finish_graph(done)
    assert t.stage is Stage.LEASED_VERIFIED and feats.work['execution_kind'] == 'stand-in program'
    with pytest.raises(ValueError, match='^Exact submitted graph completion required$'):
        t.finish_graph(done)
    with pytest.raises(RuntimeError, match='^Commit or abort before releasing feature lease$'):
        t.release_features(feats)
    t.commit(feats, {'a': 1, 'b': 1})
    assert t.stage is Stage.LEASED and t.lengths == {'a': 1, 'b': 1}
    # the lease still blocks a new round until released
    with pytest.raises(RuntimeError, match='^Finish graph submission and release feature lease first$'):
        t.add_request('c')
    t.predict(feats)
    t.release_features(feats)
    assert t.stage is Stage.READY
    t.add_request('c')


def test_graph_cancel_and_verify_dispatch():
    t, bucket = graph_target()
    chunks = {'a': ids(1, 2), 'b': ids(3)}
    ticket = t.prepare_graph_verify(chunks, bucket=bucket)
    with pytest.raises(ValueError, match='^Exact graph ticket required$'):
        t.cancel_graph(SimpleNamespace())
    t.cancel_graph(ticket)
    assert t.stage is Stage.READY and t.store.open_transaction is None
    with pytest.raises(ValueError, match='^Exact graph ticket required$'):
        t.cancel_graph(ticket)
    # verify() on a graph bucket goes through the program and leases its output
    feats = t.verify(chunks, bucket=bucket)
    assert t.stage is Stage.LEASED_VERIFIED
    t.abort(feats)
    assert t.stage is Stage.LEASED and t.lengths == {'a': 0, 'b': 0}
    t.release_features(feats)
    # prefill on a graph bucket runs eager and commits every row
    f = t.prefill(chunks, bucket=bucket)
    assert t.stage is Stage.READY and t.lengths == {'a': 2, 'b': 1} and 'execution_kind' not in f.work


def test_invalidate_keeps_only_the_lease_and_store_stays_poisoned():
    t, bucket = graph_target()
    feats = t.verify({'a': ids(1, 2), 'b': ids(3)}, bucket=bucket)
    t.invalidate()
    assert t.stage is Stage.LEASED and t.store.failed and t._graphs[bucket].invalid
    with pytest.raises(ValueError, match='^Only the outstanding verification features can commit$'):
        t.commit(feats, {'a': 0, 'b': 0})
    t.release_features(feats)
    assert t.stage is Stage.READY
    with pytest.raises(RuntimeError, match='Store invalidated'):
        t.add_request('c')


def test_owner_stream_budgets_and_close():
    t = make_target()
    bucket = admitted(t)
    t.current_stream = 'side'
    with pytest.raises(RuntimeError, match='owner stream'):
        t.add_request('c')
    with pytest.raises(RuntimeError, match='owner stream'):
        t.verify_eager({'a': ids(1, 2), 'b': ids(3)}, bucket=bucket)
    t.current_stream = 'owner'
    t._budget.workspace_limit = t._budget.workspace
    with pytest.raises(ValueError, match='^Finite bucket/workspace budget exceeded$'):
        t.register_bucket(Bucket((1,), (3,), 'beyond the workspace budget'))
    t.register_bucket(bucket)        # already registered: no new bytes
    with pytest.raises(ValueError, match='Explicit Bucket or QueryFamily'):
        t.register_bucket((1,))
    t._hooks = [SimpleNamespace(remove=lambda: None)]
    t.close()
    assert t.stage is Stage.CLOSED and t.model.config._attn_implementation == 'sdpa'
    for call in (lambda: t.add_request('c'), lambda: t.close(),
                 lambda: t.verify_eager({'a': ids(1, 2), 'b': ids(3)}, bucket=bucket)):
        with pytest.raises(RuntimeError, match='^Target adapter closed$'):
            call()


def test_hooks_refuse_foreign_forwards():
    t = make_target()
    hook = t._hook(1)
    with pytest.raises(RuntimeError, match='Foreign model forward'):
        hook(None, None, torch.zeros(1))
    t._captured = {}
    hook(None, None, (torch.ones(1),))
    assert torch.equal(t._captured[1], torch.ones(1))
