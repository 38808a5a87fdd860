"""HostStaging's reuse rule on a stand-in stream and event (CPU): copies
share one event per span; a region is rewritten only after the event of the
span that last held it, and the open span is closed before any of its bytes
are reused or the stream changes."""
import torch

from qwen3_dspark_amd import _device


class FakeEvent:
    log = []

    def __init__(self):
        self.done = False
        self.stream = None

    def record(self, stream):
        self.stream = stream
        self.done = False
        FakeEvent.log.append(('record', stream.cuda_stream))

    def query(self):
        return self.done

    def synchronize(self):
        FakeEvent.log.append(('sync', self.stream.cuda_stream))
        self.done = True


class FakeStream:
    def __init__(self, handle):
        self.cuda_stream = handle


def staging(monkeypatch, nbytes=4096, streams=None):
    current = {'s': FakeStream(1)}
    monkeypatch.setattr(torch.cuda, 'Event', FakeEvent)
    monkeypatch.setattr(torch.cuda, 'current_stream', lambda device=None: current['s'])
    st = _device.HostStaging.__new__(_device.HostStaging)
    st.device = torch.device('cpu')
    st._buf = torch.empty(nbytes, dtype=torch.uint8)
    st._head = 0
    st._inflight = __import__('collections').deque()
    st._open = None
    st._events = []
    st._lock = __import__('threading').Lock()
    return st, current


def test_one_event_per_span_and_reuse_waits(monkeypatch):
    FakeEvent.log = []
    st, current = staging(monkeypatch)
    monkeypatch.setattr(_device.HostStaging, 'MARK_BYTES', 1024)
    for i in range(3):                                   # 3 x 256 B: one open span, no event yet
        out = st.upload([i] * 10)
        assert out.tolist() == [i] * 10
    assert FakeEvent.log == [] and st._open[:2] == [0, 768]
    st.upload(list(range(64)))                           # reaches 1024 B: the span closes with one event
    assert FakeEvent.log == [('record', 1)] and st._open is None and len(st._inflight) == 1
    for _ in range(13):                                  # fill the 4 KiB ring and wrap onto the first span
        st.upload([7] * 64)
    assert ('sync', 1) in FakeEvent.log                  # the first span's event waited before its bytes are reused
    syncs = [e for e in FakeEvent.log if e[0] == 'sync']
    records = [e for e in FakeEvent.log if e[0] == 'record']
    assert len(records) < 16                             # far fewer events than uploads


def test_stream_change_closes_the_span(monkeypatch):
    FakeEvent.log = []
    st, current = staging(monkeypatch)
    st.upload([1, 2, 3])
    current['s'] = FakeStream(2)
    st.upload([4, 5, 6])
    assert FakeEvent.log == [('record', 1)]              # the stream-1 span got its own event on stream 1
    assert st._open[2].cuda_stream == 2
