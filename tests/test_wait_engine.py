"""WaitEngine / CommWork, the counterpart of CPUWaitEngine / CommWork
(managers/ring_attn_manager.py:6-62): FIFO completion, None requests,
objects with wait(), error re-raise, the singleton, shutdown; and (GPU) a
torch.cuda.Event recorded after a ring-attention launch is waited on by the
host, not merely enqueued on a stream."""

import threading
import time

import pytest
import torch

from harp_amd.wait_engine import CommWork, WaitEngine


class Gate:
    """Request whose wait() blocks until the test opens it; records order."""

    def __init__(self, log, name):
        self.log, self.name = log, name
        self.opened = threading.Event()

    def wait(self):
        assert self.opened.wait(10), f"{self.name} never opened"
        self.log.append(self.name)


class Failing:
    def wait(self):
        raise ValueError("transport broke")


@pytest.fixture
def engine():
    e = WaitEngine()
    yield e
    e.shutdown()


def test_none_request_completes(engine):
    w = engine.submit(None)
    assert w.wait(5) is True and w.is_done()
    assert w.work_handle is None


def test_requests_complete_in_fifo_order(engine):
    log = []
    gates = [Gate(log, i) for i in range(4)]
    works = [engine.submit(g) for g in gates]
    time.sleep(0.05)
    assert not any(w.is_done() for w in works)  # the first blocks the rest
    for g in reversed(gates):  # open in reverse: completion still follows submission
        g.opened.set()
    for w in works:
        assert w.wait(5)
    assert log == [0, 1, 2, 3]


def test_wait_timeout_returns_false_until_done(engine):
    log = []
    g = Gate(log, "x")
    w = engine.submit(g)
    assert w.wait(0.05) is False and not w.is_done()
    g.opened.set()
    assert w.wait(5) is True


def test_error_is_reraised_by_wait_and_engine_survives(engine):
    w = engine.submit(Failing())
    with pytest.raises(RuntimeError, match="request failed") as ei:
        w.wait(5)
    assert isinstance(ei.value.__cause__, ValueError)
    assert engine.submit(None).wait(5)  # the worker keeps going


def test_unwaitable_request_reports_type_error(engine):
    w = engine.submit(object())
    with pytest.raises(RuntimeError) as ei:
        w.wait(5)
    assert isinstance(ei.value.__cause__, TypeError)


def test_synchronize_only_request(engine):
    class Sync:
        called = False

        def synchronize(self):
            Sync.called = True

    assert engine.submit(Sync()).wait(5) and Sync.called


def test_singleton_and_shutdown_resets_it():
    a = WaitEngine.get_instance()
    assert WaitEngine.get_instance() is a
    a.shutdown()
    b = WaitEngine.get_instance()
    assert b is not a and b.worker_thread.is_alive()
    b.shutdown()
    assert not b.worker_thread.is_alive()


def test_shutdown_fails_pending_requests_instead_of_hanging():
    e = WaitEngine()
    log = []
    g = Gate(log, "blocker")
    first = e.submit(g)
    pending = [e.submit(None) for _ in range(3)]
    t = threading.Thread(target=e.shutdown)
    t.start()
    time.sleep(0.05)
    g.opened.set()  # let the in-flight request finish so the worker can stop
    t.join(10)
    assert not t.is_alive()
    assert first.wait(5)
    for w in pending:  # either waited before the stop, or failed by shutdown
        assert w.is_done()
        if w.error is not None:
            with pytest.raises(RuntimeError, match="request failed") as ei:
                w.wait(1)
            assert "shut down" in str(ei.value.__cause__)
    with pytest.raises(RuntimeError, match="shut down"):
        e.submit(None)


def test_commwork_mark_done():
    w = CommWork()
    assert not w.is_done()
    w.mark_done()
    assert w.is_done() and w.wait(0)


@pytest.mark.gpu
def test_cuda_event_is_waited_on_by_the_host(engine):
    """An event recorded after a ring-attention forward completes only when
    the GPU has passed it: after CommWork.wait() the event has been reached
    and the forward's output is final."""
    import math

    import harp_amd

    harp_amd.load_ops()
    g = torch.Generator().manual_seed(7)
    B, H, T, D, N = 1, 8, 2048, 128, 4

    def tok(t):
        return torch.randn((B, t, H, D), generator=g).to(torch.bfloat16).cuda().transpose(1, 2)

    q, k, v = tok(T), tok(N * T), tok(N * T)
    out = torch.empty(q.shape, dtype=torch.float32, device="cuda")
    m = torch.empty((B, H, T, 1), dtype=torch.bfloat16, device="cuda")
    l = torch.empty((B, H, T, 1), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    torch.ops.ring_attention_ops.ring_attention_forward(q, k, v, out, m, l, N, 1.0 / math.sqrt(D))
    ev = torch.cuda.Event()
    ev.record()
    w = engine.submit(ev)
    assert w.wait(60)
    assert ev.query(), "CommWork completed before the GPU reached the event"
    snap = out.clone()
    torch.cuda.synchronize()
    assert torch.equal(snap, out) and torch.isfinite(out).all()
