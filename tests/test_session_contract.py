"""Host-side contract of the slot session (CPU; CUDA calls are monkeypatched,
as in the reference's tests/test_prefetch.py:47-140): run finalisation and
close failures poison the session and release the run capability, a failed
consumed event poisons and releases the borrow guard, borrows need the run
token and are not reentrant, and the weight borrow of the recompute driver is
released after the whole consumer and on exceptions."""
import threading
from contextlib import contextmanager
from types import SimpleNamespace

import pytest
import torch

from spilltune_amd.recompute import _borrow_weights
from spilltune_amd.slots import Q4SlotSession


def bare_session():
    s = object.__new__(Q4SlotSession)
    s.closed = s.poisoned = False
    s.device = torch.device("cuda:0")
    s._run_lock, s._borrow_lock = threading.Lock(), threading.Lock()
    s._owner = s._token = None
    s.copy_records, s.slots, s.images = [], [], {}
    return s


@pytest.mark.parametrize("failure", ["drain", "finalize"])
def test_run_finalization_failure_poisons_and_releases_capability(monkeypatch, failure):
    s = bare_session()

    def fail(*_):
        raise RuntimeError("injected " + failure)
    monkeypatch.setattr(torch.cuda, "synchronize", fail if failure == "drain" else lambda *_: None)
    s._finalize_copies = fail if failure == "finalize" else (lambda: None)
    with pytest.raises(RuntimeError, match="injected"):
        with s.run():
            pass
    assert s.poisoned and s._token is None and s._owner is None and not s._run_lock.locked()
    with pytest.raises(RuntimeError, match="poisoned"):
        with s.run():
            pass


def test_consumer_exception_poisons_the_run(monkeypatch):
    s = bare_session()
    monkeypatch.setattr(torch.cuda, "synchronize", lambda *_: None)
    s._finalize_copies = lambda: None
    with pytest.raises(ValueError):
        with s.run():
            raise ValueError("functional failure")
    assert s.poisoned and not s._run_lock.locked()


def test_close_drain_failure_poisons_keeps_buffers_then_retry(monkeypatch):
    s = bare_session()
    s.slots, s.images = [object()], {1: object()}

    def fail(*_):
        raise RuntimeError("close drain failure")
    monkeypatch.setattr(torch.cuda, "synchronize", fail)
    with pytest.raises(RuntimeError, match="close drain failure"):
        s.close()
    assert s.poisoned and not s.closed and len(s.slots) == 1 and len(s.images) == 1
    with pytest.raises(RuntimeError, match="poisoned"):
        with s.run():
            pass
    monkeypatch.setattr(torch.cuda, "synchronize", lambda *_: None)
    s.close()
    assert s.closed and not s.slots and not s.images


def _running_session(block):
    s = bare_session()
    s._run_lock.acquire()
    s._token, s._owner = object(), threading.get_ident()
    s.positions, s.blocks = {id(block): 0}, [block]
    s.prefetch, s._clock, s.reloads, s.hits, s.trace = False, 0, 0, 0, []
    slot = {"id": 0, "block": block, "ready": object(), "consumed": None, "active": False,
            "last_use": 0, "views": {"w": torch.ones(1)}}
    s.slots = [slot]
    return s, slot


@pytest.mark.parametrize("failure", ["create", "record"])
def test_consumed_event_failure_poisons_and_releases_borrow_guard(monkeypatch, failure):
    block = SimpleNamespace(index=0)
    s, slot = _running_session(block)
    monkeypatch.setattr(torch.cuda, "current_stream",
                        lambda *_: SimpleNamespace(wait_event=lambda _: None))

    def fail(*_):
        raise RuntimeError("consumed " + failure + " failure")
    monkeypatch.setattr(torch.cuda, "Event",
                        fail if failure == "create" else (lambda: SimpleNamespace(record=fail)))
    with pytest.raises(RuntimeError, match="consumed"):
        with s.borrow(block, "forward", token=s._token) as views:
            assert torch.equal(views["w"], torch.ones(1))
    assert s.poisoned and not s._borrow_lock.locked() and slot["active"]
    with pytest.raises(RuntimeError, match="poisoned"):
        with s.borrow(block, "forward", token=s._token):
            pass


def test_borrow_needs_the_run_token_and_is_not_reentrant(monkeypatch):
    block = SimpleNamespace(index=0)
    s, slot = _running_session(block)
    monkeypatch.setattr(torch.cuda, "current_stream",
                        lambda *_: SimpleNamespace(wait_event=lambda _: None))
    monkeypatch.setattr(torch.cuda, "Event", lambda: SimpleNamespace(record=lambda _: None))
    with pytest.raises(RuntimeError, match="run capability"):
        with s.borrow(block, "forward", token=object()):
            pass
    with pytest.raises(ValueError, match="phase"):
        with s.borrow(block, "sideways", token=s._token):
            pass
    with s.borrow(block, "backward", token=s._token):
        with pytest.raises(RuntimeError, match="reentrant"):
            with s.borrow(block, "forward", token=s._token):
                pass
    assert not s.poisoned and not s._borrow_lock.locked() and not slot["active"]
    assert s.trace[-1]["cache_hit"] and s.trace[-1]["phase"] == "backward"
    with pytest.raises(RuntimeError, match="explicit consumer borrow"):
        s.reloader(block)()


def test_borrow_scope_releases_only_after_full_consumer_and_on_exception():
    events = []

    class Loader:
        @contextmanager
        def borrow(self, phase):
            events.append(("acquire", phase))
            try:
                yield {"weights": torch.ones(1)}
            finally:
                events.append(("release", phase))
    with _borrow_weights(Loader(), "backward"):
        events.extend(["recompute", "autograd.grad", "grad_A.add", "grad_B.add"])
    assert events == [("acquire", "backward"), "recompute", "autograd.grad", "grad_A.add",
                      "grad_B.add", ("release", "backward")]
    events.clear()
    with pytest.raises(ValueError):
        with _borrow_weights(Loader(), "forward"):
            raise ValueError("functional failure")
    assert events == [("acquire", "forward"), ("release", "forward")]
