"""Completion-wait engine: a counterpart of ``CPUWaitEngine``
(managers/ring_attn_manager.py:6-62).

The reference keeps one daemon thread, pinned to a core, that takes
``(request, CommWork)`` pairs from a queue, blocks on ``request.wait()`` and
then sets the ``CommWork`` event, so the caller can poll or wait for a
communication without blocking its own thread.  It is imported by
attn.py:11 and unused on the hot path.

Here the requests are whatever the GPU side produces: ``torch.cuda.Event``
(waited with ``synchronize()``), ``torch.distributed`` work handles
(``wait()``), or ``None`` (completes immediately).  Core pinning is optional:
``HARP_WAIT_ENGINE_CORE=<cpu>`` pins the worker thread (the reference derives
the core from ``OMPI_COMM_WORLD_RANK``, ring_attn_manager.py:36-40).
Errors raised while waiting are stored on the ``CommWork`` and re-raised by
its ``wait()`` instead of only being printed (ring_attn_manager.py:48-52).
"""

from __future__ import annotations

import os
import queue
import threading
from typing import Any, Optional


class CommWork:
    """Completion handle returned by :meth:`WaitEngine.submit`."""

    def __init__(self) -> None:
        self._done_event = threading.Event()
        self.work_handle: Any = None
        self.error: Optional[BaseException] = None

    def mark_done(self) -> None:
        self._done_event.set()

    def is_done(self) -> bool:
        return self._done_event.is_set()

    def wait(self, timeout: Optional[float] = None) -> bool:
        done = self._done_event.wait(timeout)
        if self.error is not None:
            raise RuntimeError("wait engine request failed") from self.error
        return done


class WaitEngine:
    """Singleton worker that waits on submitted requests in FIFO order."""

    _instance: Optional["WaitEngine"] = None
    _lock = threading.Lock()

    def __init__(self) -> None:
        self.task_queue: "queue.Queue" = queue.Queue()
        self.stop_event = threading.Event()
        self._submit_lock = threading.Lock()  # orders submit() against shutdown()
        core = os.environ.get("HARP_WAIT_ENGINE_CORE")
        self.core_id = int(core) if core not in (None, "") else None
        self.worker_thread = threading.Thread(target=self._run, daemon=True, name="harp-wait-engine")
        self.worker_thread.start()

    @classmethod
    def get_instance(cls) -> "WaitEngine":
        if cls._instance is None:
            with cls._lock:
                if cls._instance is None:
                    cls._instance = cls()
        return cls._instance

    @staticmethod
    def _wait_on(req: Any) -> None:
        if req is None:
            return
        if _is_device_event(req):
            # a device event is waited on by the host: Event.wait() would only
            # make the worker thread's current stream wait and return at once
            req.synchronize()
        elif hasattr(req, "wait"):
            req.wait()  # torch.distributed work handle (or any object with wait())
        elif hasattr(req, "synchronize"):
            req.synchronize()
        else:
            raise TypeError(f"cannot wait on {type(req).__name__}")

    def _run(self) -> None:
        if self.core_id is not None and hasattr(os, "sched_setaffinity"):
            os.sched_setaffinity(threading.get_native_id(), {self.core_id})
        while not self.stop_event.is_set():
            try:
                req, task = self.task_queue.get(timeout=0.1)
            except queue.Empty:
                continue
            try:
                self._wait_on(req)
            except BaseException as e:  # noqa: BLE001 - handed to the waiter
                task.error = e
            task.mark_done()
            self.task_queue.task_done()

    def submit(self, req: Any) -> CommWork:
        task = CommWork()
        task.work_handle = req
        with self._submit_lock:
            if self.stop_event.is_set():
                raise RuntimeError("wait engine is shut down")
            self.task_queue.put((req, task))
        return task

    def shutdown(self) -> None:
        """Stop the worker.  Requests still queued are not waited on: their
        CommWork is completed with an error, so no caller blocks forever."""
        with self._submit_lock:
            self.stop_event.set()
        self.worker_thread.join()
        while True:
            try:
                _, task = self.task_queue.get_nowait()
            except queue.Empty:
                break
            task.error = RuntimeError("wait engine shut down before the request was waited on")
            task.mark_done()
            self.task_queue.task_done()
        with WaitEngine._lock:
            if WaitEngine._instance is self:
                WaitEngine._instance = None


def _is_device_event(req: Any) -> bool:
    try:
        import torch
    except ImportError:  # pragma: no cover - torch is a dependency of the package
        return False
    return isinstance(req, torch.cuda.Event)
