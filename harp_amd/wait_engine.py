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
        if hasattr(req, "synchronize") and not hasattr(req, "wait"):
            req.synchronize()  # torch.cuda.Event
        elif hasattr(req, "wait"):
            req.wait()
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
        self.task_queue.put((req, task))
        return task

    def shutdown(self) -> None:
        self.stop_event.set()
        self.worker_thread.join()
        with WaitEngine._lock:
            if WaitEngine._instance is self:
                WaitEngine._instance = None
