"""Device-to-host copies and file writes off the training step's critical path.

The reference engines copy each step's results to the host synchronously
(graddotprod_engine.py:218-226 appends ``.cpu()`` copies to the dot-product log;
gradproj_engine.py:274-301 does ``projection.cpu()`` and ``torch.save`` inside
``collect_batch``), so the host waits for the GPU to finish the step before it can enqueue
the next one.  Here:

- ``to_host_async(t)`` snapshots ``t`` on the current stream (a device clone, so that later
  in-place writes to ``t`` by the caller cannot reach the copy), then enqueues the copy of the
  snapshot on a dedicated copy stream (default priority) into freshly allocated pinned memory,
  after that stream waits for the current stream, and returns the host tensor plus the event
  that completes it.
- ``PendingLog`` is a ``list`` of per-step records whose tensors may still be in flight; every
  read of the records (indexing, iteration, pickling) first waits for the pending copies, so
  readers always see finished values, exactly what the reference's list holds; ``clear``
  drops the records without waiting.
- ``FileWriter`` runs ``torch.save`` on a background thread once a record's copies are done;
  ``flush()`` waits for every write (the engines call it on save, detach and exit).

Saved files are the reference's formats: a plain ``list`` of dicts for
``dot_prod_log_iter_{n}.pt`` and ``{'proj', 'iter', 'batch_size'[, 'batch_idx']}`` for
``proj_iter_{iter:06d}.pt``.
"""
from __future__ import annotations

import atexit
import queue
import threading
from typing import Any, Dict, List, Optional, Tuple

import torch

_copy_streams: Dict[int, torch.cuda.Stream] = {}
_lock = threading.Lock()


def _copy_stream(idx: int) -> torch.cuda.Stream:
    with _lock:
        s = _copy_streams.get(idx)
        if s is None:
            s = torch.cuda.Stream(device=idx)   # default priority
            _copy_streams[idx] = s
    return s


def to_host_async(t: torch.Tensor) -> Tuple[torch.Tensor, Optional[torch.cuda.Event]]:
    """Host copy of `t`: for a CUDA tensor, a pinned tensor filled on the copy stream and the
    event that marks its completion; CPU tensors are returned as a private copy with no
    event."""
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        return (t.detach().clone() if isinstance(t, torch.Tensor) else t), None
    idx = t.device.index if t.device.index is not None else torch.cuda.current_device()
    cs = _copy_stream(idx)
    host = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
    with torch.cuda.device(idx):
        src = t.detach().clone()   # ordered before anything the caller enqueues on t later
    cs.wait_stream(torch.cuda.current_stream(idx))
    with torch.cuda.stream(cs):
        host.copy_(src, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(cs)
    src.record_stream(cs)
    return host, ev


def tree_to_host_async(data: Any, events: List[torch.cuda.Event]) -> Any:
    """``to_host_async`` over a tensor or a dict of tensors (the shapes the engines log)."""
    if isinstance(data, dict):
        return {k: tree_to_host_async(v, events) for k, v in data.items()}
    if isinstance(data, torch.Tensor):
        host, ev = to_host_async(data)
        if ev is not None:
            events.append(ev)
        return host
    return data


class PendingLog(list):
    """A list of records whose host copies may still be in flight; reads wait for them."""

    def __init__(self, *args):
        super().__init__(*args)
        self._pending: List[torch.cuda.Event] = []

    def append_pending(self, record: Dict[str, Any], events: List[torch.cuda.Event]) -> None:
        self._pending.extend(events)
        super().append(record)

    def resolve(self) -> None:
        pending, self._pending = self._pending, []
        for ev in pending:
            ev.synchronize()

    def plain(self) -> list:
        """A plain ``list`` with every copy finished (what gets saved)."""
        self.resolve()
        return list(super().__iter__())

    def __getitem__(self, i):
        self.resolve()
        return super().__getitem__(i)

    def __iter__(self):
        self.resolve()
        return super().__iter__()

    def __len__(self):
        return super().__len__()

    def __reduce_ex__(self, protocol):
        return (list, (self.plain(),))

    def clear(self):
        # The records are dropped unread, so their copies need not be waited for: the pinned
        # buffers are not reused before the copy stream has passed the copies (torch's host
        # allocator tracks non-blocking copies), and the device snapshots were marked in use
        # by the copy stream.
        self._pending = []
        super().clear()


class FileWriter:
    """``torch.save`` on a background thread after the record's copies complete."""

    def __init__(self):
        self._q: "queue.Queue" = queue.Queue()
        self._thread: Optional[threading.Thread] = None
        self._error: Optional[BaseException] = None
        self._lock = threading.Lock()

    def _run(self):
        while True:
            item = self._q.get()
            try:
                if item is None:
                    return
                obj, path, events = item
                for ev in events:
                    ev.synchronize()
                torch.save(obj, path)
            except BaseException as e:  # reported by the next flush()
                self._error = e
            finally:
                self._q.task_done()

    def submit(self, obj: Any, path, events: List[torch.cuda.Event]) -> None:
        if not events:   # nothing in flight (host tensors): write now, in order
            self.flush()
            torch.save(obj, path)
            return
        with self._lock:
            if self._thread is None or not self._thread.is_alive():
                self._thread = threading.Thread(target=self._run, name="ghost-file-writer",
                                                daemon=True)
                self._thread.start()
        self._q.put((obj, path, events))

    def flush(self) -> None:
        """Waits for every submitted write; re-raises the first write error."""
        if self._thread is not None:
            self._q.join()
        if self._error is not None:
            err, self._error = self._error, None
            raise err


writer = FileWriter()
atexit.register(lambda: writer.flush())
