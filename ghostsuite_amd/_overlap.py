"""Side-stream execution of the per-layer dot-product kernels, overlapped with the rest of
the backward pass.

A backward hook enqueues its layer's dot kernels on a second HIP stream (default priority)
after that stream has waited for everything the autograd stream enqueued so far.  The
hook's input tensors are marked as in use by the side stream, so the caching allocator
does not hand their memory back to the autograd stream before the side kernels finish.
At the end of the backward pass an autograd-engine callback makes the autograd stream wait
for the side stream, so the optimizer, the engines' aggregation and any host copy see
finished results.  ``join(device)`` does the same wait explicitly (the engines call it
before reading results, which also covers a backward pass that raised).

Memory written on the side stream and later read on the autograd stream needs no extra
bookkeeping: every later side-stream launch is preceded by a wait on the autograd stream.
"""
from __future__ import annotations

import contextlib
import threading
from typing import Dict

import torch

_lock = threading.Lock()
_streams: Dict[int, torch.cuda.Stream] = {}
_join_queued: Dict[int, bool] = {}

enabled = True


def side_stream(device: torch.device) -> torch.cuda.Stream:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    with _lock:
        s = _streams.get(idx)
        if s is None:
            s = torch.cuda.Stream(device=idx)   # default priority
            _streams[idx] = s
    return s


def join(device=None) -> None:
    """The current stream of `device` waits for the side stream's work so far."""
    if not _streams:
        return
    devices = [device] if device is not None else [torch.device("cuda", i) for i in _streams]
    for dev in devices:
        dev = torch.device(dev)
        if dev.type != "cuda":
            continue
        idx = dev.index if dev.index is not None else torch.cuda.current_device()
        s = _streams.get(idx)
        if s is not None:
            torch.cuda.current_stream(idx).wait_stream(s)
        _join_queued.pop(idx, None)


def _queue_join(idx: int, cur: torch.cuda.Stream, side: torch.cuda.Stream) -> None:
    if _join_queued.get(idx):
        return

    def _end_of_backward():
        cur.wait_stream(side)
        _join_queued.pop(idx, None)

    try:
        torch.autograd.Variable._execution_engine.queue_callback(_end_of_backward)
        _join_queued[idx] = True
    except RuntimeError:
        # Not inside a backward pass: order the side work before anything enqueued later.
        cur.wait_stream(side)
        _join_queued.pop(idx, None)


@contextlib.contextmanager
def on_side_stream(*tensors):
    """Runs the body on the side stream of the tensors' device (no-op on CPU or when
    disabled).  The tensors are the body's inputs produced on the current stream."""
    ts = [t for t in tensors if isinstance(t, torch.Tensor)]
    if not enabled or not ts or ts[0].device.type != "cuda":
        yield
        return
    dev = ts[0].device
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    side = side_stream(dev)
    cur = torch.cuda.current_stream(idx)
    side.wait_stream(cur)
    for t in ts:
        t.record_stream(side)
    if torch.cuda.current_device() == idx:
        # Same device: switch the current stream only (the stream context manager also
        # saves and restores the current device, several times the cost per hook).
        torch.cuda.set_stream(side)
        try:
            yield
        finally:
            torch.cuda.set_stream(cur)
    else:
        with torch.cuda.stream(side):
            yield
    _queue_join(idx, cur, side)
