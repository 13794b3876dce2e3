"""Device-side error counts read without stalling the host.

Some operators count bad inputs on the device (the fused CE's out-of-range
labels, the splice's placeholder count and out-of-range ids).  Reading such a
count at once would synchronise the host with the GPU on every call, so each
call copies its counts to pinned host memory without blocking, records an
event, and the counts are judged once the copy has landed: at the operator's
next call, or when the caller asks (``check(block=True)``, e.g. at the end
of a training or evaluation loop).  Inside HIP graph capture neither the copy
nor an event query of earlier work is allowed, so captured calls are not
tracked.
"""

from __future__ import annotations

import threading
from typing import Callable

import torch


class DeferredChecks:
    """Pending device counts of one operator, each with the function that
    judges them (raises on bad values)."""

    def __init__(self) -> None:
        self._pending: list = []
        self._lock = threading.Lock()

    def add(self, counts: torch.Tensor, judge: Callable[[list], None]) -> None:
        """Tracks ``counts`` (a small int64 device tensor); ``judge`` gets its
        values as a Python list once they have landed."""
        if torch.cuda.is_current_stream_capturing():
            return
        self.check()
        host = torch.empty(counts.shape, dtype=counts.dtype, pin_memory=True)
        host.copy_(counts, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(counts.device))
        with self._lock:
            self._pending.append((ev, host, judge))

    def check(self, block: bool = False) -> None:
        """Judges every tracked call whose counts have landed (all of them when
        ``block``); the first bad one raises, and each call is judged once."""
        landed = []
        with self._lock:
            keep = []
            for ev, host, judge in self._pending:
                if block:
                    ev.synchronize()
                if ev.query():
                    landed.append((host, judge))
                else:
                    keep.append((ev, host, judge))
            self._pending[:] = keep
        for host, judge in landed:
            judge(host.reshape(-1).tolist())

    def __len__(self) -> int:
        with self._lock:
            return len(self._pending)
