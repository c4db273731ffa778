"""One continuous-batching step of one GDN layer as one launch set.

multiplex's scheduler runs, in one engine step, prefill chunks of new
sequences next to decode and speculative-verify rounds of running ones
(``multiplex/kernel/scheduler.py:299-363`` for the prefill chunks,
``:463-608`` for a decode / verify round and its rollback).  On one MI355X
those rows are independent launches of the same layer:

* the packed prefills are one chunked launch (``prepare_chunked`` with
  ``cu_seqlens``), whose two phases differ in what they load: the prep is
  HBM-bound (it streams q, k and writes the chunk records), the scan is a
  sequential chain per head that leaves HBM mostly idle;
* the decode, verify and commit launches of the other rows
  (``prepare_recurrent``) are HBM-bound state streams.

:class:`MixedStep` has two schedules.  ``launch_serial()`` issues prep,
scan and the other launches in order on the caller's stream.
``launch_overlapped()`` issues the prep on the caller's stream, records an
event (one without a system-scope fence: it only orders), issues the scan
behind it, and runs the other launches on a second stream (default
priority) that waits for that event, so the HBM-bound launches overlap the
scan rather than the prep; the caller's stream then waits for the second
stream, so work issued after it sees every output.
Every launch writes disjoint outputs (separate rows and states), so the two
schedules give bit-identical results.

``launch()`` takes the schedule chosen at construction, overlapped by
default (the step of 1024 + 2560 + 7168 prefill tokens, 48 decode rows and
16 verify rows, with the verify and commit issued before the decode: 0.324 ms
overlapped, 0.339 ms on one stream).
"""

from __future__ import annotations

import ctypes
from typing import Optional, Sequence

import torch

from .gated_delta import PreparedChunked, PreparedRecurrent

__all__ = ["MixedStep"]

_HIP_EVENT_DISABLE_TIMING = 0x2
_HIP_EVENT_DISABLE_SYSTEM_FENCE = 0x20000000
_hip = None


def _hip_runtime():
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")  # torch's HIP runtime, already loaded
    return _hip


class _OrderEvent:
    """A HIP event that orders one stream's later work after another's, with
    no system-scope fence when recorded.

    The prep's completion only has to gate *when* the side stream's launches
    start (they read nothing the prep writes), so the cache write-back and
    invalidation of a default event buy nothing there; on the mixed step that
    fence left the caller's stream idle between the prep and the scan, and
    the step took 2.5 us longer (326.9-327.6 against 324.4-325.4 us).
    """

    def __init__(self, device):
        self._hip = _hip_runtime()
        self._ev = ctypes.c_void_p()
        with torch.cuda.device(device):
            rc = self._hip.hipEventCreateWithFlags(
                ctypes.byref(self._ev), ctypes.c_uint(_HIP_EVENT_DISABLE_TIMING | _HIP_EVENT_DISABLE_SYSTEM_FENCE))
        if rc != 0:
            raise RuntimeError(f"hipEventCreateWithFlags failed ({rc})")

    def record(self, stream: torch.cuda.Stream):
        rc = self._hip.hipEventRecord(self._ev, ctypes.c_void_p(stream.cuda_stream))
        if rc != 0:
            raise RuntimeError(f"hipEventRecord failed ({rc})")

    def wait(self, stream: torch.cuda.Stream):
        rc = self._hip.hipStreamWaitEvent(ctypes.c_void_p(stream.cuda_stream), self._ev, ctypes.c_uint(0))
        if rc != 0:
            raise RuntimeError(f"hipStreamWaitEvent failed ({rc})")

    def __del__(self):
        if getattr(self, "_ev", None) is not None and self._ev.value:
            self._hip.hipEventDestroy(self._ev)


class MixedStep:
    """A prepared prefill plus prepared recurrent launches, issued as one step.

    ``prefill``: a :class:`PreparedChunked` (the packed prefills), or None.
    ``others``: prepared recurrent launches (decode, verify, commit), issued
    in order after the prefill (on the side stream when overlapped).
    ``side``: the second stream of the overlapped schedule (created with
    default priority when not given).  ``overlap``: whether ``launch()``
    takes the overlapped schedule.
    """

    def __init__(self, prefill: Optional[PreparedChunked], others: Sequence[PreparedRecurrent],
                 side: Optional[torch.cuda.Stream] = None, overlap: bool = True):
        self.prefill = prefill
        self.others = list(others)
        devs = {p.device for p in self.others} | ({prefill.device} if prefill is not None else set())
        if len(devs) != 1:
            raise ValueError("a mixed step runs on one device")
        self.device = devs.pop()
        self.overlap = bool(overlap)
        self.side = side if side is not None else torch.cuda.Stream(self.device)
        self._prep_done = _OrderEvent(self.device)

    def launch(self, stream=None):
        """Enqueues the step with the schedule chosen at construction."""
        if self.overlap:
            self.launch_overlapped(stream)
        else:
            self.launch_serial(stream)

    def launch_overlapped(self, stream=None):
        """Enqueues the step: prep, then scan on ``stream`` (default: the
        current stream); the other launches on the side stream once the prep
        is done; ``stream`` waits for the side stream at the end."""
        main = stream if stream is not None else torch.cuda.current_stream(self.device)
        if self.prefill is not None:
            self.prefill.launch_prep(main)
            self._prep_done.record(main)
            self.prefill.launch_scan(main)
            self._prep_done.wait(self.side)
        else:
            self.side.wait_stream(main)
        for p in self.others:
            p.launch(self.side)
        main.wait_stream(self.side)

    def launch_serial(self, stream=None):
        """The same launches, in the same order, on one stream."""
        main = stream if stream is not None else torch.cuda.current_stream(self.device)
        if self.prefill is not None:
            self.prefill.launch(main)
        for p in self.others:
            p.launch(main)
