"""Per-stage HIP-event timing of the forward/backward pipeline.

Plays the role of the reference's MOE_FWD_TIMING / MOE_BWD_STAGE_TIMING
stage stamps (kernels/common.py:86-130, ops/backward.py:216-347): when a
``StageTimer`` is attached to an operator, events are recorded on the launch
stream between stages and ``summary()`` returns the mean milliseconds of each
stage over the recorded passes. Without a timer nothing is recorded.
``MOE_FWD_TIMING=1`` attaches a timer to every new ``FusedMoEForward``;
``MOE_BWD_STAGE_TIMING=1`` times each backward pass on its own.
"""

from __future__ import annotations

from collections import defaultdict

import torch


class StageTimer:
    def __init__(self):
        self._events = []          # list of (name, start_event, end_event)
        self._open = None
        self._pass_start = 0       # index of the current pass's first event

    def begin(self, name: str):
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        self._open = (name, ev)

    def end(self):
        name, start = self._open
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        self._events.append((name, start, ev))
        self._open = None

    def reset(self):
        self._events.clear()
        self._pass_start = 0

    def mark_pass(self):
        """Start a new pass: ``last_pass`` reports only stages recorded after
        this call."""
        self._pass_start = len(self._events)

    def last_pass(self) -> dict:
        """Milliseconds of each stage recorded since the last ``mark_pass``
        (the latest recording of a name wins; synchronises)."""
        torch.cuda.synchronize()
        out = {}
        for name, a, b in self._events[self._pass_start:]:
            out[name] = a.elapsed_time(b)
        return out

    def summary(self) -> dict:
        """Mean ms per stage name (synchronises)."""
        torch.cuda.synchronize()
        acc, cnt = defaultdict(float), defaultdict(int)
        for name, a, b in self._events:
            acc[name] += a.elapsed_time(b)
            cnt[name] += 1
        return {k: acc[k] / cnt[k] for k in acc}


class _NullTimer:
    def begin(self, name):
        pass

    def mark_pass(self):
        pass

    def end(self):
        pass


NULL_TIMER = _NullTimer()
