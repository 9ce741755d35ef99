"""Per-step checking of the library's sticky error flags.

Every launch ORs error bits into a caller-owned int32 flag tensor (one slot
per layer) and never clears it.  A serving worker checks them once per model
step, with the policy of the reference plugin (plugin-site/ornith_g256/
lifecycle.py:69-193):

  * the flags are zeroed before a step's first launch (eagerly, never inside
    a graph capture);
  * after the step's launches one device-to-host copy of every slot goes
    into pinned host memory, with an event behind it on the same stream;
  * before a step's output is handed on, that copy (and the copy of every
    earlier step) is read; any set bit poisons the worker, and from then on
    every call raises ``OrnithWorkerFault`` (the arena may hold garbage: the
    process is to be replaced, not reused).

This module's design: steps are plain increasing integers.  Snapshots live
in a ring of ``depth`` rows of one pinned [depth, slots] tensor; step s uses
row s % depth, so at most ``depth`` steps can be open (begun and not yet
checked) at once.  The checker keeps one watermark, ``checked``: every step
below it has been read and found clean.  ``check_through(s)`` moves the
watermark over s and everything before it in sequence order, so a healthy
later step can never be delivered past an earlier faulty one.

The device side is a ``PinnedFlagRing`` (zero, capture into a row, read a
row); the CPU tests substitute one that keeps the flags in a Python list.
"""
from __future__ import annotations

import threading


class OrnithWorkerFault(RuntimeError):
    """A native error flag was raised; this worker must not deliver more outputs."""


class PinnedFlagRing:
    """Device flags (1-D int32 CUDA tensor) and a pinned [depth, slots] ring of
    host snapshots, each row with the event recorded behind its copy."""

    def __init__(self, flags, depth):
        import torch
        if flags.device.type != 'cuda' or flags.dtype != torch.int32 or flags.ndim != 1:
            raise ValueError('flags must be a 1-D int32 CUDA tensor (one slot per layer)')
        self._torch = torch
        self.flags = flags
        self.slots = flags.numel()
        self._host = torch.zeros((depth, self.slots), dtype=torch.int32, pin_memory=True)
        self._events = [torch.cuda.Event() for _ in range(depth)]
        self.host_waits = 0

    def _eager(self):
        with self._torch.cuda.device(self.flags.device):
            if self._torch.cuda.is_current_stream_capturing():
                raise RuntimeError('the flag checks run eagerly, not inside a graph capture')

    def zero(self):
        self._eager()
        self.flags.zero_()

    def capture(self, row):
        self._eager()
        with self._torch.cuda.device(self.flags.device):
            self._host[row].copy_(self.flags, non_blocking=True)
            self._events[row].record(self._torch.cuda.current_stream(self.flags.device))

    def read(self, row):
        event = self._events[row]
        if not event.query():
            self.host_waits += 1
            event.synchronize()
        return tuple(int(v) for v in self._host[row].tolist())


class StepFlags:
    """Open, capture and check the flags of each worker step.

    ``labels`` names the flag slots (layer prefixes) for fault messages;
    ``depth`` (1..64) bounds the steps open at once.  Pass either the device
    ``flags`` tensor or a ready ``ring`` (anything with ``slots``, ``zero``,
    ``capture(row)`` and ``read(row)``).
    """

    def __init__(self, labels, depth=2, *, flags=None, ring=None):
        if type(depth) is not int or not 1 <= depth <= 64:
            raise ValueError(f'depth must be an int in 1..64, got {depth!r}')
        self.labels = tuple(labels)
        self.ring = ring if ring is not None else PinnedFlagRing(flags, depth)
        if self.ring.slots != len(self.labels):
            raise ValueError(f'{len(self.labels)} labels for {self.ring.slots} flag slots')
        self.depth = depth
        self.issued = 0                  # next step number
        self.checked = 0                 # steps below this were read and clean
        self._captured = [-1] * depth    # step whose snapshot sits in each row
        self._step_label = [''] * depth
        self._result = {}                # step -> flags, kept until taken
        self._fault = None
        self._lock = threading.RLock()
        self.zeroed = self.captured = self.read_rows = 0

    # -- poison ------------------------------------------------------------------
    @property
    def fault(self):
        return self._fault

    def _poison(self, message, cause=None):
        if self._fault is None:
            self._fault = OrnithWorkerFault(message)
            self._fault.__cause__ = cause
        return self._fault

    def raise_if_poisoned(self):
        if self._fault is not None:
            raise self._fault

    # -- steps -------------------------------------------------------------------
    def open(self, label=''):
        """Zero the device flags and return the new step's number."""
        with self._lock:
            self.raise_if_poisoned()
            if self.issued - self.checked >= self.depth:
                raise RuntimeError(f'{self.depth} steps are open; check the oldest '
                                   f'(step {self.checked}) before opening another')
            try:
                self.ring.zero()
            except BaseException as error:
                raise self._poison(f'zeroing the native flags failed: {error!r}', error) from error
            step = self.issued
            self.issued += 1
            row = step % self.depth
            self._captured[row] = -1
            self._step_label[row] = str(label)
            self.zeroed += 1
            return step

    def _row_of(self, step):
        if not self.checked <= step < self.issued:
            raise RuntimeError(f'step {step} is not open (open: {self.checked}..{self.issued - 1})')
        return step % self.depth

    def capture(self, step):
        """Queue the copy of the flags after the step's launches (idempotent)."""
        with self._lock:
            row = self._row_of(step)
            if self._captured[row] == step:
                return
            try:
                self.ring.capture(row)
            except BaseException as error:
                raise self._poison(f'copying the native flags failed: {error!r}', error) from error
            self._captured[row] = step
            self.captured += 1

    def check_through(self, step):
        """Read the snapshots of every open step up to and including `step`,
        in order.  Returns `step`'s flags; raises OrnithWorkerFault if any of
        them (or an earlier step) had a bit set."""
        with self._lock:
            if step < self.checked and step in self._result:
                self.raise_if_poisoned()
                return self._result.pop(step)
            self._row_of(step)
            while self.checked <= step:
                s = self.checked
                row = s % self.depth
                if self._captured[row] != s:
                    raise RuntimeError(f'step {s} ({self._step_label[row]}) is checked before '
                                       'its flags were captured')
                try:
                    values = tuple(self.ring.read(row))
                except BaseException as error:
                    raise self._poison(f'reading the flag snapshot failed: {error!r}', error) from error
                self.read_rows += 1
                self.checked = s + 1
                self._captured[row] = -1
                if len(values) != len(self.labels):
                    self._poison(f'flag snapshot has {len(values)} slots, expected {len(self.labels)}')
                elif any(values):
                    bad = {name: v for name, v in zip(self.labels, values) if v}
                    self._poison(f'native error flags in step {s} ({self._step_label[row]}): {bad}')
                if s != step:
                    self._result[s] = values
                else:
                    result = values
            for old in [k for k in self._result if k < self.checked - self.depth]:
                del self._result[old]
            self.raise_if_poisoned()
            return result

    def fail(self, step, error):
        """An exception escaped `step`: capture and check its flags if that is
        still possible, poison the worker, and re-raise `error` (or the flag
        fault, chained to it)."""
        try:
            if self.checked <= step < self.issued:
                self.capture(step)
                self.check_through(step)
        except OrnithWorkerFault as fault:
            if fault is error:
                raise
            raise fault from error
        except BaseException as secondary:
            error.add_note(f'capturing the native flags also failed: {secondary!r}')
        with self._lock:
            self._poison(f'worker step {step} failed: {error!r}', error)
        raise error

    def flush(self):
        """Capture and check every open step (shutdown, error boundaries)."""
        with self._lock:
            last = self.issued - 1
            for s in range(self.checked, self.issued):
                self.capture(s)
            if last >= self.checked:
                self.check_through(last)
            self._result.clear()
            self.raise_if_poisoned()
