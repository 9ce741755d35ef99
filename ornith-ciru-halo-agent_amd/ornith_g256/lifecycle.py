"""Per-step lifecycle of the sticky native error flags.

Every launch of the library ORs error bits into a caller-owned uint32 flag
(one slot per layer) and never clears it.  A serving worker therefore, per
model step (the reference's plugin-site/ornith_g256/lifecycle.py:69-193):

  1. clears the flags before the step's first launch (never inside a graph
     capture: the clear is a kernel in eager mode);
  2. after the step's launches, queues one device-to-host copy of all flag
     slots into preallocated pinned memory and records an event behind it;
  3. before handing the step's output on, waits for that event and checks
     the copy; any set bit poisons the worker: that step and every later one
     raise ``OrnithWorkerFault`` (the arena may hold garbage; the process is
     to be replaced, not reused).

Steps complete in order: completing step n first checks every earlier step,
so a healthy later step never hides an earlier fault.  Snapshot slots come
from a bounded pool (``max_inflight``).  The device side is behind a small
transport interface so the policy runs on the CPU in tests.
"""
from __future__ import annotations

import threading
from collections import deque
from dataclasses import dataclass, field


class OrnithWorkerFault(RuntimeError):
    """A native error flag was raised; this worker must not deliver more outputs."""


@dataclass
class Ticket:
    sequence: int
    name: str
    slot: object
    queued: bool = False
    done: bool = False
    flags: tuple = field(default_factory=tuple)


class TorchFlagTransport:
    """Flags live in one int32 CUDA tensor; snapshots go to pinned host
    tensors behind an event on the current stream."""

    def __init__(self, flags):
        import torch
        if flags.device.type != 'cuda' or flags.dtype != torch.int32 or flags.ndim != 1:
            raise ValueError('flags must be a 1-D int32 CUDA tensor (one slot per layer)')
        self.torch, self.flags = torch, flags
        self.blocking_waits = 0

    def _outside_capture(self):
        with self.torch.cuda.device(self.flags.device):
            if self.torch.cuda.is_current_stream_capturing():
                raise RuntimeError('the flag lifecycle must not run inside a graph capture')

    def width(self):
        return self.flags.numel()

    def new_slot(self):
        self._outside_capture()
        torch = self.torch
        return (torch.empty(self.flags.numel(), dtype=torch.int32, pin_memory=True), torch.cuda.Event())

    def clear(self):
        self._outside_capture()
        self.flags.zero_()

    def queue(self, slot):
        self._outside_capture()
        host, event = slot
        with self.torch.cuda.device(self.flags.device):
            host.copy_(self.flags, non_blocking=True)
            event.record(self.torch.cuda.current_stream(self.flags.device))

    def finish(self, slot):
        host, event = slot
        if not event.query():
            self.blocking_waits += 1
            event.synchronize()
        return tuple(int(v) for v in host.tolist())


class StepLifecycle:
    """Clear / snapshot / check the flags of each worker step (see module doc).
    `names` labels the flag slots (layer prefixes) in fault messages."""

    def __init__(self, names, max_inflight=2, transport=None, flags=None):
        if not isinstance(max_inflight, int) or not 1 <= max_inflight <= 64:
            raise ValueError('max_inflight must be an int in 1..64')
        self.names = tuple(names)
        self.transport = transport if transport is not None else TorchFlagTransport(flags)
        if self.transport.width() != len(self.names):
            raise ValueError(f'{len(self.names)} names for {self.transport.width()} flag slots')
        self._free = deque(self.transport.new_slot() for _ in range(max_inflight))
        self._pending: dict[int, Ticket] = {}
        self._next = 0
        self._fault: OrnithWorkerFault | None = None
        self._lock = threading.RLock()
        self.clears = self.snapshots = self.completed = 0

    # -- state ---------------------------------------------------------------
    @property
    def fault(self):
        return self._fault

    def raise_if_faulted(self):
        if self._fault is not None:
            raise self._fault

    def _poison(self, error, message):
        if self._fault is None:
            self._fault = OrnithWorkerFault(message)
            self._fault.__cause__ = error

    # -- step API --------------------------------------------------------------
    def begin(self, name):
        """Start a step: take a snapshot slot and clear the device flags."""
        with self._lock:
            self.raise_if_faulted()
            if not self._free:
                raise RuntimeError(f'all {len(self._pending)} flag snapshot slots are in flight')
            slot = self._free.popleft()
            try:
                self.transport.clear()
            except BaseException as error:
                self._free.appendleft(slot)
                self._poison(error, f'clearing the native flags failed: {error!r}')
                raise
            ticket = Ticket(self._next, str(name), slot)
            self._next += 1
            self._pending[ticket.sequence] = ticket
            self.clears += 1
            return ticket

    def snapshot(self, ticket):
        """Queue the device-to-host copy of the flags after the step's launches."""
        with self._lock:
            if ticket.done or ticket.sequence not in self._pending:
                raise RuntimeError(f'step {ticket.sequence} is not pending')
            if ticket.queued:
                return
            try:
                self.transport.queue(ticket.slot)
            except BaseException as error:
                self._poison(error, f'queueing the flag snapshot failed: {error!r}')
                raise
            ticket.queued = True
            self.snapshots += 1

    def complete(self, ticket):
        """Check this step and every earlier pending one; returns its flags or
        raises OrnithWorkerFault if any checked step had a flag set."""
        with self._lock:
            for seq in sorted(self._pending):
                if seq > ticket.sequence:
                    break
                step = self._pending[seq]
                if not step.queued:
                    raise RuntimeError(f'step {seq} ({step.name}) completes before its flags were snapshotted')
                try:
                    values = self.transport.finish(step.slot)
                except BaseException as error:
                    self._poison(error, f'reading the flag snapshot failed: {error!r}')
                    raise
                if len(values) != len(self.names):
                    self._poison(None, f'snapshot of {len(values)} slots, expected {len(self.names)}')
                step.flags, step.done = tuple(values), True
                if any(values):
                    raised = {n: v for n, v in zip(self.names, values) if v}
                    self._poison(None, f'native error flags in step {seq} ({step.name}): {raised}')
                del self._pending[seq]
                self._free.append(step.slot)
                self.completed += 1
            self.raise_if_faulted()
            if not ticket.done:
                raise RuntimeError(f'unknown step {ticket.sequence}')
            return ticket.flags

    def abort(self, ticket, error):
        """An exception escaped the step: capture its flags if possible, poison
        the worker and re-raise (chained with a flag fault if there is one)."""
        try:
            if not ticket.done:
                self.snapshot(ticket)
                self.complete(ticket)
        except OrnithWorkerFault as fault:
            raise fault from error
        except BaseException as secondary:
            error.add_note(f'flag capture also failed: {secondary!r}')
        with self._lock:
            self._poison(error, f'worker step {ticket.sequence} ({ticket.name}) failed: {error!r}')
        raise error

    def drain(self):
        """Snapshot and check every pending step (shutdown, error boundaries)."""
        with self._lock:
            pending = [self._pending[s] for s in sorted(self._pending)]
        for t in pending:
            if not t.queued:
                self.snapshot(t)
        if pending:
            self.complete(pending[-1])
        self.raise_if_faulted()
