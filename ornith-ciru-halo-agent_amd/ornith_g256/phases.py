"""Phase plans for mixed prefill/decode batches.

When a batch mixes requests still consuming their prompt (prefill) with
requests verifying generated tokens (decode), the reference keeps each
request's precision stable by running decode rows on the A8 entries and
prefill rows on the A4 routed entry and the bf16 dense GEMM
(plugin-site/ornith_g256/phase_dispatch.py:13-34, consumed by
native.py:121-170).  A plan is the tuple of maximal runs of consecutive
same-phase rows, (start, end, is_prefill); it is only used for batches of
more than 64 rows that really mix the two phases.

``plan_segments`` builds a plan from per-request token counts and phases;
``native.phase_segments(plan)`` applies one to the ops called inside it.
``install_vllm_hook`` wires both into vLLM's model runner when vLLM is
importable (it is not required by anything else in this package).
"""
from __future__ import annotations

from typing import Iterable, Sequence

MIN_MIXED_ROWS = 64      # plans apply to batches of more than this many rows


def plan_segments(counts: Sequence[int], prefill: Sequence[bool]) -> tuple:
    """Per-request scheduled token counts and phases (in batch order) ->
    ((start, end, is_prefill), ...) with consecutive same-phase requests
    merged; () when the batch has at most 64 rows or a single phase."""
    if len(counts) != len(prefill):
        raise ValueError(f'{len(counts)} token counts for {len(prefill)} phases')
    segments: list[tuple[int, int, bool]] = []
    row = 0
    for n, p in zip(counts, prefill):
        n = int(n)
        if n < 0:
            raise ValueError(f'negative token count {n}')
        if n == 0:
            continue
        p = bool(p)
        if segments and segments[-1][2] == p:
            segments[-1] = (segments[-1][0], row + n, p)
        else:
            segments.append((row, row + n, p))
        row += n
    phases = {p for _, _, p in segments}
    if row <= MIN_MIXED_ROWS or len(phases) < 2:
        return ()
    return tuple(segments)


def step_runs(counts: Sequence[int], prefill: Sequence[bool]) -> tuple:
    """The same runs as plan_segments without its size and mixing filter:
    the phase of every row of the step (the shared expert's decode rows)."""
    if len(counts) != len(prefill):
        raise ValueError(f'{len(counts)} token counts for {len(prefill)} phases')
    runs: list[tuple[int, int, bool]] = []
    row = 0
    for n, p in zip(counts, prefill):
        n, p = int(n), bool(p)
        if n < 0:
            raise ValueError(f'negative token count {n}')
        if n and runs and runs[-1][2] == p:
            runs[-1] = (runs[-1][0], row + n, p)
        elif n:
            runs.append((row, row + n, p))
        row += n
    return tuple(runs)


def request_phases(num_computed: Iterable[int], num_prompt: Iterable[int]) -> list[bool]:
    """A request is in prefill while fewer tokens than its prompt have been
    computed (phase_dispatch.py:15)."""
    return [int(c) < int(p) for c, p in zip(num_computed, num_prompt)]


def install_vllm_hook():
    """Wrap vLLM's GPUModelRunner so every step runs under the phase plan of
    its scheduled batch.  Raises ImportError when vLLM is not installed."""
    from vllm.v1.worker.gpu_model_runner import GPUModelRunner

    from . import native

    if getattr(GPUModelRunner, '_ornith_phase_hook', False):
        return
    prepare_inputs, execute_model = GPUModelRunner._prepare_inputs, GPUModelRunner.execute_model

    def prepare(self, scheduler_output, num_scheduled_tokens):
        batch = self.input_batch
        n = batch.num_reqs
        phases = request_phases(batch.num_computed_tokens_cpu[:n], batch.num_prompt_tokens[:n])
        counts = [int(v) for v in num_scheduled_tokens]
        plan = plan_segments(counts, phases)
        self._ornith_phase_token = native._phase_plan.set(plan)
        self._ornith_step_token = native._step_phases.set(step_runs(counts, phases))
        return prepare_inputs(self, scheduler_output, num_scheduled_tokens)

    def execute(self, *args, **kwargs):
        try:
            return execute_model(self, *args, **kwargs)
        finally:
            token = getattr(self, '_ornith_phase_token', None)
            if token is not None:
                native._phase_plan.reset(token)
                self._ornith_phase_token = None
            token = getattr(self, '_ornith_step_token', None)
            if token is not None:
                native._step_phases.reset(token)
                self._ornith_step_token = None

    GPUModelRunner._prepare_inputs, GPUModelRunner.execute_model = prepare, execute
    GPUModelRunner._ornith_phase_hook = True
