"""The 1F1B pipeline schedule: warmup forwards, steady (F, B) pairs, cooldown backwards.

Restates resihp/planner/pp.py:16-77 (``balanced_layers``, ``pipeline_phases``,
``pipeline_schedule``, ``peak_in_flight``) -- the order a pipeline stage issues
its micro-batch forwards and backwards, which the one-GPU pipeline-stage driver
in :mod:`resihp.parallel.pp` executes.  The PP repartition planner of the
reference is control-plane logic and is not part of this package.
"""


def _non_negative_int(name: str, value) -> int:
    if type(value) is not int or value < 0:
        raise ValueError(f"{name} must be a non-negative integer")
    return value


def balanced_layers(num_layers: int, num_stages: int) -> tuple[tuple[int, ...], ...]:
    """Contiguous global layer ids per stage, the remainder going to earlier stages."""
    if num_stages < 1 or num_layers < num_stages:
        raise ValueError("need at least one layer per stage")
    base, extra = divmod(num_layers, num_stages)
    out, start = [], 0
    for stage in range(num_stages):
        n = base + (1 if stage < extra else 0)
        out.append(tuple(range(start, start + n)))
        start += n
    return tuple(out)


def pipeline_phases(num_micro_batches: int, *, stage_index: int, num_stages: int) -> tuple[int, int]:
    """(warmup, steady): one warmup forward per downstream stage, capped by the micro-batch count."""
    if num_stages < 1 or not 0 <= stage_index < num_stages:
        raise ValueError("stage_index must identify a stage of the pipeline")
    _non_negative_int("num_micro_batches", num_micro_batches)
    warmup = min(num_stages - 1 - stage_index, num_micro_batches)
    return warmup, num_micro_batches - warmup


def pipeline_schedule(num_micro_batches: int, *, stage_index: int, num_stages: int) -> tuple[str, ...]:
    """'F'/'B' in issue order: warmup forwards, steady (F, B) pairs, cooldown backwards."""
    warmup, steady = pipeline_phases(num_micro_batches, stage_index=stage_index, num_stages=num_stages)
    return ("F",) * warmup + ("F", "B") * steady + ("B",) * warmup


def peak_in_flight(num_micro_batches: int, *, stage_index: int, num_stages: int) -> int:
    """Most activations held at once, replayed from the schedule (+1 per F, -1 per B)."""
    live = peak = 0
    for op in pipeline_schedule(num_micro_batches, stage_index=stage_index, num_stages=num_stages):
        live += 1 if op == "F" else -1
        peak = max(peak, live)
    return peak
