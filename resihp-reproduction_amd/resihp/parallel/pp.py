"""One pipeline stage's 1F1B micro-batch order, executed on one GPU.

Restates the issue order of ``PipelineRuntime.train_step`` (resihp/parallel/pp.py:
341-426): warmup forwards, then one forward and the oldest in-flight backward per
steady step, then the cooldown backwards, with the loss of the last stage scaled
by the global micro-batch count (pp.py:375-384) and gradients accumulating over
micro-batches (pp.py:355,393-404).  The point-to-point activation/gradient
exchanges with neighbouring stages are collectives and are not part of this
package: the caller supplies each micro-batch's received activation and
returned gradient, exactly what those exchanges would have delivered.
"""

from __future__ import annotations

from ..planner.pp import pipeline_phases
from ..reference import next_token_loss


def run_1f1b(stage, *, stage_index: int, num_stages: int, inputs=None, tokens=None, grads=None):
    """Run every micro-batch's forward and backward in 1F1B order; return the issued order.

    ``inputs[i]``: micro-batch i's received activation (ignored on a first stage, which
    embeds ``tokens[i]`` instead).  ``grads[i]``: the gradient of micro-batch i's output
    sent back by the next stage (ignored on a last stage, which backpropagates its loss).
    Returns ``(order, total_loss)``; ``total_loss`` is ``None`` unless the stage is last.
    """
    if stage.is_last and stage.tp_size > 1:
        # The reference scores the all-gathered full-vocabulary logits (pp.py:375-384 after
        # tp.py:92-110); one rank's stage only holds its [batch, seq, vocab/tp] slice, and a
        # cross-entropy over that slice has the wrong normaliser (and no target for most rows).
        raise NotImplementedError(
            "run_1f1b on a last stage with tp_size > 1 needs the all-gathered logits of every TP rank; "
            "this build computes one rank per GPU without collectives"
        )
    count = len(tokens) if stage.is_first else len(inputs)
    if not stage.is_last and (grads is None or len(grads) != count):
        raise ValueError("a non-last stage needs one returned gradient per micro-batch")
    if stage.is_last and (tokens is None or len(tokens) != count):
        raise ValueError("a last stage needs the tokens of every micro-batch for its loss")
    order: list[str] = []
    held: list[tuple[int, object]] = []
    total = None
    next_forward = 0

    def forward():
        nonlocal next_forward, total
        i = next_forward
        next_forward += 1
        order.append(f"F{i}")
        out = stage(tokens=tokens[i]) if stage.is_first else stage(hidden=inputs[i])
        if stage.is_last:
            out = next_token_loss(out, tokens[i], stage.vocab_size // stage.tp_size) / count
            total = out.detach() if total is None else total + out.detach()
        held.append((i, out))

    def backward():
        i, out = held.pop(0)  # the oldest in-flight micro-batch retires first
        order.append(f"B{i}")
        if stage.is_last:
            out.backward()
        else:
            out.backward(grads[i])

    warmup, steady = pipeline_phases(count, stage_index=stage_index, num_stages=num_stages)
    for _ in range(warmup):
        forward()
    for _ in range(steady):
        forward()
        backward()
    for _ in range(warmup):
        backward()
    return order, total
