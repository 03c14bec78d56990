"""Single-process reference training run, on the GPU kernels.

Keeps the reference's one loss, one optimizer, seeded token stream and
sha256 step records (resihp/reference.py:20-161): ``next_token_loss`` is the
fused cross-entropy kernel, ``adamw`` the fused AdamW update.  ``ReferenceRun``
builds the model on the CPU from ``config.seed`` exactly as the reference does
(so the init is the reference's), then moves it to ``device`` / ``dtype`` and
steps there.
"""

from dataclasses import dataclass
from hashlib import sha256

import torch

from . import ops
from .config import TrainConfig
from .model import ReferenceTransformer
from .optim import AdamW

LEARNING_RATE = 1e-3
WEIGHT_DECAY = 0.01
ADAM_BETAS = (0.9, 0.999)
ADAM_EPS = 1e-8

_OPTIM_STATES = ("exp_avg", "exp_avg_sq", "step")


def adamw(params):
    """The project's one optimizer configuration (resihp/reference.py:29-38)."""
    return AdamW(params, lr=LEARNING_RATE, betas=ADAM_BETAS, eps=ADAM_EPS, weight_decay=WEIGHT_DECAY)


def next_token_loss(logits, tokens, vocab_size):
    """Mean next-token cross-entropy over the whole batch (resihp/reference.py:41-50).

    ``logits`` [batch, seq, vocab] and ``tokens`` [batch, seq] on the same GPU.
    The shifted view ``logits[:, :-1]`` is never materialised.
    """
    return ops.next_token_loss(logits, tokens, vocab_size)


@dataclass(frozen=True)
class StepRecord:
    step: int
    tokens: tuple[tuple[int, ...], ...]
    loss: float
    param_digest: str
    optim_digest: str


def _digest(items) -> str:
    """sha256 over (name, tensor) pairs by their exact fp32 bytes (resihp/reference.py:64-72)."""
    hasher = sha256()
    for name, tensor in items:
        array = tensor.detach().cpu().to(torch.float32).contiguous().numpy()
        hasher.update(name.encode("utf-8"))
        hasher.update(repr(array.shape).encode("utf-8"))
        hasher.update(array.tobytes())
    return hasher.hexdigest()


def logical_state_digest(model) -> str:
    return _digest(sorted(model.logical_state_dict().items()))


def _optim_digest(optimizer, name_by_param) -> str:
    items = []
    for param, state in optimizer.state.items():
        name = name_by_param[param]
        for key in _OPTIM_STATES:
            value = state[key]
            tensor = value if torch.is_tensor(value) else torch.tensor(value)
            items.append((f"{name}.{key}", tensor))
    return _digest(sorted(items))


def _token_stream(vocab_size, sequence_length, batch_size, count, seed):
    """Fixed, reproducible sequence of token batches (resihp/reference.py:97-103)."""
    generator = torch.Generator().manual_seed(seed)
    return [
        torch.randint(0, vocab_size, (batch_size, sequence_length), generator=generator)
        for _ in range(count)
    ]


class ReferenceRun:
    """A resumable single-process training run (resihp/reference.py:106-150)."""

    def __init__(self, config: TrainConfig, *, vocab_size: int, sequence_length: int, device="cuda",
                 dtype=torch.float32):
        if sequence_length < 2:
            raise ValueError("sequence_length must be at least 2 for next-token loss")
        torch.manual_seed(config.seed)
        self.config = config
        self.vocab_size = vocab_size
        self.sequence_length = sequence_length
        self.device = torch.device(device)
        self.model = ReferenceTransformer(config, vocab_size=vocab_size, sequence_length=sequence_length)
        self.model.to(device=self.device, dtype=dtype)
        self.model.train()
        self.optimizer = adamw(self.model.parameters())
        self.batches = _token_stream(vocab_size, sequence_length, config.batch_size, config.iterations, config.seed)
        self.name_by_param = {param: name for name, param in self.model.named_parameters()}
        self.cursor = 0

    def step(self) -> StepRecord:
        tokens = self.batches[self.cursor]
        dev_tokens = tokens.to(self.device)
        logits = self.model(dev_tokens)
        loss = next_token_loss(logits, dev_tokens, self.vocab_size)
        self.optimizer.zero_grad()
        loss.backward()
        self.optimizer.step()
        record = StepRecord(
            step=self.cursor,
            tokens=tuple(tuple(int(t) for t in row) for row in tokens.tolist()),
            loss=float(loss.detach()),
            param_digest=logical_state_digest(self.model),
            optim_digest=_optim_digest(self.optimizer, self.name_by_param),
        )
        self.cursor += 1
        return record


def run_reference(config: TrainConfig, *, vocab_size: int, sequence_length: int, device="cuda",
                  dtype=torch.float32) -> list[StepRecord]:
    run = ReferenceRun(config, vocab_size=vocab_size, sequence_length=sequence_length, device=device, dtype=dtype)
    return [run.step() for _ in range(config.iterations)]
