"""Training configuration record consumed by the model constructors.

Restates the field set of ``TrainConfig`` (resihp/config.py:13-34) -- the model
reads ``model_dim``, ``num_layers``, ``num_heads`` and ``seed``; the parallel
degrees and iteration counts are carried for callers.  The closed-schema JSON
loader and failure-event schedule of the reference belong to its control plane
and are not part of this package.
"""

from dataclasses import dataclass


class ConfigError(ValueError):
    """Raised when a training configuration is invalid."""


@dataclass(frozen=True)
class TrainConfig:
    model_dim: int
    num_layers: int
    num_heads: int
    batch_size: int
    micro_batch_size: int
    seed: int
    tp: int
    pp: int
    dp: int
    iterations: int
    memory_budget_bytes: int | None = None

    @property
    def world_size(self) -> int:
        return self.tp * self.pp * self.dp
