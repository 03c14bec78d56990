"""One tensor-parallel rank's shard of a pipeline stage, on the HIP kernels.

Mirrors ``TensorParallelStage`` / ``_TPBlock`` (resihp/parallel/tp.py:113-273):
same constructor arguments, parameter names, ``local_shards()`` layout
(q/k/v/fc1/lm_head/token embedding split on dim 0, out_proj/fc2 on dim 1,
LayerNorms and the position embedding replicated) and ``forward(*, tokens=None,
hidden=None)``.  The math is the reference's shard math:

* vocab-parallel embedding: ids outside this rank's slice give zero rows
  (tp.py:222-228), then the position embedding is added (tp.py:256-257);
* per block: LN -> local-head causal attention -> out_proj partial -> + residual,
  LN -> fc1 -> GELU -> fc2 partial -> + residual (tp.py:230-249,260-265);
* last stage: final LN and the column-parallel LM head (tp.py:266-272).

This package computes one rank on one GPU and issues no collectives.  The
Megatron ``f``/``g`` regions (tp.py:63-89) are therefore identities: the
row-parallel out_proj / fc2 outputs and the vocab-parallel embedding stay
**partial sums**, input gradients of column-parallel regions stay this rank's
partials, and the last stage returns this rank's ``[batch, seq, vocab/tp]``
logits instead of all-gathering them (tp.py:92-110).  With ``tp_size == 1``
every collective is a no-op in the reference too, and the results coincide.

The degree and rank come from ``tp_rank`` / ``tp_size`` (one GPU computing
"rank 2 of 4" has no process group to read them from, tp.py:174-176); with
neither given they are read from ``group`` when torch.distributed is
initialised, and a multi-rank group is refused because reducing across it is a
collective.
"""

import torch
import torch.distributed as dist
from torch import nn

from .. import ops
from ..config import TrainConfig


def _require_divisible(config: TrainConfig, vocab_size: int, tp_size: int) -> None:
    if config.model_dim % tp_size or config.num_heads % tp_size:
        raise ValueError("tp_size must divide model_dim and num_heads")
    if vocab_size % tp_size:
        raise ValueError("tp_size must divide vocab_size")


def _resolve_rank(group, tp_rank, tp_size) -> tuple[int, int]:
    if tp_rank is not None or tp_size is not None:
        if tp_rank is None or tp_size is None:
            raise ValueError("give both tp_rank and tp_size")
        if tp_size < 1 or not 0 <= tp_rank < tp_size:
            raise ValueError(f"tp_rank {tp_rank} is not a rank of a degree-{tp_size} group")
        return tp_rank, tp_size
    if dist.is_available() and dist.is_initialized():
        size = dist.get_world_size(group)
        if size > 1:
            raise NotImplementedError(
                "this build computes one TP rank per GPU without collectives; pass tp_rank/tp_size "
                "to compute that rank's shard (row-parallel outputs are returned as partial sums)"
            )
        return dist.get_rank(group), size
    return 0, 1


class _TPBlock(nn.Module):
    """One Transformer block's local shards and replicated LayerNorms (tp.py:113-148)."""

    def __init__(self, local_state: dict, gid: int):
        super().__init__()
        prefix = f"layers.{gid}"

        def take(suffix):
            return nn.Parameter(local_state[f"{prefix}.{suffix}"].detach().clone())

        self.attn_norm_weight = take("attn_norm.weight")
        self.attn_norm_bias = take("attn_norm.bias")
        self.q_proj = take("attn.q_proj.weight")
        self.k_proj = take("attn.k_proj.weight")
        self.v_proj = take("attn.v_proj.weight")
        self.out_proj = take("attn.out_proj.weight")
        self.mlp_norm_weight = take("mlp_norm.weight")
        self.mlp_norm_bias = take("mlp_norm.bias")
        self.fc1 = take("mlp.fc1.weight")
        self.fc2 = take("mlp.fc2.weight")

    def local_shards(self, gid: int) -> dict[str, tuple[nn.Parameter, int | None]]:
        prefix = f"layers.{gid}"
        return {
            f"{prefix}.attn_norm.weight": (self.attn_norm_weight, None),
            f"{prefix}.attn_norm.bias": (self.attn_norm_bias, None),
            f"{prefix}.attn.q_proj.weight": (self.q_proj, 0),
            f"{prefix}.attn.k_proj.weight": (self.k_proj, 0),
            f"{prefix}.attn.v_proj.weight": (self.v_proj, 0),
            f"{prefix}.attn.out_proj.weight": (self.out_proj, 1),
            f"{prefix}.mlp_norm.weight": (self.mlp_norm_weight, None),
            f"{prefix}.mlp_norm.bias": (self.mlp_norm_bias, None),
            f"{prefix}.mlp.fc1.weight": (self.fc1, 0),
            f"{prefix}.mlp.fc2.weight": (self.fc2, 1),
        }


class TensorParallelStage(nn.Module):
    """A pipeline stage's layers as computed by one TP rank (tp.py:151-273)."""

    def __init__(
        self,
        config: TrainConfig,
        *,
        vocab_size: int,
        sequence_length: int,
        layer_ids,
        is_first: bool,
        is_last: bool,
        local_state: dict,
        group=None,
        tp_rank: int | None = None,
        tp_size: int | None = None,
    ):
        super().__init__()
        self.group = group
        self.tp_rank, self.tp_size = _resolve_rank(group, tp_rank, tp_size)
        _require_divisible(config, vocab_size, self.tp_size)

        self.config = config
        self.vocab_size = vocab_size
        self.sequence_length = sequence_length
        self.num_heads = config.num_heads
        self.dim = config.model_dim
        self.layer_ids = tuple(sorted(int(gid) for gid in layer_ids))
        self.is_first = bool(is_first)
        self.is_last = bool(is_last)
        self.vocab_per_rank = vocab_size // self.tp_size
        self.vocab_start = self.tp_rank * self.vocab_per_rank

        def take(name):
            return nn.Parameter(local_state[name].detach().clone())

        if self.is_first:
            self.token_embedding = take("token_embedding.weight")
            self.position_embedding = take("position_embedding.weight")
        self.blocks = nn.ModuleDict({str(gid): _TPBlock(local_state, gid) for gid in self.layer_ids})
        if self.is_last:
            self.final_norm_weight = take("final_norm.weight")
            self.final_norm_bias = take("final_norm.bias")
            self.lm_head = take("lm_head.weight")

    def local_shards(self) -> dict[str, tuple[nn.Parameter, int | None]]:
        shards: dict[str, tuple[nn.Parameter, int | None]] = {}
        if self.is_first:
            shards["token_embedding.weight"] = (self.token_embedding, 0)
            shards["position_embedding.weight"] = (self.position_embedding, None)
        for gid in self.layer_ids:
            shards.update(self.blocks[str(gid)].local_shards(gid))
        if self.is_last:
            shards["final_norm.weight"] = (self.final_norm_weight, None)
            shards["final_norm.bias"] = (self.final_norm_bias, None)
            shards["lm_head.weight"] = (self.lm_head, 0)
        return shards

    def logical_state_dict(self) -> dict[str, nn.Parameter]:
        return {name: param for name, (param, _dim) in self.local_shards().items()}

    def _block(self, block: _TPBlock, x: torch.Tensor) -> torch.Tensor:
        return ops.transformer_block(
            x,
            block.attn_norm_weight,
            block.attn_norm_bias,
            block.q_proj,
            block.k_proj,
            block.v_proj,
            block.out_proj,
            block.mlp_norm_weight,
            block.mlp_norm_bias,
            block.fc1,
            block.fc2,
            self.num_heads // self.tp_size,
        )

    def forward(self, *, tokens=None, hidden=None):
        """Embed ``tokens`` (first stage) or continue from ``hidden``; this rank's logits on the last."""
        if self.is_first:
            if tokens.shape[1] != self.sequence_length:
                raise ValueError("token sequence length does not match the stage")
            x = ops.embedding(tokens, self.token_embedding, self.position_embedding,
                              vocab_start=self.vocab_start, vocab_rows=self.vocab_per_rank)
        else:
            x = hidden
        for gid in self.layer_ids:
            x = self._block(self.blocks[str(gid)], x)
        if not self.is_last:
            return x
        x = ops.layer_norm(x, self.final_norm_weight, self.final_norm_bias)
        return ops.linear(x, self.lm_head)
