"""Decoder-only Transformer with stable global layer identity, on the HIP kernels.

Same classes, constructor signatures, parameter names, shapes and initialisation
as resihp/model.py:48-137 of the reference, so ``logical_state_dict()`` names
and the seeded init are unchanged and the parallel/recovery code that consumes
them keeps working:

* ``CausalSelfAttention(model_dim, num_heads)`` -- bias-free q/k/v/out
  projections, ``ValueError`` when ``model_dim % num_heads`` (model.py:48-58);
* ``MLP(model_dim)`` -- fc1 ``model_dim -> MLP_RATIO*model_dim``, exact GELU,
  fc2 back (model.py:74-81);
* ``TransformerBlock(model_dim, num_heads)`` -- pre-LN
  ``x + attn(norm(x))`` then ``x + mlp(norm(x))`` (model.py:84-97);
* ``ReferenceTransformer(config, *, vocab_size, sequence_length)`` -- token and
  learned position embeddings, blocks keyed by global layer id in a
  ``ModuleDict``, final LayerNorm, untied bias-free LM head (model.py:100-137).

The submodules subclass ``nn.Linear`` / ``nn.LayerNorm`` / ``nn.Embedding`` so
their parameters and ``reset_parameters`` (and hence the RNG stream consumed at
construction) are exactly the reference's; only ``forward`` differs, and it
runs through :mod:`resihp.ops` on the GPU.  ``TransformerBlock.forward`` is one
fused autograd node.  Models work in float32 (the reference's precision) or
bfloat16 (``model.to(torch.bfloat16)``), always with fp32 accumulation.

The LM head returns logits as a ``[batch, seq, vocab]`` view whose row stride
is rounded up to a multiple of 8 elements, so every row starts 16-byte aligned
for the kernels that read it next.
"""

import torch
from torch import nn

from . import ops
from .config import TrainConfig

# The reference pins full-precision fp32 matmuls for every process that builds a
# model (resihp/model.py:42); kept so torch-side code behaves the same.
torch.set_float32_matmul_precision("highest")

#: MLP hidden width as a multiple of ``model_dim`` (resihp/model.py:45).
MLP_RATIO = 4


class Linear(nn.Linear):
    """Bias-free ``nn.Linear`` whose forward is the HIP GEMM."""

    def __init__(self, in_features: int, out_features: int):
        super().__init__(in_features, out_features, bias=False)

    def forward(self, x):
        return ops.linear(x, self.weight)


class LayerNorm(nn.LayerNorm):
    """``nn.LayerNorm`` over the last dim whose forward is the HIP kernel."""

    def forward(self, x):
        return ops.layer_norm(x, self.weight, self.bias, self.eps)


class Embedding(nn.Embedding):
    """``nn.Embedding`` whose forward is the HIP gather."""

    def forward(self, ids):
        return ops.embedding(ids, self.weight)


class CausalSelfAttention(nn.Module):
    def __init__(self, model_dim: int, num_heads: int):
        super().__init__()
        if model_dim % num_heads:
            raise ValueError("model_dim must be divisible by num_heads")
        self.num_heads = num_heads
        self.head_dim = model_dim // num_heads
        self.q_proj = Linear(model_dim, model_dim)
        self.k_proj = Linear(model_dim, model_dim)
        self.v_proj = Linear(model_dim, model_dim)
        self.out_proj = Linear(model_dim, model_dim)

    def forward(self, x):
        return ops.causal_self_attention(
            x, self.q_proj.weight, self.k_proj.weight, self.v_proj.weight, self.out_proj.weight, self.num_heads
        )


class MLP(nn.Module):
    def __init__(self, model_dim: int):
        super().__init__()
        self.fc1 = Linear(model_dim, MLP_RATIO * model_dim)
        self.fc2 = Linear(MLP_RATIO * model_dim, model_dim)

    def forward(self, x):
        return ops.mlp(x, self.fc1.weight, self.fc2.weight)


class TransformerBlock(nn.Module):
    """Pre-norm block: ``x + attn(norm(x))`` then ``x + mlp(norm(x))``."""

    def __init__(self, model_dim: int, num_heads: int):
        super().__init__()
        self.attn_norm = LayerNorm(model_dim)
        self.attn = CausalSelfAttention(model_dim, num_heads)
        self.mlp_norm = LayerNorm(model_dim)
        self.mlp = MLP(model_dim)

    def forward(self, x):
        a, m = self.attn, self.mlp
        return ops.transformer_block(
            x,
            self.attn_norm.weight,
            self.attn_norm.bias,
            a.q_proj.weight,
            a.k_proj.weight,
            a.v_proj.weight,
            a.out_proj.weight,
            self.mlp_norm.weight,
            self.mlp_norm.bias,
            m.fc1.weight,
            m.fc2.weight,
            a.num_heads,
            self.attn_norm.eps,
        )


class ReferenceTransformer(nn.Module):
    """Decoder-only Transformer keyed by stable global layer ids."""

    def __init__(self, config: TrainConfig, *, vocab_size: int, sequence_length: int):
        super().__init__()
        self.config = config
        self.vocab_size = vocab_size
        self.sequence_length = sequence_length
        self.token_embedding = Embedding(vocab_size, config.model_dim)
        self.position_embedding = Embedding(sequence_length, config.model_dim)
        self.layers = nn.ModuleDict(
            {str(gid): TransformerBlock(config.model_dim, config.num_heads) for gid in range(config.num_layers)}
        )
        self.final_norm = LayerNorm(config.model_dim)
        self.lm_head = Linear(config.model_dim, vocab_size)

    @property
    def layer_ids(self) -> tuple[int, ...]:
        return tuple(sorted(int(gid) for gid in self.layers))

    def forward(self, tokens):
        _, seq = tokens.shape
        if seq != self.sequence_length:
            raise ValueError("token sequence length does not match the model")
        # token lookup and the position add (model.py:128-129) in one kernel
        x = ops.embedding(tokens, self.token_embedding.weight, self.position_embedding.weight)
        for gid in self.layer_ids:
            x = self.layers[str(gid)](x)
        x = self.final_norm(x)
        return self.lm_head(x)

    def next_token_loss(self, tokens):
        """``next_token_loss(self(tokens), tokens, vocab_size)`` (resihp/reference.py:41-50) with the LM
        head fused into the loss, so the [batch, seq, vocab] logits and their gradient never exist
        (bf16 models; an fp32 model takes the unfused path).  Not in the reference: a memory-saving
        variant of its forward + loss."""
        _, seq = tokens.shape
        if seq != self.sequence_length:
            raise ValueError("token sequence length does not match the model")
        if self.lm_head.weight.dtype != torch.bfloat16:
            from .reference import next_token_loss

            return next_token_loss(self(tokens), tokens, self.vocab_size)
        x = ops.embedding(tokens, self.token_embedding.weight, self.position_embedding.weight)
        for gid in self.layer_ids:
            x = self.layers[str(gid)](x)
        x = self.final_norm(x)
        return ops.lm_head_next_token_loss(x, self.lm_head.weight, tokens)

    def logical_state_dict(self) -> dict[str, "torch.Tensor"]:
        """Parameters keyed by stable logical name (``layers.<gid>.<...>``)."""
        return {name: param for name, param in self.named_parameters()}
