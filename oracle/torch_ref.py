"""Torch-CPU restatement of the reference decoder step (oracle; test infrastructure only).

Written from the reference's math, op for op, on CPU tensors, so that torch's
own CPU kernels and autograd produce the expected values:

* ``Model``: the module tree of resihp/model.py:48-137 built in the same order
  (token embedding, position embedding, per layer [attn_norm, q, k, v, out,
  mlp_norm, fc1, fc2], final_norm, lm_head) from torch.nn primitives, so a
  seeded construction consumes the RNG exactly like the reference;
* ``block_forward`` / ``model_forward``: the functional forward over a
  name -> tensor state dict (model.py:60-97,124-133);
* ``shard_forward``: one TP rank's stage forward, resihp/parallel/tp.py:222-273,
  with the f/g collectives as identities (partial sums) and the local logits;
* ``next_token_loss``: resihp/reference.py:41-50;
* ``adamw``: torch.optim.AdamW with resihp/reference.py:20-23's constants;
* ``shard_dims`` / ``local_slice`` / ``cat``: resihp/parallel/reshard.py:41-123;
* ``pipeline_schedule``: resihp/planner/pp.py:36-60.
"""

from __future__ import annotations

import math

import torch
from torch import nn
from torch.nn import functional as F

MLP_RATIO = 4
LEARNING_RATE = 1e-3
WEIGHT_DECAY = 0.01
ADAM_BETAS = (0.9, 0.999)
ADAM_EPS = 1e-8

LAYER_NAMES = (
    "attn_norm.weight",
    "attn_norm.bias",
    "attn.q_proj.weight",
    "attn.k_proj.weight",
    "attn.v_proj.weight",
    "attn.out_proj.weight",
    "mlp_norm.weight",
    "mlp_norm.bias",
    "mlp.fc1.weight",
    "mlp.fc2.weight",
)


class _Attn(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.q_proj = nn.Linear(d, d, bias=False)
        self.k_proj = nn.Linear(d, d, bias=False)
        self.v_proj = nn.Linear(d, d, bias=False)
        self.out_proj = nn.Linear(d, d, bias=False)


class _Mlp(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.fc1 = nn.Linear(d, MLP_RATIO * d, bias=False)
        self.fc2 = nn.Linear(MLP_RATIO * d, d, bias=False)


class _Block(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.attn_norm = nn.LayerNorm(d)
        self.attn = _Attn(d)
        self.mlp_norm = nn.LayerNorm(d)
        self.mlp = _Mlp(d)


class Model(nn.Module):
    """Parameter container in the reference's construction order (model.py:103-116)."""

    def __init__(self, model_dim, num_layers, num_heads, vocab_size, sequence_length):
        super().__init__()
        if model_dim % num_heads:
            raise ValueError("model_dim must be divisible by num_heads")
        self.num_heads = num_heads
        self.token_embedding = nn.Embedding(vocab_size, model_dim)
        self.position_embedding = nn.Embedding(sequence_length, model_dim)
        self.layers = nn.ModuleDict({str(g): _Block(model_dim) for g in range(num_layers)})
        self.final_norm = nn.LayerNorm(model_dim)
        self.lm_head = nn.Linear(model_dim, vocab_size, bias=False)

    def state(self) -> dict[str, torch.Tensor]:
        return dict(self.named_parameters())


def seeded_state(model_dim, num_layers, num_heads, vocab_size, sequence_length, seed) -> dict[str, torch.Tensor]:
    """The reference's seeded init (reference.py:121-125): manual_seed, then construct."""
    torch.manual_seed(seed)
    m = Model(model_dim, num_layers, num_heads, vocab_size, sequence_length)
    return {k: v.detach().clone() for k, v in m.state().items()}


def synthetic_state(model_dim, num_layers, vocab_size, sequence_length, *, std=0.02, seed=0, dtype=torch.float32,
                    layer_ids=None, tp_size=1, tp_rank=0, first=True, last=True):
    """Weights N(0, std), LayerNorm gamma=1 / beta=0 (the synthetic init of the GPU configs).

    With ``tp_size > 1`` returns this rank's shards (q/k/v/fc1/lm_head/tok rows, out/fc2 cols)
    cut from the full synthetic matrices, exactly like shard_logical_state.
    """
    g = torch.Generator().manual_seed(seed)
    d, f = model_dim, MLP_RATIO * model_dim
    ids = list(range(num_layers)) if layer_ids is None else list(layer_ids)

    def rnd(*shape):
        return (torch.randn(*shape, generator=g) * std).to(dtype)

    full = {}
    if first:
        full["token_embedding.weight"] = rnd(vocab_size, d)
        full["position_embedding.weight"] = rnd(sequence_length, d)
    for gid in ids:
        p = f"layers.{gid}."
        full[p + "attn_norm.weight"] = torch.ones(d, dtype=dtype)
        full[p + "attn_norm.bias"] = torch.zeros(d, dtype=dtype)
        for n in ("q_proj", "k_proj", "v_proj", "out_proj"):
            full[p + f"attn.{n}.weight"] = rnd(d, d)
        full[p + "mlp_norm.weight"] = torch.ones(d, dtype=dtype)
        full[p + "mlp_norm.bias"] = torch.zeros(d, dtype=dtype)
        full[p + "mlp.fc1.weight"] = rnd(f, d)
        full[p + "mlp.fc2.weight"] = rnd(d, f)
    if last:
        full["final_norm.weight"] = torch.ones(d, dtype=dtype)
        full["final_norm.bias"] = torch.zeros(d, dtype=dtype)
        full["lm_head.weight"] = rnd(vocab_size, d)
    if tp_size == 1:
        return full
    layout = shard_dims(ids)
    return {k: local_slice(v, layout[k], tp_rank, tp_size) for k, v in full.items()}


# ---------------------------------------------------------------------------
# forward
# ---------------------------------------------------------------------------
def attention(x, wq, wk, wv, wo, num_heads):
    """CausalSelfAttention.forward (model.py:60-71) with explicit weights; num_heads = local heads."""
    batch, seq, _ = x.shape
    width = wq.shape[0]
    head_dim = width // num_heads
    shape = (batch, seq, num_heads, head_dim)
    q = F.linear(x, wq).view(shape).transpose(1, 2)
    k = F.linear(x, wk).view(shape).transpose(1, 2)
    v = F.linear(x, wv).view(shape).transpose(1, 2)
    scores = (q @ k.transpose(-2, -1)) / math.sqrt(head_dim)
    future = torch.triu(torch.ones(seq, seq, dtype=torch.bool, device=x.device), diagonal=1)
    scores = scores.masked_fill(future, float("-inf"))
    weights = F.softmax(scores, dim=-1)
    context = (weights @ v).transpose(1, 2).reshape(batch, seq, width)
    return F.linear(context, wo)


def mlp(x, w1, w2):
    return F.linear(F.gelu(F.linear(x, w1)), w2)


def block_forward(x, p: dict, prefix: str, num_heads: int, eps: float = 1e-5):
    """TransformerBlock.forward (model.py:94-97) / one shard block (tp.py:260-265)."""
    d = x.shape[-1]
    n = F.layer_norm(x, (d,), p[prefix + "attn_norm.weight"], p[prefix + "attn_norm.bias"], eps)
    x = x + attention(n, p[prefix + "attn.q_proj.weight"], p[prefix + "attn.k_proj.weight"],
                      p[prefix + "attn.v_proj.weight"], p[prefix + "attn.out_proj.weight"], num_heads)
    n = F.layer_norm(x, (d,), p[prefix + "mlp_norm.weight"], p[prefix + "mlp_norm.bias"], eps)
    return x + mlp(n, p[prefix + "mlp.fc1.weight"], p[prefix + "mlp.fc2.weight"])


def model_forward(p: dict, tokens, num_heads: int, layer_ids):
    """ReferenceTransformer.forward (model.py:124-133)."""
    seq = tokens.shape[1]
    positions = torch.arange(seq, device=tokens.device)
    x = F.embedding(tokens, p["token_embedding.weight"]) + F.embedding(positions, p["position_embedding.weight"])
    for gid in sorted(layer_ids):
        x = block_forward(x, p, f"layers.{gid}.", num_heads)
    d = x.shape[-1]
    x = F.layer_norm(x, (d,), p["final_norm.weight"], p["final_norm.bias"])
    return F.linear(x, p["lm_head.weight"])


def shard_forward(p: dict, *, num_heads, tp_rank, tp_size, vocab_size, layer_ids, is_first, is_last,
                  tokens=None, hidden=None):
    """TensorParallelStage.forward (tp.py:222-273) for one rank, collectives as identities."""
    local_heads = num_heads // tp_size
    if is_first:
        per = vocab_size // tp_size
        start = tp_rank * per
        outside = (tokens < start) | (tokens >= start + per)
        local_ids = (tokens - start).clamp(0, per - 1)
        x = F.embedding(local_ids, p["token_embedding.weight"]).masked_fill(outside.unsqueeze(-1), 0.0)
        x = x + F.embedding(torch.arange(tokens.shape[1], device=tokens.device), p["position_embedding.weight"])
    else:
        x = hidden
    for gid in sorted(layer_ids):
        x = block_forward(x, p, f"layers.{gid}.", local_heads)
    if not is_last:
        return x
    d = x.shape[-1]
    x = F.layer_norm(x, (d,), p["final_norm.weight"], p["final_norm.bias"])
    return F.linear(x, p["lm_head.weight"])


def next_token_loss(logits, tokens, vocab_size):
    """reference.py:41-50."""
    return F.cross_entropy(logits[:, :-1].reshape(-1, vocab_size), tokens[:, 1:].reshape(-1))


def adamw(params):
    return torch.optim.AdamW(params, lr=LEARNING_RATE, betas=ADAM_BETAS, eps=ADAM_EPS, weight_decay=WEIGHT_DECAY)


def loss_and_grads(p: dict, tokens, num_heads, layer_ids, vocab_size, dtype=torch.float32):
    """Forward + next-token loss + backward on CPU; returns (logits, loss, {name: grad})."""
    leaves = {k: v.detach().to(dtype).clone().requires_grad_(True) for k, v in p.items()}
    logits = model_forward(leaves, tokens, num_heads, layer_ids)
    loss = next_token_loss(logits, tokens, vocab_size)
    loss.backward()
    return logits.detach(), loss.detach(), {k: v.grad for k, v in leaves.items()}


# ---------------------------------------------------------------------------
# reshard and schedule
# ---------------------------------------------------------------------------
_GLOBAL = {"token_embedding.weight": 0, "position_embedding.weight": None, "final_norm.weight": None,
           "final_norm.bias": None, "lm_head.weight": 0}
_LAYER = {"attn_norm.weight": None, "attn_norm.bias": None, "attn.q_proj.weight": 0, "attn.k_proj.weight": 0,
          "attn.v_proj.weight": 0, "attn.out_proj.weight": 1, "mlp_norm.weight": None, "mlp_norm.bias": None,
          "mlp.fc1.weight": 0, "mlp.fc2.weight": 1}


def shard_dims(layer_ids):
    """reshard.py:70-81."""
    dims = dict(_GLOBAL)
    for gid in layer_ids:
        for suffix, dim in _LAYER.items():
            dims[f"layers.{gid}.{suffix}"] = dim
    return dims


def local_slice(full, dim, rank, size):
    """reshard.py:107-111."""
    if dim is None:
        return full.detach().clone()
    return torch.chunk(full, size, dim=dim)[rank].contiguous().clone()


def cat(parts, dim):
    """reshard.py:101."""
    return torch.cat(parts, dim=dim)


def pipeline_schedule(num_micro, stage_index, num_stages):
    """planner/pp.py:36-60."""
    warmup = min(num_stages - 1 - stage_index, num_micro)
    steady = num_micro - warmup
    return ("F",) * warmup + ("F", "B") * steady + ("B",) * warmup


def issue_order(num_micro, stage_index, num_stages):
    """The F<i>/B<i> labels parallel/pp.py:365-422 appends (oldest in-flight retires first)."""
    out, nf, held = [], 0, []
    for op in pipeline_schedule(num_micro, stage_index, num_stages):
        if op == "F":
            out.append(f"F{nf}")
            held.append(nf)
            nf += 1
        else:
            out.append(f"B{held.pop(0)}")
    return out


def scatter_routing(up, down):
    """parallel/pp.py:57-80: chunk k of N = max(U, D) travels up[k*U//N] -> down[k*D//N]."""
    n = max(len(up), len(down))
    return [(up[k * len(up) // n], down[k * len(down) // n]) for k in range(n)]


def boundary_slab(tensor, up, down, rank, backward=False):
    """The slab one rank of a pipeline hop collects (parallel/pp.py:262-281): the chunks of the
    flattened boundary tensor routed to it, in chunk order (forward: downstream receivers;
    backward: the same pairs reversed, upstream receivers)."""
    flat = tensor.reshape(-1)
    routing = scatter_routing(up, down)
    width = flat.numel() // len(routing)
    end = 0 if backward else 1
    return torch.cat([flat[k * width:(k + 1) * width] for k, pair in enumerate(routing) if pair[end] == rank])


def boundary_reconstruct(slabs, shape):
    """parallel/pp.py:283-295: the stage's slabs in TP-rank order, concatenated."""
    return torch.cat(list(slabs)).view(shape)
