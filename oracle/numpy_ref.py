"""Independent fp64 numpy restatement of the decoder step with a hand-derived backward.

Oracle / test infrastructure only.  Same math as resihp/model.py:60-133 and
resihp/reference.py:41-50, written without autograd so that it can pin the
torch restatement (oracle.torch_ref) and be pinned itself by central finite
differences.  Every array is float64; the forward caches what the backward
needs.

Derivatives used (per row, d = width):
  LayerNorm   x^ = (x - mu) * r,  y = x^ g + b
              dx = r * (dy g - mean(dy g) - x^ mean(dy g x^))
  GELU        gelu(u) = u Phi(u),  gelu'(u) = Phi(u) + u phi(u)
  attention   P = softmax(q k^T / sqrt(Dh) + mask),  o = P v
              dv = P^T do,  dP = do v^T,  dS = P (dP - rowsum(dP P))
              dq = dS k / sqrt(Dh),  dk = dS^T q / sqrt(Dh)
  CE          loss = mean(lse(x) - x_t),  dx = (softmax(x) - onehot(t)) / N
"""

from __future__ import annotations

import math

import numpy as np
from scipy.special import erf

SQRT1_2 = 1.0 / math.sqrt(2.0)
INV_SQRT_2PI = 1.0 / math.sqrt(2.0 * math.pi)


def gelu(u):
    return 0.5 * u * (1.0 + erf(u * SQRT1_2))


def gelu_grad(u):
    return 0.5 * (1.0 + erf(u * SQRT1_2)) + u * np.exp(-0.5 * u * u) * INV_SQRT_2PI


def ln_fwd(x, g, b, eps=1e-5):
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    r = 1.0 / np.sqrt(var + eps)
    xh = (x - mu) * r
    return xh * g + b, (xh, r)


def ln_bwd(dy, cache, g):
    xh, r = cache
    gy = dy * g
    dx = r * (gy - gy.mean(-1, keepdims=True) - xh * (gy * xh).mean(-1, keepdims=True))
    axes = tuple(range(dy.ndim - 1))
    return dx, (dy * xh).sum(axes), dy.sum(axes)


def attn_fwd(q, k, v, causal=True):
    """q, k, v [B, H, S, Dh] -> o, P."""
    dh = q.shape[-1]
    s = q @ np.swapaxes(k, -1, -2) / math.sqrt(dh)
    if causal:
        S = q.shape[-2]
        s = np.where(np.triu(np.ones((S, S), dtype=bool), 1), -np.inf, s)
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    return p @ v, p


def attn_bwd(do, q, k, v, p):
    dh = q.shape[-1]
    dv = np.swapaxes(p, -1, -2) @ do
    dp = do @ np.swapaxes(v, -1, -2)
    ds = p * (dp - (dp * p).sum(-1, keepdims=True))
    dq = ds @ k / math.sqrt(dh)
    dk = np.swapaxes(ds, -1, -2) @ q / math.sqrt(dh)
    return dq, dk, dv


def _split(x, heads):
    B, S, W = x.shape
    return x.reshape(B, S, heads, W // heads).transpose(0, 2, 1, 3)


def _merge(x):
    B, H, S, D = x.shape
    return x.transpose(0, 2, 1, 3).reshape(B, S, H * D)


def block_fwd(x, p, pre, heads):
    c = {}
    n1, c["ln1"] = ln_fwd(x, p[pre + "attn_norm.weight"], p[pre + "attn_norm.bias"])
    c["n1"] = n1
    q = _split(n1 @ p[pre + "attn.q_proj.weight"].T, heads)
    k = _split(n1 @ p[pre + "attn.k_proj.weight"].T, heads)
    v = _split(n1 @ p[pre + "attn.v_proj.weight"].T, heads)
    o, P = attn_fwd(q, k, v)
    c.update(q=q, k=k, v=v, P=P, ctx=_merge(o))
    x1 = x + c["ctx"] @ p[pre + "attn.out_proj.weight"].T
    n2, c["ln2"] = ln_fwd(x1, p[pre + "mlp_norm.weight"], p[pre + "mlp_norm.bias"])
    c["n2"] = n2
    u = n2 @ p[pre + "mlp.fc1.weight"].T
    h = gelu(u)
    c.update(u=u, h=h)
    return x1 + h @ p[pre + "mlp.fc2.weight"].T, c


def _acc(grads, name, g):
    grads[name] = grads.get(name, 0.0) + g


def block_bwd(dy, c, p, pre, heads, grads):
    def wgrad(dout, inp):
        return dout.reshape(-1, dout.shape[-1]).T @ inp.reshape(-1, inp.shape[-1])

    _acc(grads, pre + "mlp.fc2.weight", wgrad(dy, c["h"]))
    dh = dy @ p[pre + "mlp.fc2.weight"]
    du = dh * gelu_grad(c["u"])
    _acc(grads, pre + "mlp.fc1.weight", wgrad(du, c["n2"]))
    dn2 = du @ p[pre + "mlp.fc1.weight"]
    dx1, dg, db = ln_bwd(dn2, c["ln2"], p[pre + "mlp_norm.weight"])
    _acc(grads, pre + "mlp_norm.weight", dg)
    _acc(grads, pre + "mlp_norm.bias", db)
    dx1 = dx1 + dy
    _acc(grads, pre + "attn.out_proj.weight", wgrad(dx1, c["ctx"]))
    dctx = dx1 @ p[pre + "attn.out_proj.weight"]
    dq, dk, dv = attn_bwd(_split(dctx, heads), c["q"], c["k"], c["v"], c["P"])
    dq, dk, dv = _merge(dq), _merge(dk), _merge(dv)
    _acc(grads, pre + "attn.q_proj.weight", wgrad(dq, c["n1"]))
    _acc(grads, pre + "attn.k_proj.weight", wgrad(dk, c["n1"]))
    _acc(grads, pre + "attn.v_proj.weight", wgrad(dv, c["n1"]))
    dn1 = dq @ p[pre + "attn.q_proj.weight"] + dk @ p[pre + "attn.k_proj.weight"] + dv @ p[pre + "attn.v_proj.weight"]
    dx, dg, db = ln_bwd(dn1, c["ln1"], p[pre + "attn_norm.weight"])
    _acc(grads, pre + "attn_norm.weight", dg)
    _acc(grads, pre + "attn_norm.bias", db)
    return dx + dx1


def xent(logits, tokens):
    """Mean next-token CE over logits[:, :-1] vs tokens[:, 1:] and its gradient (zero last position)."""
    x = logits[:, :-1]
    t = tokens[:, 1:]
    m = x.max(-1, keepdims=True)
    lse = m[..., 0] + np.log(np.exp(x - m).sum(-1))
    picked = np.take_along_axis(x, t[..., None], -1)[..., 0]
    n = t.size
    loss = (lse - picked).mean()
    d = np.exp(x - lse[..., None])
    np.put_along_axis(d, t[..., None], np.take_along_axis(d, t[..., None], -1) - 1.0, -1)
    dl = np.zeros_like(logits)
    dl[:, :-1] = d / n
    return loss, dl


def model_loss_and_grads(p: dict, tokens: np.ndarray, heads: int, layer_ids):
    """Full-model loss and every parameter gradient (fp64)."""
    p = {k: np.asarray(v, dtype=np.float64) for k, v in p.items()}
    B, S = tokens.shape
    x = p["token_embedding.weight"][tokens] + p["position_embedding.weight"][np.arange(S)][None]
    caches = []
    for gid in sorted(layer_ids):
        x, c = block_fwd(x, p, f"layers.{gid}.", heads)
        caches.append((gid, c))
    xf, lnf = ln_fwd(x, p["final_norm.weight"], p["final_norm.bias"])
    logits = xf @ p["lm_head.weight"].T
    loss, dl = xent(logits, tokens)
    grads: dict = {}
    grads["lm_head.weight"] = dl.reshape(-1, dl.shape[-1]).T @ xf.reshape(-1, xf.shape[-1])
    dxf = dl @ p["lm_head.weight"]
    dx, dg, db = ln_bwd(dxf, lnf, p["final_norm.weight"])
    grads["final_norm.weight"], grads["final_norm.bias"] = dg, db
    for gid, c in reversed(caches):
        dx = block_bwd(dx, c, p, f"layers.{gid}.", heads, grads)
    dtok = np.zeros_like(p["token_embedding.weight"])
    np.add.at(dtok, tokens.reshape(-1), dx.reshape(-1, dx.shape[-1]))
    grads["token_embedding.weight"] = dtok
    dpos = np.zeros_like(p["position_embedding.weight"])
    dpos[:S] = dx.sum(0)
    grads["position_embedding.weight"] = dpos
    return logits, loss, grads


def model_loss(p: dict, tokens: np.ndarray, heads: int, layer_ids) -> float:
    return float(model_loss_and_grads(p, tokens, heads, layer_ids)[1])
