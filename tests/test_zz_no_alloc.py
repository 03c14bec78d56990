"""rh_attn_bwd_noalloc (the backward with its scratch in a static device array) against
rh_attn_bwd (the same kernels with a caller-provided workspace), through the C ABI: bit-identical
gradients on two calls in a row, the second with a smaller input; sizes beyond the static array
are refused."""

import ctypes
import math

import pytest
import torch

from resihp import _hip as H
from resihp import ops

pytestmark = pytest.mark.gpu


def _case(batch, seq, heads, head_dim, seed):
    g = torch.Generator().manual_seed(seed)
    W = heads * head_dim
    qkv = torch.randn(batch * seq, 3 * W, generator=g).to("cuda", torch.bfloat16)
    dout = torch.randn(batch * seq, W, generator=g).to("cuda", torch.bfloat16)
    ctx, lse, ctx_lo = ops.attn_fwd(qkv, batch, seq, heads, head_dim)
    return qkv, dout, ctx, lse, ctx_lo


def _bwd(entry, qkv, dout, ctx, lse, ctx_lo, batch, seq, heads, head_dim):
    W = heads * head_dim
    es = qkv.element_size()
    dqkv = torch.full((batch * seq, 3 * W), float("nan"), dtype=qkv.dtype, device=qkv.device)
    base, dbase = qkv.data_ptr(), dqkv.data_ptr()
    args = [H.RH_DTYPE_BF16, batch, seq, heads, head_dim, base, base + W * es, base + 2 * W * es, 3 * W,
            ctx.data_ptr(), ctx_lo.data_ptr(), W, dout.data_ptr(), W, lse.data_ptr(), dbase, dbase + W * es,
            dbase + 2 * W * es, 3 * W, 1.0 / math.sqrt(head_dim), 1]
    if entry == "rh_attn_bwd":
        nbytes = H.query("rh_attn_bwd_workspace_bytes", batch, seq, heads)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=qkv.device)
        H.call("rh_attn_bwd", *args, ws.data_ptr(), nbytes, torch.cuda.current_stream().cuda_stream)
    else:
        H.call("rh_attn_bwd_noalloc", *args, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return dqkv


def test_noalloc_attention_backward_matches_workspace_entry(cuda):
    for batch, seq, heads, head_dim, seed in ((4, 2048, 4, 128, 1), (2, 1024, 3, 64, 2)):  # second call smaller
        case = _case(batch, seq, heads, head_dim, seed)
        want = _bwd("rh_attn_bwd", *case, batch, seq, heads, head_dim)
        got = _bwd("rh_attn_bwd_noalloc", *case, batch, seq, heads, head_dim)
        assert not torch.isnan(got).any()
        assert torch.equal(got, want), (batch, seq, heads, head_dim)


def test_noalloc_attention_backward_rejects_sizes_beyond_its_scratch(cuda):
    rows = 2097152 + 1  # RH_ATTN_NOALLOC_MAX_ROWS + 1 query rows: refused before any launch
    with pytest.raises(ValueError, match="static scratch"):
        H.call("rh_attn_bwd_noalloc", H.RH_DTYPE_BF16, 1, rows, 1, 128, 16, 16, 16, 384, 16, 16, 128, 16, 128, 16,
               16, 16, 16, 384, 0.088, 1, None)
