"""Autograd operators that run the decoder step on the HIP kernels.

Each operator restates one reference computation (cited per function) as an
``torch.autograd.Function`` whose forward and backward call the C ABI through
:mod:`resihp._hip`.  PyTorch supplies device memory, the current stream and the
autograd graph; every FLOP runs in the library.

Parameter gradients are written straight into ``param.grad`` by the kernels
(``beta = 1`` accumulation in the GEMM epilogue, ``accumulate`` in the
LayerNorm / embedding column sums) instead of being returned to autograd, so
repeated backward passes accumulate exactly like the reference's
``loss.backward()`` over micro-batches (resihp/parallel/pp.py:355,393-404)
without an extra read-modify-write pass per parameter.  The backward of a
Function therefore returns ``None`` for its parameters.
"""

from __future__ import annotations

import ctypes
import math
import os

import torch

from . import _hip as H
from . import profiling

LN_EPS = 1e-5  # nn.LayerNorm / F.layer_norm default, resihp/model.py:89,91,115


# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------
def _same_dtype(*tensors: torch.Tensor) -> int:
    code = None
    for t in tensors:
        if t is None:
            continue
        c = H.dtype_code(t)
        if code is None:
            code = c
        elif c != code:
            raise TypeError("resihp kernels need every operand in one dtype (float32 or bfloat16)")
    return code


def _rows(M: int, N: int, like: torch.Tensor) -> torch.Tensor:
    """[M, N] output whose row stride is a multiple of 8 elements (16-byte rows)."""
    ld = (N + 7) // 8 * 8
    buf = torch.empty((M, ld), dtype=like.dtype, device=like.device)
    return buf if ld == N else buf[:, :N]


def _ld(t: torch.Tensor) -> int:
    if t.dim() != 2 or t.stride(1) != 1:
        raise ValueError("expected a row-major 2-D view")
    return t.stride(0)


def _as_rows(x: torch.Tensor) -> torch.Tensor:
    """Flatten leading dims to a row-major [rows, last] view (copy only if needed)."""
    x2 = x.reshape(-1, x.shape[-1])
    if x2.stride(-1) != 1 or (x2.shape[0] > 1 and x2.stride(0) < x2.shape[1]):
        x2 = x2.contiguous()
    return x2


def _grad_target(p: torch.Tensor) -> tuple[torch.Tensor, bool]:
    """Where a kernel should put p's gradient: (buffer, accumulate)."""
    g = p.grad
    if g is not None and g.is_contiguous() and g.dtype == p.dtype and g.device == p.device:
        return g, True
    buf = torch.empty_like(p, memory_format=torch.contiguous_format)
    if g is None:
        p.grad = buf
        return buf, False
    return buf, False  # unusual layout: caller adds it in


def _finish_grad(p: torch.Tensor, buf: torch.Tensor) -> None:
    if p.grad is not buf:
        p.grad.add_(buf)


def _wants(p: torch.Tensor | None) -> bool:
    return p is not None and p.requires_grad


# ---------------------------------------------------------------------------
# GEMM
# ---------------------------------------------------------------------------
def gemm(layout: int, M: int, N: int, K: int, A: torch.Tensor, lda: int, B: list, ldb: int, D: list, ldd: int, *,
         alpha: float = 1.0, beta: float = 0.0, C: torch.Tensor | None = None, ldc: int = 0,
         epilogue: int = H.RH_EPI_NONE, aux: torch.Tensor | None = None, aux_out: torch.Tensor | None = None,
         ldaux: int = 0, b_seg_rows: int = 0, d_seg_rows: int = 0) -> None:
    """One rh_gemm call (see include/resihp_hip.h for the layouts)."""
    dev = H.require_gpu(A, *B, *D, C, aux, aux_out)
    desc = _gemm_desc(layout, M, N, K, A, lda, B, ldb, D, ldd, alpha=alpha, beta=beta, C=C, ldc=ldc,
                      epilogue=epilogue, aux=aux, aux_out=aux_out, ldaux=ldaux, b_seg_rows=b_seg_rows,
                      d_seg_rows=d_seg_rows)
    nbytes = H.query("rh_gemm_workspace_bytes", ctypes.byref(desc))
    ws = H.workspace(nbytes, dev)
    if profiling.active():
        # main kernel and split-K reduce timed apart (the reduce is a bandwidth kernel)
        name = ctypes.create_string_buffer(128)
        H.call("rh_gemm_kernel_name", ctypes.byref(desc), name, 128)
        with profiling.launch(name.value.decode(), 2.0 * M * N * K):
            H.call("rh_gemm_stage", ctypes.byref(desc), H.ptr(ws), nbytes, H.RH_GEMM_STAGE_MAIN, H.stream_of(A))
        if nbytes:
            # fp32 partials read once; D written, C / aux read or written once (2-byte bf16 storage)
            es = A.element_size()
            io = 1 + (beta != 0.0) + (epilogue != H.RH_EPI_NONE)
            with profiling.launch("gemm_splitk_reduce", 0.0, nbytes + io * M * N * es):
                H.call("rh_gemm_stage", ctypes.byref(desc), H.ptr(ws), nbytes, H.RH_GEMM_STAGE_REDUCE,
                       H.stream_of(A))
        return
    H.call("rh_gemm", ctypes.byref(desc), H.ptr(ws), nbytes, H.stream_of(A))


def _gemm_desc(layout, M, N, K, A, lda, B, ldb, D, ldd, *, alpha=1.0, beta=0.0, C=None, ldc=0,
               epilogue=H.RH_EPI_NONE, aux=None, aux_out=None, ldaux=0, b_seg_rows=0, d_seg_rows=0):
    desc = H.rh_gemm_desc()
    desc.dtype = _same_dtype(A, *B, *D, C, aux, aux_out)
    desc.layout = layout
    desc.epilogue = epilogue
    desc.b_nseg = len(B)
    desc.d_nseg = len(D)
    desc.M, desc.N, desc.K = M, N, K
    desc.A = A.data_ptr()
    desc.lda = lda
    for i, b in enumerate(B):
        desc.B[i] = b.data_ptr()
    desc.ldb = ldb
    desc.b_seg_rows = b_seg_rows
    desc.alpha = alpha
    desc.beta = beta
    desc.C = None if C is None else C.data_ptr()
    desc.ldc = ldc
    for i, d in enumerate(D):
        desc.D[i] = d.data_ptr()
    desc.ldd = ldd
    desc.d_seg_rows = d_seg_rows
    desc.aux = None if aux is None else aux.data_ptr()
    desc.aux_out = None if aux_out is None else aux_out.data_ptr()
    desc.ldaux = ldaux
    return desc


def linear_fwd(x2: torch.Tensor, ws: list, *, residual: torch.Tensor | None = None,
               gelu_pre: torch.Tensor | None = None, gelu_deriv: torch.Tensor | None = None) -> torch.Tensor:
    """y = x . W^T for W = cat(ws, 0) (+ residual).  GELU epilogue when ``gelu_pre`` (receives the
    pre-activation) or ``gelu_deriv`` (receives gelu'(pre-activation), for the backward) is given."""
    M, K = x2.shape
    seg = ws[0].shape[0]
    N = seg * len(ws)
    for w in ws:
        if w.shape != (seg, K) or not w.is_contiguous():
            raise ValueError(f"weight of shape {tuple(w.shape)} does not match input width {K}")
    y = _rows(M, N, x2)
    aux_out = gelu_pre if gelu_pre is not None else gelu_deriv
    epi = H.RH_EPI_GELU if gelu_pre is not None else (H.RH_EPI_GELU_DERIV if gelu_deriv is not None else H.RH_EPI_NONE)
    gemm(H.RH_GEMM_NT, M, N, K, x2, _ld(x2), ws, K, [y], _ld(y),
         beta=0.0 if residual is None else 1.0, C=residual, ldc=0 if residual is None else _ld(residual),
         epilogue=epi, aux_out=aux_out, ldaux=0 if aux_out is None else _ld(aux_out),
         b_seg_rows=seg if len(ws) > 1 else 0)
    return y


def linear_dgrad(dy2: torch.Tensor, ws: list, *, gelu_pre: torch.Tensor | None = None,
                 gelu_deriv: torch.Tensor | None = None) -> torch.Tensor:
    """dx = dy . W for W = cat(ws, 0); times gelu'(gelu_pre), or times the stored derivative
    ``gelu_deriv``, when given."""
    M, N_out = dy2.shape
    seg = ws[0].shape[0]
    K_in = ws[0].shape[1]
    dx = _rows(M, K_in, dy2)
    aux = gelu_pre if gelu_pre is not None else gelu_deriv
    epi = H.RH_EPI_GELU_GRAD if gelu_pre is not None else (H.RH_EPI_MUL_AUX if gelu_deriv is not None else H.RH_EPI_NONE)
    gemm(H.RH_GEMM_NN, M, K_in, N_out, dy2, _ld(dy2), ws, K_in, [dx], _ld(dx),
         epilogue=epi, aux=aux, ldaux=0 if aux is None else _ld(aux), b_seg_rows=seg if len(ws) > 1 else 0)
    return dx


def _wgrad_setup(dy2: torch.Tensor, x2: torch.Tensor, params: list, allow_pad: bool = True):
    """The TN GEMM of param.grad (+)= dy^T . x (dy's columns split over ``params``, rows of W):
    (desc, finish) with ``finish()`` folding any side buffer into .grad, or None when no
    parameter wants a gradient."""
    want = [_wants(p) for p in params]
    if not any(want):
        return None
    M_rows, N_out = dy2.shape
    K_in = x2.shape[1]
    seg = params[0].shape[0]
    targets, accs = [], []
    for p, w in zip(params, want):
        # a frozen segment still needs somewhere to land in the one fused GEMM
        buf, acc = _grad_target(p) if w else (torch.empty_like(p, memory_format=torch.contiguous_format), False)
        targets.append(buf)
        accs.append(acc)
    if len(set(accs)) > 1:  # some grads exist, some not: start the new ones from zero
        for i, acc in enumerate(accs):
            if not acc:
                targets[i].zero_()
        accs = [True] * len(accs)
    M_gemm, d_seg = N_out, (seg if len(params) > 1 else 0)
    pad_rows = -N_out % 8
    if (allow_pad and len(params) == 1 and pad_rows and dy2.dtype == torch.bfloat16
            and _ld(dy2) >= N_out + pad_rows
            and dy2.storage_offset() + (M_rows - 1) * _ld(dy2) + N_out + pad_rows
            <= dy2.untyped_storage().nbytes() // dy2.element_size()):
        # A ragged output count (the LM head's vocabulary, 50257) keeps the m-contiguous dy off the
        # direct-to-LDS kernel.  dy's rows are padded in memory (the logits layout) and the padding
        # lies inside its allocation, so the GEMM runs over the rounded count; the extra output rows
        # land in a scratch segment and are dropped.
        M_gemm, d_seg = N_out + pad_rows, N_out
        targets = targets + [torch.empty(pad_rows, K_in, dtype=targets[0].dtype, device=targets[0].device)]
    desc = _gemm_desc(H.RH_GEMM_TN, M_gemm, K_in, M_rows, dy2, _ld(dy2), [x2], _ld(x2), targets, K_in,
                      beta=1.0 if accs[0] else 0.0, d_seg_rows=d_seg)

    def finish():
        for p, buf, w in zip(params, targets, want):
            if w:
                _finish_grad(p, buf)

    return desc, finish, (dy2, x2, targets)


def linear_wgrad(dy2: torch.Tensor, x2: torch.Tensor, params: list) -> None:
    """param.grad (+)= dy^T . x, with dy's columns split over ``params`` (rows of W)."""
    setup = _wgrad_setup(dy2, x2, params)
    if setup is None:
        return
    desc, finish, keep = setup
    d = desc
    targets = keep[2]
    gemm(H.RH_GEMM_TN, d.M, d.N, d.K, dy2, d.lda, [x2], d.ldb, targets, d.ldd, beta=d.beta,
         d_seg_rows=d.d_seg_rows)
    finish()


def linear_wgrad_group(items: list) -> None:
    """Several weight gradients -- [(dy2, x2, params)], at most 4 -- as ONE grouped GEMM launch
    (rh_gemm_grouped): the wgrads of a decoder block share the token count as K and together fill
    the chip, so none of them needs a split-K pass of its own."""
    setups = [s for s in (_wgrad_setup(dy2, x2, ps, allow_pad=False) for dy2, x2, ps in items) if s is not None]
    if not setups:
        return
    all_descs = [s[0] for s in setups]
    n = len(all_descs)
    descs = (H.rh_gemm_desc * n)(*all_descs)
    dev = setups[0][2][0].device
    nbytes = H.query("rh_gemm_grouped_workspace_bytes", descs, n)
    ws = H.workspace(nbytes, dev)
    stream = H.stream_of(setups[0][2][0])
    if profiling.active():
        splits = ctypes.c_int(0)
        H.call("rh_gemm_grouped_plan", descs, n, ctypes.byref(splits))
        name = ctypes.create_string_buffer(128)
        H.call("rh_gemm_grouped_kernel_name", descs, n, name, 128)
        flops = sum(2.0 * d.M * d.N * d.K for d in all_descs)
        label = (name.value.decode() + (" + split-K reduce" if splits.value > 1 else "")) if splits.value \
            else "gemm (group as single calls)"
        with profiling.launch(label, flops):
            H.call("rh_gemm_grouped", descs, n, H.ptr(ws), nbytes, stream)
    else:
        H.call("rh_gemm_grouped", descs, n, H.ptr(ws), nbytes, stream)
    for s in setups:
        s[1]()


# ---------------------------------------------------------------------------
# LayerNorm
# ---------------------------------------------------------------------------
def ln_fwd(x2: torch.Tensor, w: torch.Tensor, b: torch.Tensor, eps: float):
    rows, dim = x2.shape
    x2 = x2.contiguous()
    y = torch.empty_like(x2)
    mean = torch.empty(rows, dtype=torch.float32, device=x2.device)
    rstd = torch.empty(rows, dtype=torch.float32, device=x2.device)
    H.require_gpu(x2, w, b)
    es = x2.element_size()
    with profiling.launch("ln_fwd", 0.0, 2 * rows * dim * es + 8 * rows + 2 * dim * es):
        H.call("rh_layernorm_fwd", _same_dtype(x2, w, b), rows, dim, x2.data_ptr(), w.data_ptr(), b.data_ptr(),
               float(eps), y.data_ptr(), mean.data_ptr(), rstd.data_ptr(), H.stream_of(x2))
    return y, mean, rstd


def ln_bwd(dy2: torch.Tensor, x2: torch.Tensor, mean: torch.Tensor, rstd: torch.Tensor, w: torch.Tensor,
           b: torch.Tensor, dres: torch.Tensor | None) -> torch.Tensor:
    rows, dim = x2.shape
    dy2 = dy2.contiguous()
    x2 = x2.contiguous()
    if dres is not None:
        dres = dres.contiguous()
    dev = H.require_gpu(dy2, x2, w)
    dx = torch.empty_like(x2)
    gw_t = _grad_target(w) if _wants(w) else None
    gb_t = _grad_target(b) if _wants(b) else None
    present = [t for t in (gw_t, gb_t) if t is not None]
    acc = bool(present) and all(t[1] for t in present)
    if present and not acc and any(t[1] for t in present):
        # one gradient exists, the other is fresh: start the fresh one at zero, accumulate both
        for t in present:
            if not t[1]:
                t[0].zero_()
        acc = True
    gw = gw_t[0] if gw_t else None
    gb = gb_t[0] if gb_t else None
    nbytes = H.query("rh_layernorm_bwd_workspace_bytes", rows, dim)
    ws = H.workspace(nbytes, dev)
    # dy, x, (dres) read and dx written once; mean/rstd read; dgamma/dbeta written (and read when accumulating)
    es = x2.element_size()
    moved = (3 + (dres is not None)) * rows * dim * es + 8 * rows + len(present) * dim * es * (2 if acc else 1)
    with profiling.launch("ln_bwd (+ column sums)", 0.0, moved):
        H.call("rh_layernorm_bwd", _same_dtype(dy2, x2, w, dres), rows, dim, dy2.data_ptr(), x2.data_ptr(),
               mean.data_ptr(), rstd.data_ptr(), w.data_ptr(), H.ptr(dres), dx.data_ptr(), H.ptr(gw), H.ptr(gb),
               1 if acc else 0, H.ptr(ws), nbytes, H.stream_of(x2))
    if gw is not None:
        _finish_grad(w, gw)
    if gb is not None:
        _finish_grad(b, gb)
    return dx


# ---------------------------------------------------------------------------
# attention core
# ---------------------------------------------------------------------------
def attn_fwd(qkv: torch.Tensor, batch: int, seq: int, heads: int, head_dim: int):
    """qkv [T, 3*d_l] (q | k | v) -> context [T, d_l], lse [batch, heads, seq] and, for bf16, the
    context's rounding residual [T, d_l] (context - bf16(context)), which the backward needs to form
    delta = do . o from the unrounded output (None for fp32)."""
    dl = heads * head_dim
    T = qkv.shape[0]
    ctx = torch.empty((T, dl), dtype=qkv.dtype, device=qkv.device)
    ctx_lo = torch.empty((T, dl), dtype=qkv.dtype, device=qkv.device) if qkv.dtype == torch.bfloat16 else None
    lse = torch.empty((batch, heads, seq), dtype=torch.float32, device=qkv.device)
    es = qkv.element_size()
    base = qkv.data_ptr()
    with profiling.launch(f"attn_fwd_mfma<{head_dim}>", attn_flops(batch, seq, heads, head_dim)):
        H.call("rh_attn_fwd", H.dtype_code(qkv), batch, seq, heads, head_dim, base, base + dl * es,
               base + 2 * dl * es, _ld(qkv), ctx.data_ptr(), H.ptr(ctx_lo), dl, lse.data_ptr(),
               1.0 / math.sqrt(head_dim), 1, H.stream_of(qkv))
    return ctx, lse, ctx_lo


def attn_flops(batch: int, seq: int, heads: int, head_dim: int) -> float:
    """Causal attention forward: QK^T and PV over the lower triangle, diagonal included."""
    return 4.0 * batch * heads * head_dim * seq * (seq + 1) / 2


def attn_bwd(dctx: torch.Tensor, qkv: torch.Tensor, ctx: torch.Tensor, lse: torch.Tensor, batch: int, seq: int,
             heads: int, head_dim: int, ctx_lo: torch.Tensor | None = None) -> torch.Tensor:
    dl = heads * head_dim
    T = qkv.shape[0]
    dctx = dctx.contiguous()
    dqkv = torch.empty((T, 3 * dl), dtype=qkv.dtype, device=qkv.device)
    es = qkv.element_size()
    base, dbase = qkv.data_ptr(), dqkv.data_ptr()
    nbytes = H.query("rh_attn_bwd_workspace_bytes", batch, seq, heads)
    ws = H.workspace(nbytes, qkv.device)
    with profiling.launch(f"attn_bwd_dq_mfma<{head_dim}> + attn_bwd_dkdv_mfma<{head_dim}>",
                          2.0 * attn_flops(batch, seq, heads, head_dim)):
        H.call("rh_attn_bwd", H.dtype_code(qkv), batch, seq, heads, head_dim, base, base + dl * es,
               base + 2 * dl * es, _ld(qkv), ctx.data_ptr(), H.ptr(ctx_lo), dl, dctx.data_ptr(), _ld(dctx),
               lse.data_ptr(), dbase, dbase + dl * es, dbase + 2 * dl * es, 3 * dl, 1.0 / math.sqrt(head_dim), 1,
               H.ptr(ws), nbytes, H.stream_of(qkv))
    return dqkv


# ---------------------------------------------------------------------------
# composite pieces shared by the Functions
# ---------------------------------------------------------------------------
def _check_heads(width: int, num_heads: int) -> int:
    if num_heads <= 0 or width % num_heads:
        raise ValueError("model_dim must be divisible by num_heads")
    return width // num_heads


def _attention_forward(n1, wq, wk, wv, num_heads, batch, seq):
    head_dim = _check_heads(wq.shape[0], num_heads)
    qkv = linear_fwd(n1, [wq, wk, wv])
    ctx, lse, ctx_lo = attn_fwd(qkv, batch, seq, num_heads, head_dim)
    return qkv, ctx, lse, ctx_lo, head_dim


# ---------------------------------------------------------------------------
# autograd Functions
# ---------------------------------------------------------------------------
class _LinearFn(torch.autograd.Function):
    """F.linear(x, w), bias-free (resihp/model.py:55-58,77-78,116; resihp/parallel/tp.py:235-237,243,247-248,272)."""

    @staticmethod
    def forward(ctx, x, w):
        H.require_gpu(x, w)
        x2 = _as_rows(x)
        y = linear_fwd(x2, [w.contiguous()])
        ctx.save_for_backward(x2)
        ctx.w = w
        ctx.in_shape = x.shape
        return y.view(*x.shape[:-1], w.shape[0]) if y.is_contiguous() else y.unflatten(0, x.shape[:-1])

    @staticmethod
    def backward(ctx, dy):
        (x2,) = ctx.saved_tensors
        w = ctx.w
        dy2 = _as_rows(dy)
        dx = None
        if ctx.needs_input_grad[0]:
            dx = linear_dgrad(dy2, [w.contiguous()]).reshape(ctx.in_shape)
        linear_wgrad(dy2, x2, [w])
        return dx, None


class _LayerNormFn(torch.autograd.Function):
    """F.layer_norm over the last dim (resihp/model.py:89,91,115; resihp/parallel/tp.py:262,264,268)."""

    @staticmethod
    def forward(ctx, x, w, b, eps):
        H.require_gpu(x, w, b)
        x2 = _as_rows(x).contiguous()
        y, mean, rstd = ln_fwd(x2, w, b, eps)
        ctx.save_for_backward(x2, mean, rstd)
        ctx.params = (w, b)
        ctx.shape = x.shape
        return y.view(x.shape)

    @staticmethod
    def backward(ctx, dy):
        x2, mean, rstd = ctx.saved_tensors
        w, b = ctx.params
        dx = ln_bwd(_as_rows(dy), x2, mean, rstd, w, b, None)
        return (dx.view(ctx.shape) if ctx.needs_input_grad[0] else None), None, None, None


class _EmbeddingFn(torch.autograd.Function):
    """Token embedding (+ learned positions): resihp/model.py:108-109,128-129; the vocab-parallel form
    with out-of-slice ids zeroed is resihp/parallel/tp.py:222-228,256-257."""

    @staticmethod
    def forward(ctx, tokens, wtok, wpos, vocab_start, vocab_rows):
        H.require_gpu(tokens, wtok, wpos)
        if tokens.dtype != torch.int64:
            raise TypeError("token ids must be int64")
        if tokens.dim() != 2:
            raise ValueError("tokens must be [batch, seq]")
        batch, seq = tokens.shape
        dim = wtok.shape[1]
        tokens = tokens.contiguous()
        out = torch.empty((batch, seq, dim), dtype=wtok.dtype, device=wtok.device)
        if wpos is not None and wpos.shape[0] < seq:
            raise ValueError("sequence longer than the position table")
        H.call("rh_embedding_fwd", _same_dtype(wtok, wpos), batch, seq, dim, tokens.data_ptr(), wtok.data_ptr(),
               vocab_start, vocab_rows, H.ptr(wpos), out.data_ptr(), H.stream_of(wtok))
        ctx.save_for_backward(tokens)
        ctx.params = (wtok, wpos)
        ctx.vocab = (vocab_start, vocab_rows)
        return out

    @staticmethod
    def backward(ctx, dout):
        (tokens,) = ctx.saved_tensors
        wtok, wpos = ctx.params
        batch, seq = tokens.shape
        dim = wtok.shape[1]
        dout = dout.contiguous()
        want_tok, want_pos = _wants(wtok), _wants(wpos)
        if not (want_tok or want_pos):
            return None, None, None, None, None
        gt = gp = None
        acc = True
        if want_tok:
            gt, acc_t = _grad_target(wtok)
        if want_pos:
            gp, acc_p = _grad_target(wpos)
        # dpos covers only the first `seq` rows of the position table
        if want_pos and wpos.shape[0] != seq:
            if not acc_p:
                gp.zero_()
            acc_p = True
        nbytes = H.query("rh_embedding_bwd_workspace_bytes", batch, seq, dim)
        ws = H.workspace(nbytes, dout.device)
        stream = H.stream_of(dout)
        if want_tok:
            H.call("rh_embedding_bwd", H.dtype_code(dout), batch, seq, dim, tokens.data_ptr(), dout.data_ptr(),
                   ctx.vocab[0], ctx.vocab[1], gt.data_ptr(), None, 1 if acc_t else 0, H.ptr(ws), nbytes, stream)
            _finish_grad(wtok, gt)
        if want_pos:
            H.call("rh_embedding_bwd", H.dtype_code(dout), batch, seq, dim, tokens.data_ptr(), dout.data_ptr(),
                   ctx.vocab[0], ctx.vocab[1], None, gp.data_ptr(), 1 if acc_p else 0, H.ptr(ws), nbytes, stream)
            _finish_grad(wpos, gp)
        return None, None, None, None, None


class _AttentionFn(torch.autograd.Function):
    """CausalSelfAttention.forward (resihp/model.py:60-71): q/k/v projections, causal softmax
    attention, out_proj -- as one fused QKV GEMM, the flash kernel and the out GEMM."""

    @staticmethod
    def forward(ctx, x, wq, wk, wv, wo, num_heads):
        H.require_gpu(x, wq, wk, wv, wo)
        batch, seq, dim = x.shape
        x2 = _as_rows(x).contiguous()
        qkv, c, lse, c_lo, head_dim = _attention_forward(x2, wq, wk, wv, num_heads, batch, seq)
        out = linear_fwd(c, [wo])
        ctx.save_for_backward(x2, qkv, c, lse, c_lo)
        ctx.params = (wq, wk, wv, wo)
        ctx.meta = (batch, seq, num_heads, head_dim)
        return out.view(batch, seq, wo.shape[0])

    @staticmethod
    def backward(ctx, dout):
        x2, qkv, c, lse, c_lo = ctx.saved_tensors
        wq, wk, wv, wo = ctx.params
        batch, seq, num_heads, head_dim = ctx.meta
        dout2 = _as_rows(dout).contiguous()
        dctx = linear_dgrad(dout2, [wo])
        dqkv = attn_bwd(dctx, qkv, c, lse, batch, seq, num_heads, head_dim, c_lo)
        dx = linear_dgrad(dqkv, [wq, wk, wv]) if ctx.needs_input_grad[0] else None
        linear_wgrad_group([(dout2, c, [wo]), (dqkv, x2, [wq, wk, wv])])
        return (dx.view(batch, seq, -1) if dx is not None else None), None, None, None, None, None


class _MLPFn(torch.autograd.Function):
    """MLP.forward = fc2(gelu(fc1(x))) (resihp/model.py:74-81): GELU fused into the fc1 epilogue
    forward and into the fc2 dgrad epilogue backward."""

    @staticmethod
    def forward(ctx, x, w1, w2):
        H.require_gpu(x, w1, w2)
        x2 = _as_rows(x).contiguous()
        gd = _rows(x2.shape[0], w1.shape[0], x2)  # gelu'(fc1 output), kept for the backward
        h = linear_fwd(x2, [w1], gelu_deriv=gd)
        y = linear_fwd(h, [w2])
        ctx.save_for_backward(x2, gd, h)
        ctx.params = (w1, w2)
        ctx.shape = x.shape
        return y.view(*x.shape[:-1], w2.shape[0])

    @staticmethod
    def backward(ctx, dy):
        x2, gd, h = ctx.saved_tensors
        w1, w2 = ctx.params
        dy2 = _as_rows(dy).contiguous()
        du = linear_dgrad(dy2, [w2], gelu_deriv=gd)
        dx = linear_dgrad(du, [w1]) if ctx.needs_input_grad[0] else None
        linear_wgrad_group([(dy2, h, [w2]), (du, x2, [w1])])
        return (dx.view(ctx.shape) if dx is not None else None), None, None


_SIDE_STREAMS: dict = {}


def _side_stream(device: torch.device) -> torch.cuda.Stream:
    """One extra stream per device (default priority) for work that overlaps the main chain."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    st = _SIDE_STREAMS.get(idx)
    if st is None:
        st = _SIDE_STREAMS[idx] = torch.cuda.Stream(device=idx)
    return st


class _BlockFn(torch.autograd.Function):
    """One pre-LN decoder block, x + attn(LN1 x) then + mlp(LN2 .) (resihp/model.py:94-97), or one
    TP rank's shard of it with row-parallel partial sums (resihp/parallel/tp.py:260-265).

    Forward: LN1 -> fused QKV GEMM -> flash attention -> out GEMM with the residual add in its
    epilogue -> LN2 -> fc1 GEMM with GELU epilogue (which also stores gelu' of its input for the
    backward) -> fc2 GEMM with the residual add.  Backward reverses it; the residual-branch
    gradient is added inside the LayerNorm backward kernels and the stored gelu' is applied in
    the fc2 dgrad epilogue.
    """

    @staticmethod
    def forward(ctx, x, g1, b1, wq, wk, wv, wo, g2, b2, w1, w2, num_heads, eps):
        H.require_gpu(x, g1, b1, wq, wk, wv, wo, g2, b2, w1, w2)
        batch, seq, dim = x.shape
        x2 = _as_rows(x).contiguous()
        n1, mu1, rs1 = ln_fwd(x2, g1, b1, eps)
        qkv, c, lse, c_lo, head_dim = _attention_forward(n1, wq, wk, wv, num_heads, batch, seq)
        x1 = linear_fwd(c, [wo], residual=x2)
        n2, mu2, rs2 = ln_fwd(x1, g2, b2, eps)
        gd = _rows(x2.shape[0], w1.shape[0], x2)  # gelu'(fc1 output), kept for the backward
        h = linear_fwd(n2, [w1], gelu_deriv=gd)
        out = linear_fwd(h, [w2], residual=x1)
        ctx.save_for_backward(x2, n1, mu1, rs1, qkv, c, lse, c_lo, x1, n2, mu2, rs2, gd, h)
        ctx.params = (g1, b1, wq, wk, wv, wo, g2, b2, w1, w2)
        ctx.meta = (batch, seq, num_heads, head_dim)
        return out.view(batch, seq, dim)

    @staticmethod
    def backward(ctx, dout):
        x2, n1, mu1, rs1, qkv, c, lse, c_lo, x1, n2, mu2, rs2, gd, h = ctx.saved_tensors
        g1, b1, wq, wk, wv, wo, g2, b2, w1, w2 = ctx.params
        batch, seq, num_heads, head_dim = ctx.meta
        d2 = _as_rows(dout).contiguous()
        # the chain of input gradients first: MLP branch, then the attention branch
        du = linear_dgrad(d2, [w2], gelu_deriv=gd)
        dn2 = linear_dgrad(du, [w1])
        dx1 = ln_bwd(dn2, x1, mu2, rs2, g2, b2, dres=d2)
        dctx = linear_dgrad(dx1, [wo])
        dqkv = attn_bwd(dctx, qkv, c, lse, batch, seq, num_heads, head_dim, c_lo)
        wgrads = [(d2, h, [w2]), (du, n2, [w1]), (dx1, c, [wo]), (dqkv, n1, [wq, wk, wv])]
        if os.environ.get("RESIHP_WGRAD_STREAM", "1") != "0" and not profiling.active():
            # the block's four weight gradients (token count as K, one grouped launch) on a side
            # stream, issued first, so the q/k/v input gradient and the LN1 backward run on the
            # CUs its tiles leave idle (measured: 0.950 against 0.975 ms per step at the TP=4
            # shard of the 1.3B block); the main stream joins it before returning.  Per-kernel
            # timing (profiling) runs them one after another, each on the whole chip.
            main = torch.cuda.current_stream(d2.device)
            side = _side_stream(d2.device)
            side.wait_stream(main)
            with torch.cuda.stream(side):
                linear_wgrad_group(wgrads)
            dn1 = linear_dgrad(dqkv, [wq, wk, wv])
            dx = ln_bwd(dn1, x2, mu1, rs1, g1, b1, dres=dx1)
            main.wait_stream(side)
        else:  # RESIHP_WGRAD_STREAM=0: one stream, input gradients first
            dn1 = linear_dgrad(dqkv, [wq, wk, wv])
            dx = ln_bwd(dn1, x2, mu1, rs1, g1, b1, dres=dx1)
            linear_wgrad_group(wgrads)
        return (dx.view(batch, seq, -1),) + (None,) * 12


class _NextTokenLossFn(torch.autograd.Function):
    """next_token_loss = F.cross_entropy(logits[:, :-1].reshape(-1, V), tokens[:, 1:].reshape(-1))
    (resihp/reference.py:41-50), read in place from the [B, S, V] logits."""

    @staticmethod
    def forward(ctx, logits, tokens, vocab_size):
        H.require_gpu(logits, tokens)
        batch, seq, vocab = logits.shape
        if vocab != vocab_size:
            raise ValueError(f"logits last dim {vocab} != vocab_size {vocab_size}")
        if tokens.shape != (batch, seq):
            raise ValueError("tokens must be [batch, seq] matching the logits")
        if seq < 2:
            raise ValueError("next-token loss needs seq >= 2")
        if logits.stride(2) != 1 or logits.stride(0) != seq * logits.stride(1):
            logits = logits.contiguous()
        ld = logits.stride(1)
        tokens = tokens.contiguous()
        dev = logits.device
        rows = batch * seq
        lse = torch.empty(rows, dtype=torch.float32, device=dev)
        loss = torch.empty((), dtype=torch.float32, device=dev)
        dl = None
        # (grad mode is off inside Function.forward; needs_input_grad says whether backward will run)
        if ctx.needs_input_grad[0]:
            ld_d = (vocab + 7) // 8 * 8
            dl = torch.empty((rows, ld_d), dtype=logits.dtype, device=dev)
        nbytes = H.query("rh_xent_workspace_bytes", batch, seq)
        ws = H.workspace(nbytes, dev)
        es = logits.element_size()
        moved = rows * vocab * es * (1 if dl is None else 2) + 12 * rows  # logits (+ dlogits), tokens, lse
        with profiling.launch("xent_fwd" if dl is None else "xent_fwd (+ dlogits)", 0.0, moved):
            H.call("rh_xent_fwd", H.dtype_code(logits), batch, seq, vocab, logits.data_ptr(), ld, tokens.data_ptr(),
                   lse.data_ptr(), loss.data_ptr(), H.ptr(dl), 0 if dl is None else dl.shape[1], H.ptr(ws), nbytes,
                   H.stream_of(logits))
        ctx.save_for_backward(logits, tokens, lse)
        ctx.dl = dl
        ctx.shape = (batch, seq, vocab)
        return loss

    @staticmethod
    def backward(ctx, grad):
        logits, tokens, lse = ctx.saved_tensors
        batch, seq, vocab = ctx.shape
        grad = grad.to(torch.float32).contiguous()
        dl = ctx.dl
        if dl is not None:
            ctx.dl = None  # fused gradient: scale by the incoming grad (no-op when it is 1)
            H.call("rh_scale_by", H.dtype_code(dl), dl.shape[0], vocab, dl.shape[1], dl.data_ptr(), grad.data_ptr(),
                   H.stream_of(dl))
        else:
            ld_d = (vocab + 7) // 8 * 8
            dl = torch.empty((batch * seq, ld_d), dtype=logits.dtype, device=logits.device)
            H.call("rh_xent_bwd", H.dtype_code(logits), batch, seq, vocab, logits.data_ptr(), logits.stride(1),
                   tokens.data_ptr(), lse.data_ptr(), grad.data_ptr(), dl.data_ptr(), ld_d, H.stream_of(logits))
        return dl.view(batch, seq, dl.shape[1])[:, :, :vocab], None, None


class _LMHeadNextTokenLossFn(torch.autograd.Function):
    """lm_head then next_token_loss, fused (resihp/model.py:116,133 + resihp/reference.py:41-50):
    the loss from x [B, S, d] (the final LayerNorm's output) and W [V, d] without the [B, S, V]
    logits or their gradient in memory.  Backward returns dx and writes W.grad (accumulating,
    like the other parameters)."""

    @staticmethod
    def forward(ctx, x, w, tokens):
        H.require_gpu(x, w, tokens)
        if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
            raise TypeError("the fused LM-head loss runs in bfloat16")
        if tokens.dtype != torch.int64:
            raise TypeError("token ids must be int64")
        batch, seq, dim = x.shape
        if tokens.shape != (batch, seq):
            raise ValueError("tokens must be [batch, seq] matching the hidden states")
        vocab = w.shape[0]
        if w.shape[1] != dim:
            raise ValueError(f"LM head of width {w.shape[1]} applied to hidden states of width {dim}")
        x2 = _as_rows(x).contiguous()
        wc = w.contiguous()
        tokens = tokens.contiguous()
        fwd_b = ctypes.c_int64(0)
        bwd_b = ctypes.c_int64(0)
        H.call("rh_lmhead_xent_workspace_bytes", batch, seq, vocab, dim, ctypes.byref(fwd_b), ctypes.byref(bwd_b))
        ws = H.workspace(fwd_b.value, x.device)
        lse = torch.empty(batch * seq, dtype=torch.float32, device=x.device)
        loss = torch.empty((), dtype=torch.float32, device=x.device)
        with profiling.launch("lmhead_xent_fwd (LSE GEMM + combine)", 2.0 * batch * seq * vocab * dim):
            H.call("rh_lmhead_xent_fwd", batch, seq, vocab, dim, x2.data_ptr(), wc.data_ptr(), tokens.data_ptr(),
                   lse.data_ptr(), loss.data_ptr(), H.ptr(ws), fwd_b.value, H.stream_of(x))
        ctx.save_for_backward(x2, tokens, lse)
        ctx.w = w
        ctx.meta = (batch, seq, vocab, dim, bwd_b.value)
        return loss

    @staticmethod
    def backward(ctx, grad):
        x2, tokens, lse = ctx.saved_tensors
        w = ctx.w
        batch, seq, vocab, dim, nbytes = ctx.meta
        grad = grad.to(torch.float32).contiguous()
        dx = torch.empty_like(x2)
        if _wants(w):
            gw, acc = _grad_target(w)
        else:
            gw, acc = torch.empty_like(w, memory_format=torch.contiguous_format), False
        ws = H.workspace(nbytes, x2.device)
        with profiling.launch("lmhead_xent_bwd (recompute + dW + dX, chunked)", 3 * 2.0 * batch * seq * vocab * dim):
            H.call("rh_lmhead_xent_bwd", batch, seq, vocab, dim, x2.data_ptr(), w.contiguous().data_ptr(),
                   tokens.data_ptr(), lse.data_ptr(), grad.data_ptr(), dx.data_ptr(), gw.data_ptr(), 1 if acc else 0,
                   H.ptr(ws), nbytes, H.stream_of(x2))
        if _wants(w):
            _finish_grad(w, gw)
        return dx.view(batch, seq, dim), None, None


# ---------------------------------------------------------------------------
# functional entry points
# ---------------------------------------------------------------------------
def linear(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    return _LinearFn.apply(x, weight)


def layer_norm(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, eps: float = LN_EPS) -> torch.Tensor:
    return _LayerNormFn.apply(x, weight, bias, eps)


def embedding(tokens: torch.Tensor, weight: torch.Tensor, position: torch.Tensor | None = None, *,
              vocab_start: int = 0, vocab_rows: int | None = None) -> torch.Tensor:
    rows = weight.shape[0] if vocab_rows is None else vocab_rows
    return _EmbeddingFn.apply(tokens, weight, position, vocab_start, rows)


def causal_self_attention(x, wq, wk, wv, wo, num_heads: int) -> torch.Tensor:
    return _AttentionFn.apply(x, wq, wk, wv, wo, num_heads)


def mlp(x, w1, w2) -> torch.Tensor:
    return _MLPFn.apply(x, w1, w2)


def transformer_block(x, g1, b1, wq, wk, wv, wo, g2, b2, w1, w2, num_heads: int, eps: float = LN_EPS):
    return _BlockFn.apply(x, g1, b1, wq, wk, wv, wo, g2, b2, w1, w2, num_heads, eps)


def next_token_loss(logits: torch.Tensor, tokens: torch.Tensor, vocab_size: int) -> torch.Tensor:
    return _NextTokenLossFn.apply(logits, tokens, vocab_size)


def lm_head_next_token_loss(x: torch.Tensor, weight: torch.Tensor, tokens: torch.Tensor) -> torch.Tensor:
    """next_token_loss(F.linear(x, weight), tokens, V) without materialising the logits (bf16)."""
    return _LMHeadNextTokenLossFn.apply(x, weight, tokens)
