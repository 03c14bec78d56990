"""Kernel-level parity on the GPU: every C ABI entry point against fp32 torch / the oracle.

Tolerances are relative to the reference's infinity norm (max|a-b| / max|ref|):
1e-5 for fp32 paths, bf16 paths at the storage precision (a bf16 output carries
~4e-3 rounding), bit-exact for byte movement.
"""

import ctypes
import math

import pytest
import torch
from torch.nn import functional as F

from conftest import rel_inf
from oracle import torch_ref
from resihp import _hip as H
from resihp import ops
from resihp.parallel import reshard

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2  # one bf16 rounding of the output plus fp32 accumulation-order noise
F32_TOL = 1e-5


def _rand(*shape, dtype=torch.bfloat16, scale=1.0, seed=0, dev="cuda"):
    g = torch.Generator(device="cpu").manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dev, dtype)


def _gemm_ref(layout, A, B):
    A32, B32 = A.float(), B.float()
    if layout == H.RH_GEMM_NT:
        return A32 @ B32.t()
    if layout == H.RH_GEMM_NN:
        return A32 @ B32
    return A32.t() @ B32


SHAPES = [(128, 128, 64), (256, 384, 512), (100, 77, 50), (33, 200, 129), (1, 8, 8), (513, 257, 1000),
          (256, 384, 1000)]  # ragged K with aligned M/N: direct-to-LDS bulk + register-staged K tail


@pytest.fixture(params=["auto", "0", "0w4", "0w8", "1", "2", "3"])
def gemm_tile(request, monkeypatch):
    """Pin the bf16 GEMM tile shape (256x256 / 256x128 / 128x128 / 256x192, the last for NT
    only) or let the planner choose; "0w4" / "0w8" run every 256x256 tile on the 4-wave / 8-wave
    kernel (by default unsplit single GEMMs take the 8-wave one, split-K slices the 4-wave one)."""
    monkeypatch.delenv("RESIHP_GEMM_WAVES", raising=False)
    if request.param == "auto":
        monkeypatch.delenv("RESIHP_GEMM_TILE", raising=False)
    elif request.param in ("0w4", "0w8"):
        monkeypatch.setenv("RESIHP_GEMM_TILE", "0")
        monkeypatch.setenv("RESIHP_GEMM_WAVES", request.param[-1])
    else:
        monkeypatch.setenv("RESIHP_GEMM_TILE", request.param)
    return request.param


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("layout", [H.RH_GEMM_NT, H.RH_GEMM_NN, H.RH_GEMM_TN])
@pytest.mark.parametrize("M,N,K", SHAPES)
def test_gemm_layouts(cuda, gemm_tile, dtype, layout, M, N, K):
    if dtype == torch.float32 and gemm_tile != "auto":
        pytest.skip("the tile override only applies to the bf16 kernels")
    a_shape = (K, M) if layout == H.RH_GEMM_TN else (M, K)
    b_shape = (N, K) if layout == H.RH_GEMM_NT else (K, N)
    A = _rand(*a_shape, dtype=dtype, seed=1)
    B = _rand(*b_shape, dtype=dtype, seed=2)
    D = torch.empty(M, N, dtype=dtype, device=cuda)
    ops.gemm(layout, M, N, K, A, A.stride(0), [B], B.stride(0), [D], N)
    err = rel_inf(D, _gemm_ref(layout, A, B))
    assert err <= (BF16_TOL if dtype == torch.bfloat16 else F32_TOL), err


@pytest.mark.parametrize("layout", [H.RH_GEMM_NT, H.RH_GEMM_NN, H.RH_GEMM_TN])
def test_gemm_split_k_matches_unsplit(cuda, gemm_tile, layout):
    """Few output tiles and a long K take the split-K path; it must agree with fp32."""
    M, N, K = 256, 384, 8192
    a_shape = (K, M) if layout == H.RH_GEMM_TN else (M, K)
    b_shape = (N, K) if layout == H.RH_GEMM_NT else (K, N)
    A = _rand(*a_shape, seed=3)
    B = _rand(*b_shape, seed=4)
    D = torch.empty(M, N, dtype=torch.bfloat16, device=cuda)
    ops.gemm(layout, M, N, K, A, A.stride(0), [B], B.stride(0), [D], N)
    assert rel_inf(D, _gemm_ref(layout, A, B)) <= BF16_TOL


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_gemm_epilogues(cuda, gemm_tile, dtype):
    M, N, K = 192, 320, 256
    A = _rand(M, K, dtype=dtype, seed=5)
    B = _rand(N, K, dtype=dtype, seed=6, scale=0.1)
    R = _rand(M, N, dtype=dtype, seed=7)
    tol = BF16_TOL if dtype == torch.bfloat16 else F32_TOL
    acc = A.float() @ B.float().t()
    # residual: D = acc + R
    D = torch.empty(M, N, dtype=dtype, device=cuda)
    ops.gemm(H.RH_GEMM_NT, M, N, K, A, K, [B], K, [D], N, beta=1.0, C=R, ldc=N)
    assert rel_inf(D, acc + R.float()) <= tol
    # alpha / in-place beta accumulate
    D2 = R.clone()
    ops.gemm(H.RH_GEMM_NT, M, N, K, A, K, [B], K, [D2], N, alpha=0.5, beta=2.0)
    assert rel_inf(D2, 0.5 * acc + 2 * R.float()) <= tol
    # GELU: aux_out = pre-activation, D = gelu(pre)
    U = torch.empty(M, N, dtype=dtype, device=cuda)
    ops.gemm(H.RH_GEMM_NT, M, N, K, A, K, [B], K, [D], N, epilogue=H.RH_EPI_GELU, aux_out=U, ldaux=N)
    assert rel_inf(U, acc) <= tol
    assert rel_inf(D, F.gelu(acc)) <= tol
    # GELU_GRAD: D = acc * gelu'(aux)
    ops.gemm(H.RH_GEMM_NT, M, N, K, A, K, [B], K, [D], N, epilogue=H.RH_EPI_GELU_GRAD, aux=R, ldaux=N)
    x = R.float().requires_grad_(True)
    F.gelu(x).backward(acc)
    assert rel_inf(D, x.grad) <= tol
    # GELU_DERIV: aux_out = gelu'(pre-activation), D = gelu(pre)
    G = torch.empty(M, N, dtype=dtype, device=cuda)
    ops.gemm(H.RH_GEMM_NT, M, N, K, A, K, [B], K, [D], N, epilogue=H.RH_EPI_GELU_DERIV, aux_out=G, ldaux=N)
    pre = acc.clone().requires_grad_(True)
    F.gelu(pre).backward(torch.ones_like(acc))
    assert rel_inf(D, F.gelu(acc)) <= tol
    assert rel_inf(G, pre.grad) <= tol
    # MUL_AUX: D = acc * aux
    ops.gemm(H.RH_GEMM_NT, M, N, K, A, K, [B], K, [D], N, epilogue=H.RH_EPI_MUL_AUX, aux=R, ldaux=N)
    assert rel_inf(D, acc * R.float()) <= tol


def test_gemm_stages_equal_one_call(cuda):
    """rh_gemm_stage MAIN then REDUCE (a split-K plan) gives exactly rh_gemm's result."""
    import ctypes

    M, N, K = 512, 768, 8192  # TN wgrad shape with few tiles: the planner splits K
    A = _rand(K, M, seed=50)
    B = _rand(K, N, seed=51)
    outs = []
    for staged in (False, True):
        D = torch.empty(M, N, dtype=torch.bfloat16, device=cuda)
        desc = H.rh_gemm_desc()
        desc.dtype, desc.layout, desc.epilogue = H.RH_DTYPE_BF16, H.RH_GEMM_TN, H.RH_EPI_NONE
        desc.b_nseg = desc.d_nseg = 1
        desc.M, desc.N, desc.K = M, N, K
        desc.A, desc.lda, desc.B[0], desc.ldb, desc.D[0], desc.ldd = A.data_ptr(), M, B.data_ptr(), N, D.data_ptr(), N
        desc.alpha = 1.0
        nbytes = H.query("rh_gemm_workspace_bytes", ctypes.byref(desc))
        assert nbytes > 0
        ws = H.workspace(nbytes, cuda)
        if staged:
            H.call("rh_gemm_stage", ctypes.byref(desc), H.ptr(ws), nbytes, H.RH_GEMM_STAGE_MAIN, None)
            H.call("rh_gemm_stage", ctypes.byref(desc), H.ptr(ws), nbytes, H.RH_GEMM_STAGE_REDUCE, None)
        else:
            H.call("rh_gemm", ctypes.byref(desc), H.ptr(ws), nbytes, None)
        torch.cuda.synchronize()
        outs.append(D)
    assert torch.equal(outs[0], outs[1])
    assert rel_inf(outs[0], A.float().t() @ B.float()) <= BF16_TOL


@pytest.mark.parametrize("K", [64, 96])
def test_gemm_bf16_rounding_matches_torch(cuda, K):
    """The bf16 store rounds to nearest even exactly like torch's float->bfloat16 conversion:
    D[m, n] = hi[n] + lo[n] is an exact fp32 sum (two bf16 terms of a one-hot-pair product)
    whose bf16 rounding is compared bit for bit, ties and negative values included.
    K = 64 takes the direct-to-LDS kernel, K = 96 the register-staged one."""
    g = torch.Generator().manual_seed(40)
    N = 256
    hi = torch.cat([torch.ones(64), -torch.ones(32), torch.randn(160, generator=g) * 100]).to(torch.bfloat16)
    # low parts around the bf16 rounding boundary of hi: exact ties (2^-8 * |hi|), just above/below
    rel = torch.tensor([0.5, 0.75, 0.25, 0.5 + 2 ** -6, 0.5 - 2 ** -6, 1.5, -0.5, -0.75])
    lo = (hi.float().abs() * 2 ** -7 * rel.repeat(N // len(rel))).to(torch.bfloat16)
    A = torch.zeros(64, K, dtype=torch.bfloat16)
    A[:, 0] = 1.0
    A[:, 1] = 1.0
    B = torch.zeros(N, K, dtype=torch.bfloat16)
    B[:, 0] = hi
    B[:, 1] = lo
    want = (hi.float() + lo.float()).to(torch.bfloat16).expand(64, N)
    D = torch.empty(64, N, dtype=torch.bfloat16, device=cuda)
    ops.gemm(H.RH_GEMM_NT, 64, N, K, A.to(cuda), K, [B.to(cuda)], K, [D], N)
    assert torch.equal(D.cpu().view(torch.int16), want.contiguous().view(torch.int16))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_gemm_segments_act_as_one_matrix(cuda, gemm_tile, dtype):
    """Three separate q/k/v weights as B segments (forward, dgrad) and as D segments (wgrad)."""
    T, d, dl = 320, 256, 128
    tol = BF16_TOL if dtype == torch.bfloat16 else F32_TOL
    x = _rand(T, d, dtype=dtype, seed=8)
    ws = [_rand(dl, d, dtype=dtype, seed=9 + i, scale=0.05) for i in range(3)]
    W = torch.cat(ws, 0)
    y = ops.linear_fwd(x, ws)
    assert rel_inf(y, x.float() @ W.float().t()) <= tol
    dy = _rand(T, 3 * dl, dtype=dtype, seed=12)
    dx = ops.linear_dgrad(dy, ws)
    assert rel_inf(dx, dy.float() @ W.float()) <= tol
    params = [torch.nn.Parameter(w.clone()) for w in ws]
    ops.linear_wgrad(dy, x, params)
    ops.linear_wgrad(dy, x, params)  # second call accumulates into .grad
    full = 2 * (dy.float().t() @ x.float())
    for i, p in enumerate(params):
        assert rel_inf(p.grad, full[i * dl:(i + 1) * dl]) <= tol


def test_gemm_qkv_projection_at_shard_size(cuda):
    """The one-TP-rank QKV projection of a 1.3B block: M 8192, N 1536, K 2048."""
    x = _rand(8192, 2048, seed=13)
    ws = [_rand(512, 2048, seed=14 + i, scale=0.02) for i in range(3)]
    y = ops.linear_fwd(x, ws)
    ref = x.float() @ torch.cat(ws, 0).float().t()
    assert rel_inf(y, ref) <= 2e-2


@pytest.mark.parametrize("padded", [True, False])
def test_linear_wgrad_ragged_outputs(cuda, padded):
    """LM-head-style weight gradient: 50257 output rows.  With dy a view of rows padded to a
    multiple of 8 (the logits layout) the GEMM runs over the rounded count into a scratch row
    segment; without padding it takes the plain path.  Both equal the fp32 product, and a second
    call accumulates."""
    T, V, d = 128, 50257, 64
    buf = _rand(T, V + 7, dtype=torch.bfloat16, seed=40, scale=0.01)
    dy = buf[:, :V] if padded else buf[:, :V].contiguous()
    x = _rand(T, d, dtype=torch.bfloat16, seed=41)
    w = torch.nn.Parameter(torch.zeros(V, d, dtype=torch.bfloat16, device=cuda))
    ops.linear_wgrad(dy, x, [w])
    ref = dy.float().t() @ x.float()
    assert rel_inf(w.grad, ref) <= BF16_TOL
    ops.linear_wgrad(dy, x, [w])
    assert rel_inf(w.grad, 2 * ref) <= BF16_TOL


def _attn_ref(q, k, v, heads):
    """fp32 reference attention on [B, S, H*Dh] rows (the reference's explicit S x S form)."""
    B, S, W = q.shape
    dh = W // heads
    qh, kh, vh = (t.float().view(B, S, heads, dh).transpose(1, 2) for t in (q, k, v))
    s = (qh @ kh.transpose(-2, -1).contiguous()) / math.sqrt(dh)
    s = s.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool, device=q.device), 1), float("-inf"))
    return (torch.softmax(s, -1) @ vh).transpose(1, 2).reshape(B, S, W)


@pytest.mark.parametrize("dtype,head_dim,seq,heads,batch", [
    (torch.bfloat16, 128, 256, 2, 2),
    (torch.bfloat16, 128, 200, 1, 1),
    (torch.bfloat16, 64, 320, 3, 2),
    (torch.bfloat16, 64, 1024, 2, 1),
    (torch.bfloat16, 128, 2048, 2, 2),
    (torch.bfloat16, 128, 1000, 3, 1),
    (torch.bfloat16, 64, 63, 1, 3),
    (torch.bfloat16, 32, 96, 2, 2),
    (torch.float32, 16, 32, 4, 4),
    (torch.float32, 64, 130, 2, 1),
])
def test_attention_forward_backward(cuda, dtype, head_dim, seq, heads, batch):
    W = heads * head_dim
    qkv = _rand(batch * seq, 3 * W, dtype=dtype, seed=20)
    ctx, lse, ctx_lo = ops.attn_fwd(qkv, batch, seq, heads, head_dim)
    q, k, v = (qkv[:, i * W:(i + 1) * W].reshape(batch, seq, W).float().requires_grad_(True) for i in range(3))
    ref = _attn_ref(q, k, v, heads)
    tol = 2e-2 if dtype == torch.bfloat16 else F32_TOL
    assert rel_inf(ctx.view(batch, seq, W), ref) <= tol
    # lse = log sum_j exp(s_ij)
    qh = q.detach().view(batch, seq, heads, head_dim).transpose(1, 2)
    kh = k.detach().view(batch, seq, heads, head_dim).transpose(1, 2)
    s = (qh @ kh.transpose(-2, -1).contiguous()) / math.sqrt(head_dim)
    s = s.masked_fill(torch.triu(torch.ones(seq, seq, dtype=torch.bool, device=cuda), 1), float("-inf"))
    assert rel_inf(lse, torch.logsumexp(s, -1)) <= (1e-5 if dtype == torch.float32 else 5e-3)
    dout = _rand(batch * seq, W, dtype=dtype, seed=21)
    dqkv = ops.attn_bwd(dout, qkv, ctx, lse, batch, seq, heads, head_dim, ctx_lo)
    ref.backward(dout.float().view(batch, seq, W))
    errs = {}
    for i, t in enumerate((q, k, v)):
        errs["d" + "qkv"[i]] = rel_inf(dqkv[:, i * W:(i + 1) * W].reshape(batch, seq, W), t.grad)
    print({k: f"{e:.2e}" for k, e in errs.items()})
    for name, err in errs.items():
        assert err <= (2e-2 if dtype == torch.bfloat16 else 1e-4), (name, err)


@pytest.mark.parametrize("dtype,rows,dim", [(torch.float32, 64, 64), (torch.float32, 37, 100),
                                            (torch.bfloat16, 512, 2048), (torch.bfloat16, 130, 768),
                                            (torch.float32, 8, 5000), (torch.bfloat16, 3, 24),
                                            # two waves per row (1024 < dim <= 2048): ragged dim,
                                            # odd rows, a last row pair with one row
                                            (torch.bfloat16, 37, 1544), (torch.bfloat16, 8193, 2048),
                                            (torch.bfloat16, 1, 1032)])
def test_layernorm_forward_backward(cuda, dtype, rows, dim):
    x = _rand(rows, dim, dtype=dtype, seed=30, scale=2.0) + 0.5
    w = torch.nn.Parameter(_rand(dim, dtype=dtype, seed=31) * 0.2 + 1.0)
    b = torch.nn.Parameter(_rand(dim, dtype=dtype, seed=32) * 0.2)
    y, mean, rstd = ops.ln_fwd(x, w, b, 1e-5)
    xr = x.float().requires_grad_(True)
    wr = w.detach().float().requires_grad_(True)
    br = b.detach().float().requires_grad_(True)
    yr = F.layer_norm(xr, (dim,), wr, br, 1e-5)
    tol = F32_TOL if dtype == torch.float32 else BF16_TOL
    assert rel_inf(y, yr) <= tol
    dy = _rand(rows, dim, dtype=dtype, seed=33)
    dres = _rand(rows, dim, dtype=dtype, seed=34)
    dx = ops.ln_bwd(dy, x, mean, rstd, w, b, dres)
    yr.backward(dy.float())
    assert rel_inf(dx, xr.grad + dres.float()) <= (1e-4 if dtype == torch.float32 else 2e-2)
    assert rel_inf(w.grad, wr.grad) <= (1e-4 if dtype == torch.float32 else 2e-2)
    assert rel_inf(b.grad, br.grad) <= (1e-4 if dtype == torch.float32 else 2e-2)
    # second backward accumulates
    ops.ln_bwd(dy, x, mean, rstd, w, b, None)
    assert rel_inf(w.grad, 2 * wr.grad) <= (1e-4 if dtype == torch.float32 else 2e-2)


@pytest.mark.parametrize("dtype,batch,seq,vocab", [(torch.float32, 4, 32, 256), (torch.bfloat16, 2, 64, 50257),
                                                   (torch.float32, 3, 5, 1001), (torch.bfloat16, 2, 2, 7)])
def test_next_token_loss(cuda, dtype, batch, seq, vocab):
    logits = _rand(batch, seq, vocab, dtype=dtype, seed=40, scale=3.0).requires_grad_(True)
    g = torch.Generator().manual_seed(41)
    tokens = torch.randint(0, vocab, (batch, seq), generator=g).to(cuda)
    loss = ops.next_token_loss(logits, tokens, vocab)
    lr = logits.detach().float().requires_grad_(True)
    ref = torch_ref.next_token_loss(lr, tokens, vocab)
    assert abs(float(loss) - float(ref)) <= (1e-5 if dtype == torch.float32 else 1e-3) * max(1.0, abs(float(ref)))
    (loss * 0.5).backward()
    (ref * 0.5).backward()
    assert rel_inf(logits.grad, lr.grad) <= (F32_TOL if dtype == torch.float32 else BF16_TOL)
    assert torch.all(logits.grad[:, -1] == 0)


@pytest.mark.parametrize("batch,seq,vocab,ld", [(2, 64, 50257, 50264), (3, 5, 13, 16), (2, 4, 65536, 65536)])
def test_next_token_loss_padded_bf16_rows(cuda, batch, seq, vocab, ld):
    """bf16 logits whose rows start 16-byte aligned (row stride a multiple of 8, as the LM head lays
    them out): the fused forward keeps each row in registers; vocab not a multiple of 8 exercises
    the tail columns."""
    buf = _rand(batch, seq, ld, dtype=torch.bfloat16, seed=42, scale=3.0)
    logits = buf[..., :vocab].requires_grad_(True)
    g = torch.Generator().manual_seed(43)
    tokens = torch.randint(0, vocab, (batch, seq), generator=g).to(cuda)
    loss = ops.next_token_loss(logits, tokens, vocab)
    lr = logits.detach().float().requires_grad_(True)
    ref = torch_ref.next_token_loss(lr, tokens, vocab)
    assert abs(float(loss) - float(ref)) <= 1e-3 * max(1.0, abs(float(ref)))
    loss.backward()
    ref.backward()
    assert rel_inf(logits.grad, lr.grad) <= BF16_TOL
    assert torch.all(logits.grad[:, -1] == 0)


def test_next_token_loss_of_zero_logits_is_log_vocab(cuda):
    logits = torch.zeros(2, 16, 1000, device=cuda)
    tokens = torch.randint(0, 1000, (2, 16), device=cuda)
    assert abs(float(ops.next_token_loss(logits, tokens, 1000)) - math.log(1000)) < 1e-6


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_embedding_forward_backward_deterministic(cuda, dtype):
    vocab, dim, batch, seq = 50, 64, 4, 33
    W = torch.nn.Parameter(_rand(vocab, dim, dtype=dtype, seed=50))
    P = torch.nn.Parameter(_rand(seq, dim, dtype=dtype, seed=51))
    g = torch.Generator().manual_seed(52)
    tokens = torch.randint(0, 7, (batch, seq), generator=g).to(cuda)  # many duplicates
    out = ops.embedding(tokens, W, P)
    ref = F.embedding(tokens, W.detach().float()) + P.detach().float()[None]
    assert rel_inf(out, ref) <= (0 if dtype == torch.float32 else 4e-3)
    dout = _rand(batch, seq, dim, dtype=dtype, seed=53)
    out.backward(dout)
    gW1, gP1 = W.grad.clone(), P.grad.clone()
    want = torch.zeros(vocab, dim, device=cuda, dtype=torch.float64)
    want.index_add_(0, tokens.reshape(-1), dout.double().reshape(-1, dim))
    assert rel_inf(gW1, want) <= (1e-6 if dtype == torch.float32 else 1e-2)
    assert rel_inf(gP1, dout.double().sum(0)) <= (1e-6 if dtype == torch.float32 else 1e-2)
    W.grad = None
    P.grad = None
    ops.embedding(tokens, W, P).backward(dout)
    assert torch.equal(W.grad, gW1) and torch.equal(P.grad, gP1)  # bit-reproducible


def test_vocab_parallel_embedding_masks_other_ranks(cuda):
    vocab, dim, tp = 40, 16, 4
    full = _rand(vocab, dim, dtype=torch.float32, seed=54)
    tokens = torch.randint(0, vocab, (2, 9), device=cuda)
    total = torch.zeros(2, 9, dim, device=cuda)
    for r in range(tp):
        shard = full[r * 10:(r + 1) * 10].contiguous()
        total += ops.embedding(tokens, shard, None, vocab_start=r * 10, vocab_rows=10)
    assert torch.equal(total, F.embedding(tokens, full))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16, torch.int8])
@pytest.mark.parametrize("shape", [(12, 20), (7, 9), (2048, 512), (3, 1)])
def test_reshard_cat_and_chunk_bit_exact(cuda, dtype, shape):
    g = torch.Generator().manual_seed(60)
    full = (torch.randn(*shape, generator=g) * 100).to(dtype).to(cuda)
    for dim in (0, 1):
        for old, new in ((4, 2), (2, 4), (3, 2), (1, 3)):
            if full.shape[dim] < old:
                continue
            shards = [torch.chunk(full, old, dim)[r].contiguous() for r in range(len(torch.chunk(full, old, dim)))]
            got = reshard.device_cat(shards, dim)
            assert torch.equal(got, torch.cat(shards, dim))
            pieces = torch.chunk(full, new, dim)
            for r in range(len(pieces)):
                assert torch.equal(reshard.local_slice(full, dim, r, new), pieces[r])
                assert torch.equal(reshard.repack_shards(shards, dim, r, new), pieces[r])


def test_reshard_tp4_to_tp2_layer_at_full_size(cuda):
    """A d2048 / FFN 8192 layer's column- and row-parallel bf16 shards, TP4 -> TP2, torch.equal."""
    g = torch.Generator().manual_seed(61)
    mats = {"q": (2048, 2048, 0), "k": (2048, 2048, 0), "v": (2048, 2048, 0), "out": (2048, 2048, 1),
            "fc1": (8192, 2048, 0), "fc2": (2048, 8192, 1)}
    for name, (r, c, dim) in mats.items():
        full = (torch.randn(r, c, generator=g) * 0.02).to(torch.bfloat16).to(cuda)
        old = [t.contiguous() for t in torch.chunk(full, 4, dim)]
        for new_rank in range(2):
            got = reshard.repack_shards(old, dim, new_rank, 2)
            assert torch.equal(got, torch.chunk(full, 2, dim)[new_rank]), name


def test_reshard_repack_many_matches_per_tensor_repack(cuda):
    """One batched launch for a whole layer (plus a 3-D tensor, a replicated one and ragged
    old -> new degrees) equals repack_shards tensor by tensor, bit for bit."""
    g = torch.Generator().manual_seed(62)
    fulls = {"q": ((512, 256), 0), "out": ((256, 512), 1), "ln": ((256,), None), "t3": ((6, 10, 4), 1),
             "odd": ((7, 9), 0)}
    for old_n, new_n in ((4, 2), (3, 2), (2, 3)):
        items, expect = [], []
        for name, (shape, dim) in fulls.items():
            full = (torch.randn(*shape, generator=g) * 10).to(torch.bfloat16).to(cuda)
            if dim is None:
                old = [full.clone()]
            else:
                if full.shape[dim] < old_n:
                    continue
                old = [t.contiguous() for t in torch.chunk(full, old_n, dim)]
            items.append((old, dim))
            expect.append([reshard.repack_shards(old, dim, r, new_n) for r in range(new_n)])
        for r in range(new_n):
            got = reshard.repack_many(items, r, new_n)
            for i, t in enumerate(got):
                assert torch.equal(t, expect[i][r]), (old_n, new_n, r, i)


def test_reshard_unpack_entry_point(cuda):
    src = torch.arange(6 * 10, dtype=torch.int32, device=cuda).view(6, 10)
    outs = [torch.empty(6, e, dtype=torch.int32, device=cuda) for e in (3, 3, 4)]
    ptrs = (ctypes.c_void_p * 3)(*[o.data_ptr() for o in outs])
    ext = (ctypes.c_int64 * 3)(3, 3, 4)
    H.call("rh_reshard_unpack", src.data_ptr(), 6, 10, 1, 4, 3, ptrs, ext, H.stream_of(src))
    for o, want in zip(outs, torch.split(src, [3, 3, 4], 1)):
        assert torch.equal(o, want)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_optimizer_steps(cuda, dtype):
    from resihp.optim import SGD, AdamW

    p0 = _rand(1000, dtype=torch.float32, seed=70)
    grads = [_rand(1000, dtype=torch.float32, seed=71 + i) for i in range(3)]
    ours = torch.nn.Parameter(p0.clone().to(dtype))
    ref = torch.nn.Parameter(p0.clone().to(dtype).float())
    opt = AdamW([ours], lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
    ref_opt = torch.optim.AdamW([ref], lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
    for gr in grads:
        ours.grad = gr.to(dtype)
        ref.grad = gr.to(dtype).float()
        opt.step()
        ref_opt.step()
    assert rel_inf(ours, ref) <= (1e-6 if dtype == torch.float32 else 4e-3)
    assert float(opt.state[ours]["step"]) == 3.0
    s = torch.nn.Parameter(p0.clone().to(dtype))
    s.grad = grads[0].to(dtype)
    SGD([s], lr=1e-3).step()
    assert rel_inf(s, p0.to(dtype).float() - 1e-3 * grads[0].to(dtype).float()) <= (1e-7 if dtype == torch.float32 else 4e-3)


def test_gemm_unaligned_views(cuda, gemm_tile):
    """Operands and outputs that are column-offset views (rows not 16-byte aligned)."""
    M, N, K = 300, 260, 200
    Abuf = _rand(M, K + 3, seed=80)
    Bbuf = _rand(N, K + 3, seed=81, scale=0.1)
    Cbuf = _rand(M, N + 5, seed=82)
    Dbuf = torch.zeros(M, N + 5, dtype=torch.bfloat16, device=cuda)
    Ubuf = torch.zeros(M, N + 5, dtype=torch.bfloat16, device=cuda)
    A, B, C, D, U = Abuf[:, 1:K + 1], Bbuf[:, 3:K + 3], Cbuf[:, 1:N + 1], Dbuf[:, 1:N + 1], Ubuf[:, 5:N + 5]
    ops.gemm(H.RH_GEMM_NT, M, N, K, A, A.stride(0), [B], B.stride(0), [D], D.stride(0), beta=1.0, C=C,
             ldc=C.stride(0), epilogue=H.RH_EPI_GELU, aux_out=U, ldaux=U.stride(0))
    pre = A.float() @ B.float().t() + C.float()
    assert rel_inf(U, pre) <= BF16_TOL
    assert rel_inf(D, F.gelu(pre)) <= BF16_TOL
    assert torch.all(Dbuf[:, 0] == 0) and torch.all(Ubuf[:, :5] == 0)  # nothing written outside the views


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_adamw_multi_tensor_matches_torch(cuda, dtype):
    """adamw(params).step() over every parameter of the tiny LM (2 layers, d 64, vocab 256, seq 32;
    25 tensors) plus 110 extra tensors of ragged sizes (one empty), so the update spans several
    64-tensor launches: 3 steps against torch.optim.AdamW with the reference's constants, fp32
    within 1e-6 (params and both moments); bf16 against the same fp32 update, within the three
    roundings of the stored bf16 values (each at most half an ulp, 2^-8 of the value at the bottom
    of a binade); device step counts equal 3."""
    from resihp.config import TrainConfig
    from resihp.model import ReferenceTransformer
    from resihp.reference import adamw

    cfg = TrainConfig(model_dim=64, num_layers=2, num_heads=4, batch_size=4, micro_batch_size=4, seed=1234, tp=1,
                      pp=1, dp=1, iterations=1)
    torch.manual_seed(1234)
    model = ReferenceTransformer(cfg, vocab_size=256, sequence_length=32)
    params = [torch.nn.Parameter(p.detach().clone()) for p in model.parameters()]
    g = torch.Generator().manual_seed(90)
    params += [torch.nn.Parameter(torch.randn(n, generator=g) * 0.1) for n in list(range(0, 100)) + [1000 + 37 * i for i in range(10)]]
    ours = [torch.nn.Parameter(p.detach().to(cuda, dtype)) for p in params]
    ref = [torch.nn.Parameter(p.detach().to(cuda, dtype).float()) for p in params]
    opt = adamw(ours)
    ref_opt = torch_ref.adamw(ref)
    for step in range(3):
        for a, b in zip(ours, ref):
            gr = torch.randn(a.shape, generator=g).to(cuda)
            a.grad = gr.to(dtype)
            b.grad = gr.to(dtype).float()
        opt.step()
        ref_opt.step()
    tol = 1e-6 if dtype == torch.float32 else 3 * 2.0 ** -8
    for i, (a, b) in enumerate(zip(ours, ref)):
        if a.numel() == 0:
            continue
        sa, sb = opt.state[a], ref_opt.state[b]
        assert float(sa["step"]) == 3.0
        assert rel_inf(a, b) <= tol, (i, "param", rel_inf(a, b))
        assert rel_inf(sa["exp_avg"], sb["exp_avg"]) <= tol, (i, "exp_avg")
        assert rel_inf(sa["exp_avg_sq"], sb["exp_avg_sq"]) <= 2 * tol, (i, "exp_avg_sq")


def test_adamw_multi_rejects_shared_step_counters(cuda):
    p = torch.zeros(8, device=cuda)
    step = torch.zeros((), device=cuda)
    e = H.rh_adamw_tensor(p.data_ptr(), p.data_ptr(), p.data_ptr(), p.data_ptr(), step.data_ptr(), 8)
    arr = (H.rh_adamw_tensor * 2)(e, e)
    with pytest.raises(ValueError, match="share a step counter"):
        H.call("rh_adamw_multi", H.RH_DTYPE_F32, 2, arr, 1e-3, 0.9, 0.999, 1e-8, 0.01, None)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("batch,seq,vocab,repeat", [
    (32, 1024, 50257, 0.7),   # 32768 tokens, 70 % of them one id: a 23k-row segment
    (16, 1024, 50257, 0.0),   # GPT-2-small vocabulary, uniform ids
    (3, 4097, 40, 0.5),       # ragged token count, few ids: every chunk boundary inside a segment
    (1, 20000, 1, 0.0),       # a single id for every token
])
def test_embedding_backward_any_token_count(cuda, dtype, batch, seq, vocab, repeat):
    """Token-embedding gradient beyond one workgroup's sort: 32768 tokens with one id repeated
    ~23k times, ragged counts, a one-row vocabulary -- against an fp64 index_add, and bit-identical
    on a second run."""
    dim = 64 if dtype == torch.bfloat16 else 48
    g = torch.Generator().manual_seed(55)
    tokens = torch.randint(0, vocab, (batch, seq), generator=g)
    tokens[torch.rand(batch, seq, generator=g) < repeat] = vocab // 2
    tokens = tokens.to(cuda)
    W = torch.nn.Parameter(torch.zeros(vocab, dim, device=cuda, dtype=dtype))
    dout = _rand(batch, seq, dim, dtype=dtype, seed=56)
    out = ops.embedding(tokens, W)
    out.backward(dout)
    first = W.grad.clone()
    want = torch.zeros(vocab, dim, device=cuda, dtype=torch.float64)
    want.index_add_(0, tokens.reshape(-1), dout.double().reshape(-1, dim))
    assert rel_inf(first, want) <= (1e-6 if dtype == torch.float32 else 4e-3)
    W.grad = None
    ops.embedding(tokens, W).backward(dout)
    assert torch.equal(W.grad, first)


def _wgrad_desc(dy, x, D, beta, d_seg=0):
    """TN descriptor of D (+)= dy^T . x (D a list of row segments)."""
    return ops._gemm_desc(H.RH_GEMM_TN, dy.shape[1], x.shape[1], dy.shape[0], dy, dy.stride(0), [x], x.stride(0), D,
                          x.shape[1], beta=beta, d_seg_rows=d_seg)


@pytest.mark.parametrize("shapes,want_splits", [
    # one TP=4 rank of the 1.3B block: fc2, fc1, out_proj, q|k|v (K = 8192 tokens)
    ([(2048, 2048), (2048, 2048), (2048, 512), (1536, 2048)], None),
    # GPT-2-small's block (d 768, FFN 3072): too few tiles alone, so K is split
    ([(768, 3072), (3072, 768), (768, 768), (2304, 768)], 2),
    ([(256, 512)], None),
])
@pytest.mark.parametrize("waves", ["4", "8"])
def test_gemm_grouped_weight_gradients(cuda, shapes, want_splits, waves, monkeypatch):
    """rh_gemm_grouped over a block's weight gradients (dW = dy^T x, K = tokens): every problem
    equals its fp32 product within bf16 rounding, accumulates into existing gradients (beta 1), writes
    three q|k|v row segments, and agrees with separate rh_gemm calls; the plan uses the expected
    split count.  Both 256x256 kernels (4 and 8 waves) are run."""
    monkeypatch.setenv("RESIHP_GEMM_WAVES", waves)
    T = 8192
    descs, outs, refs, keep = [], [], [], []
    for i, (m, n) in enumerate(shapes):
        dy = _rand(T, m, seed=100 + i, scale=0.1)
        x = _rand(T, n, seed=200 + i)
        prev = _rand(m, n, seed=300 + i)
        ref = dy.float().t() @ x.float() + prev.float()
        if i == 3:  # q|k|v: three row segments of m/3
            segs = [prev[j * m // 3:(j + 1) * m // 3].clone() for j in range(3)]
            descs.append(_wgrad_desc(dy, x, segs, 1.0, d_seg=m // 3))
            outs.append(segs)
        else:
            D = prev.clone()
            descs.append(_wgrad_desc(dy, x, [D], 1.0))
            outs.append([D])
        refs.append(ref)
        keep += [dy, x]
    arr = (H.rh_gemm_desc * len(descs))(*descs)
    splits = ctypes.c_int(-1)
    H.call("rh_gemm_grouped_plan", arr, len(descs), ctypes.byref(splits))
    assert splits.value >= 1  # one launch for the whole group
    if want_splits is not None:
        assert splits.value == want_splits
    nbytes = H.query("rh_gemm_grouped_workspace_bytes", arr, len(descs))
    ws = H.workspace(nbytes, torch.device(cuda))
    H.call("rh_gemm_grouped", arr, len(descs), H.ptr(ws), nbytes, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    for i, (o, ref) in enumerate(zip(outs, refs)):
        got = torch.cat(o, 0)
        assert rel_inf(got, ref) <= BF16_TOL, (i, rel_inf(got, ref))
    # separate calls on the same inputs agree to within the bf16 rounding of two summation orders
    for i, (m, n) in enumerate(shapes):
        dy, x = keep[2 * i], keep[2 * i + 1]
        D = torch.zeros(m, n, dtype=torch.bfloat16, device=cuda)
        ops.gemm(H.RH_GEMM_TN, m, n, T, dy, m, [x], n, [D], n)
        assert rel_inf(torch.cat(outs[i], 0).float() - (refs[i] - dy.float().t() @ x.float()), D) <= BF16_TOL


def test_gemm_grouped_falls_back_for_mixed_groups(cuda):
    """A group the single launch cannot take (an fp32 problem, a ragged K) runs as consecutive
    rh_gemm calls with the same results."""
    a32, b32 = _rand(100, 48, dtype=torch.float32, seed=1), _rand(100, 40, dtype=torch.float32, seed=2)
    D32 = torch.zeros(48, 40, device=cuda)
    abf, bbf = _rand(96, 64, seed=3), _rand(96, 128, seed=4)
    Dbf = torch.zeros(64, 128, dtype=torch.bfloat16, device=cuda)
    for descs, outs in (([_wgrad_desc(a32, b32, [D32], 0.0)], [(D32, a32, b32)]),
                        ([_wgrad_desc(abf, bbf, [Dbf], 0.0)], [(Dbf, abf, bbf)])):
        arr = (H.rh_gemm_desc * len(descs))(*descs)
        splits = ctypes.c_int(-1)
        H.call("rh_gemm_grouped_plan", arr, len(descs), ctypes.byref(splits))
        assert splits.value == 0
        nbytes = H.query("rh_gemm_grouped_workspace_bytes", arr, len(descs))
        ws = H.workspace(nbytes, torch.device(cuda))
        H.call("rh_gemm_grouped", arr, len(descs), H.ptr(ws), nbytes, None)
        torch.cuda.synchronize()
        for D, a, b in outs:
            tol = F32_TOL if D.dtype == torch.float32 else BF16_TOL
            assert rel_inf(D, a.float().t() @ b.float()) <= tol
