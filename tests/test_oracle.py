"""Pins the CPU oracle (CPU only).

* golden vectors written from the reference itself: seeded init, logits, loss,
  every gradient, the post-AdamW step records;
* the independent fp64 numpy restatement, and central finite differences on it;
* closed forms that a dropped term, wrong sign or transposed operand would break.
"""

import hashlib
import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch
from torch.nn import functional as F

from oracle import numpy_ref, torch_ref

GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(autouse=True)
def _one_thread():
    """The golden vectors were written single-threaded; CPU reductions then match bit for bit."""
    before = torch.get_num_threads()
    torch.set_num_threads(1)
    yield
    torch.set_num_threads(before)


@pytest.fixture(scope="module")
def cfg1():
    data = np.load(GOLDEN / "cfg1_step.npz", allow_pickle=False)
    meta = json.loads(str(data["meta"]))
    return data, meta


def _sha(t):
    return hashlib.sha256(t.detach().float().contiguous().numpy().tobytes()).hexdigest()


def _cfg1_state(meta):
    c = meta["config"]
    return torch_ref.seeded_state(c["model_dim"], c["num_layers"], c["num_heads"], c["vocab"], c["seq"], c["seed"])


def test_seeded_init_matches_reference(cfg1):
    _, meta = cfg1
    state = _cfg1_state(meta)
    assert set(state) == set(meta["init_sha256"])
    for name, t in state.items():
        assert _sha(t) == meta["init_sha256"][name], name


def test_forward_loss_and_grads_match_reference(cfg1):
    data, meta = cfg1
    c = meta["config"]
    state = _cfg1_state(meta)
    tokens = torch.from_numpy(data["tokens"])
    logits, loss, grads = torch_ref.loss_and_grads(state, tokens, c["num_heads"], range(c["num_layers"]), c["vocab"])
    assert torch.equal(logits, torch.from_numpy(data["logits"]))
    assert float(loss) == float(data["loss"])
    for name, g in grads.items():
        ref = torch.from_numpy(data["grad/" + name])
        assert torch.equal(g, ref), name


def test_token_stream_matches_reference():
    rec = json.loads((GOLDEN / "ref_records.json").read_text())
    gen = torch.Generator().manual_seed(1234)
    got = [torch.randint(0, 32, (4, 8), generator=gen).tolist() for _ in range(2)]
    assert got == rec["token_stream_check"]


def _digest(items):
    h = hashlib.sha256()
    for name, t in items:
        a = t.detach().cpu().to(torch.float32).contiguous().numpy()
        h.update(name.encode())
        h.update(repr(a.shape).encode())
        h.update(a.tobytes())
    return h.hexdigest()


def test_adamw_step_records_match_reference():
    """Three AdamW iterations of the reference suite's config, digest for digest."""
    rec = json.loads((GOLDEN / "ref_records.json").read_text())
    c = rec["config"]
    torch.manual_seed(c["seed"])
    model = torch_ref.Model(c["model_dim"], c["num_layers"], c["num_heads"], c["vocab"], c["seq"])
    opt = torch_ref.adamw(model.parameters())
    names = {p: n for n, p in model.named_parameters()}
    gen = torch.Generator().manual_seed(c["seed"])
    batches = [torch.randint(0, c["vocab"], (c["batch_size"], c["seq"]), generator=gen) for _ in range(c["iterations"])]
    for step, want in enumerate(rec["records"]):
        tokens = batches[step]
        assert tokens.tolist() == rec["tokens"][step]
        logits = torch_ref.model_forward(model.state(), tokens, c["num_heads"], range(c["num_layers"]))
        loss = torch_ref.next_token_loss(logits, tokens, c["vocab"])
        opt.zero_grad()
        loss.backward()
        opt.step()
        assert float(loss) == want["loss"]
        assert _digest(sorted(model.state().items())) == want["param_digest"]
        items = []
        for p, st in opt.state.items():
            for key in ("exp_avg", "exp_avg_sq", "step"):
                v = st[key]
                items.append((f"{names[p]}.{key}", v if torch.is_tensor(v) else torch.tensor(v)))
        assert _digest(sorted(items)) == want["optim_digest"]


def test_numpy_restatement_agrees_with_torch_fp64(cfg1):
    data, meta = cfg1
    c = meta["config"]
    state = _cfg1_state(meta)
    tokens = torch.from_numpy(data["tokens"])
    logits_t, loss_t, grads_t = torch_ref.loss_and_grads(state, tokens, c["num_heads"], range(c["num_layers"]),
                                                         c["vocab"], dtype=torch.float64)
    np_state = {k: v.double().numpy() for k, v in state.items()}
    logits_n, loss_n, grads_n = numpy_ref.model_loss_and_grads(np_state, tokens.numpy(), c["num_heads"],
                                                               range(c["num_layers"]))
    assert abs(float(loss_t) - loss_n) < 1e-12
    assert np.abs(logits_t.numpy() - logits_n).max() < 1e-11
    for name in state:
        g_t = grads_t[name].numpy()
        g_n = np.asarray(grads_n[name])
        assert np.abs(g_t - g_n).max() <= 1e-10 * max(np.abs(g_t).max(), 1e-30), name


def _tiny_state(seed=3, d=8, layers=1, heads=2, vocab=11, seq=5):
    g = torch.Generator().manual_seed(seed)
    st = torch_ref.synthetic_state(d, layers, vocab, seq, std=0.5, seed=seed, dtype=torch.float64)
    for k in st:  # non-trivial LayerNorm affine so gamma/beta enter every path
        if k.endswith("norm.weight"):
            st[k] = 1.0 + 0.3 * torch.randn(st[k].shape, generator=g, dtype=torch.float64)
        elif k.endswith("norm.bias"):
            st[k] = 0.3 * torch.randn(st[k].shape, generator=g, dtype=torch.float64)
    tokens = torch.randint(0, vocab, (2, seq), generator=g)
    tokens[0, 1] = tokens[1, 3]  # a duplicated id exercises the embedding scatter-add
    return {k: v.numpy() for k, v in st.items()}, tokens.numpy(), heads, range(layers)


def test_numpy_backward_matches_finite_differences():
    state, tokens, heads, layers = _tiny_state()
    _, _, grads = numpy_ref.model_loss_and_grads(state, tokens, heads, layers)
    rng = np.random.default_rng(0)
    h = 1e-6
    for name, w in state.items():
        flat = w.reshape(-1)
        for idx in rng.choice(flat.size, size=min(4, flat.size), replace=False):
            old = flat[idx]
            flat[idx] = old + h
            lp = numpy_ref.model_loss(state, tokens, heads, layers)
            flat[idx] = old - h
            lm = numpy_ref.model_loss(state, tokens, heads, layers)
            flat[idx] = old
            fd = (lp - lm) / (2 * h)
            an = np.asarray(grads[name]).reshape(-1)[idx]
            assert abs(fd - an) <= 1e-6 * max(1.0, abs(fd)), (name, idx, fd, an)


def test_zero_lm_head_gives_log_vocab():
    state, tokens, heads, layers = _tiny_state()
    state["lm_head.weight"] = np.zeros_like(state["lm_head.weight"])
    _, loss, grads = numpy_ref.model_loss_and_grads(state, tokens, heads, layers)
    assert abs(loss - math.log(11)) < 1e-14
    t = {k: torch.from_numpy(v) for k, v in state.items()}
    logits = torch_ref.model_forward(t, torch.from_numpy(tokens), heads, layers)
    assert abs(float(torch_ref.next_token_loss(logits, torch.from_numpy(tokens), 11)) - math.log(11)) < 1e-14


def test_cross_entropy_gradient_rows_sum_to_zero_and_last_position_is_zero():
    rng = np.random.default_rng(1)
    logits = rng.standard_normal((3, 7, 13))
    tokens = rng.integers(0, 13, (3, 7))
    loss, dl = numpy_ref.xent(logits, tokens)
    assert np.abs(dl.sum(-1)).max() < 1e-15
    assert np.all(dl[:, -1] == 0)
    ref = F.cross_entropy(torch.from_numpy(logits[:, :-1]).reshape(-1, 13), torch.from_numpy(tokens[:, 1:]).reshape(-1))
    assert abs(float(ref) - loss) < 1e-14


def test_attention_closed_forms():
    rng = np.random.default_rng(2)
    q, k, v = (rng.standard_normal((2, 3, 9, 4)) for _ in range(3))
    o, p = numpy_ref.attn_fwd(q, k, v)
    assert np.abs(p.sum(-1) - 1).max() < 1e-14
    assert np.abs(o[:, :, 0] - v[:, :, 0]).max() < 1e-14  # the first query sees only key 0
    assert np.all(np.triu(p[0, 0], 1) == 0)  # no weight on future keys
    # brute force: row i is softmax over keys <= i
    i = 5
    s = q[1, 2, i] @ k[1, 2, : i + 1].T / 2.0
    w = np.exp(s - s.max())
    w /= w.sum()
    assert np.abs(w @ v[1, 2, : i + 1] - o[1, 2, i]).max() < 1e-14


def test_layernorm_and_gelu_closed_forms():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((6, 10)) * 3 + 1
    y, _ = numpy_ref.ln_fwd(x, np.ones(10), np.zeros(10))
    assert np.abs(y.mean(-1)).max() < 1e-14
    assert np.abs(y.var(-1) - 1 / (1 + 1e-5 / x.var(-1))).max() < 1e-12
    u = np.linspace(-6, 6, 101)
    ref = np.array([0.5 * t * (1 + math.erf(t / math.sqrt(2))) for t in u])
    assert np.abs(numpy_ref.gelu(u) - ref).max() < 1e-15
    fd = (numpy_ref.gelu(u + 1e-6) - numpy_ref.gelu(u - 1e-6)) / 2e-6
    assert np.abs(numpy_ref.gelu_grad(u) - fd).max() < 1e-8


def test_shard_sublayers_sum_to_the_full_sublayer():
    """Row-parallel partials over every rank add up to the unsharded output (what g would reduce)."""
    d, heads, tp = 16, 4, 4
    full = torch_ref.synthetic_state(d, 1, 32, 6, std=0.3, seed=5, dtype=torch.float64)
    x = torch.randn(2, 6, d, dtype=torch.float64, generator=torch.Generator().manual_seed(9))
    pre = "layers.0."
    want_attn = torch_ref.attention(x, *(full[pre + f"attn.{n}.weight"] for n in ("q_proj", "k_proj", "v_proj", "out_proj")), heads)
    want_mlp = torch_ref.mlp(x, full[pre + "mlp.fc1.weight"], full[pre + "mlp.fc2.weight"])
    got_attn = torch.zeros_like(want_attn)
    got_mlp = torch.zeros_like(want_mlp)
    for r in range(tp):
        sh = torch_ref.synthetic_state(d, 1, 32, 6, std=0.3, seed=5, dtype=torch.float64, tp_size=tp, tp_rank=r)
        got_attn += torch_ref.attention(x, *(sh[pre + f"attn.{n}.weight"] for n in ("q_proj", "k_proj", "v_proj", "out_proj")), heads // tp)
        got_mlp += torch_ref.mlp(x, sh[pre + "mlp.fc1.weight"], sh[pre + "mlp.fc2.weight"])
    assert (got_attn - want_attn).abs().max() < 1e-12
    assert (got_mlp - want_mlp).abs().max() < 1e-12


def test_tp1_shard_is_the_full_model():
    st = torch_ref.synthetic_state(16, 2, 32, 8, std=0.3, seed=4)
    tokens = torch.randint(0, 32, (2, 8), generator=torch.Generator().manual_seed(1))
    full = torch_ref.model_forward(st, tokens, 4, range(2))
    shard = torch_ref.shard_forward(st, num_heads=4, tp_rank=0, tp_size=1, vocab_size=32, layer_ids=range(2),
                                    is_first=True, is_last=True, tokens=tokens)
    assert torch.equal(full, shard)


def test_vocab_parallel_embedding_partials_sum_to_full():
    st = torch_ref.synthetic_state(8, 0, 12, 5, std=1.0, seed=2)
    tokens = torch.randint(0, 12, (3, 5), generator=torch.Generator().manual_seed(2))
    pos = F.embedding(torch.arange(5), st["position_embedding.weight"])
    want = F.embedding(tokens, st["token_embedding.weight"])
    got = torch.zeros_like(want)
    for r in range(3):
        sh = torch_ref.synthetic_state(8, 0, 12, 5, std=1.0, seed=2, tp_size=3, tp_rank=r)
        got += torch_ref.shard_forward(sh, num_heads=1, tp_rank=r, tp_size=3, vocab_size=12, layer_ids=[],
                                       is_first=True, is_last=False, tokens=tokens) - pos
    assert torch.allclose(got, want, atol=1e-6)


def test_reshard_round_trips():
    w = torch.randn(12, 20)
    for dim in (0, 1):
        for old, new in ((4, 2), (2, 4), (4, 1), (3, 2)):
            shards = [torch_ref.local_slice(w, dim, r, old) for r in range(old)]
            full = torch_ref.cat(shards, dim)
            assert torch.equal(full, w)
            again = [torch_ref.local_slice(full, dim, r, new) for r in range(new)]
            assert torch.equal(torch_ref.cat(again, dim), w)


def test_schedule_literals_of_the_reference_tests():
    # tests/test_parallel_pp.py:71-74 (2 stages, 4 micro-batches)
    assert torch_ref.issue_order(4, 0, 2) == ["F0", "F1", "B0", "F2", "B1", "F3", "B2", "B3"]
    assert torch_ref.issue_order(4, 1, 2) == ["F0", "B0", "F1", "B1", "F2", "B2", "F3", "B3"]
    # the cfg4 stage: index 1 of 4, 8 micro-batches
    assert " ".join(torch_ref.issue_order(8, 1, 4)) == "F0 F1 F2 B0 F3 B1 F4 B2 F5 B3 F6 B4 F7 B5 B6 B7"
