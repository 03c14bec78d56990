"""Write the golden vectors of the reference's seeded training step.

Run in the build container only (it imports the reference from /root/reference,
which never travels to the GPU box):

    python tests/golden/make_golden.py

What it pins that no closed form does: the seeded initial weights of
``ReferenceTransformer`` (they depend on module construction order and on how
torch's initialisers consume the RNG, resihp/model.py:100-116) and everything
downstream of them -- the loss, the gradients and the sha256 step records of
``ReferenceRun`` (resihp/reference.py:106-150).

Outputs (data only):
  cfg1_step.npz    tiny decoder LM (2 layers, d 64, 4 heads, vocab 256, seq 32,
                   batch 4, seed 1234): tokens, per-parameter init sha256,
                   fp32 logits, loss, every gradient, post-AdamW digests
  ref_records.json the reference test suite's config (d 16, 4 layers, 4 heads,
                   vocab 32, seq 8, batch 4, seed 1234, 3 iterations):
                   StepRecord loss / param_digest / optim_digest per step
"""

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

REF = Path("/root/reference")
OUT = Path(__file__).resolve().parent


def _sha(t) -> str:
    return hashlib.sha256(t.detach().cpu().float().contiguous().numpy().tobytes()).hexdigest()


def main() -> None:
    sys.path.insert(0, str(REF))
    import torch
    from torch.nn import functional as F

    from resihp.config import TrainConfig
    from resihp.model import ReferenceTransformer
    from resihp.reference import ReferenceRun, _token_stream, run_reference

    torch.set_num_threads(1)

    # --- tiny decoder LM, one fwd+bwd+AdamW step -------------------------------------
    cfg = TrainConfig(model_dim=64, num_layers=2, num_heads=4, batch_size=4, micro_batch_size=4, seed=1234,
                      tp=1, pp=1, dp=1, iterations=1)
    vocab, seq = 256, 32
    run = ReferenceRun(cfg, vocab_size=vocab, sequence_length=seq)
    init = {name: _sha(p) for name, p in run.model.named_parameters()}
    tokens = run.batches[0]
    logits = run.model(tokens)
    loss = F.cross_entropy(logits[:, :-1].reshape(-1, vocab), tokens[:, 1:].reshape(-1))
    run.model.zero_grad()
    loss.backward()
    grads = {name: p.grad.detach().clone() for name, p in run.model.named_parameters()}
    # a fresh run for the StepRecord (same seed -> same init, batch and update)
    record = ReferenceRun(cfg, vocab_size=vocab, sequence_length=seq).step()
    arrays = {
        "tokens": tokens.numpy().astype(np.int64),
        "logits": logits.detach().numpy().astype(np.float32),
        "loss": np.array(float(loss.detach()), dtype=np.float64),
    }
    for name, g in grads.items():
        arrays["grad/" + name] = g.numpy().astype(np.float32)
    meta = {
        "config": dict(model_dim=64, num_layers=2, num_heads=4, batch_size=4, seed=1234, vocab=vocab, seq=seq),
        "init_sha256": init,
        "step_record": {"loss": record.loss, "param_digest": record.param_digest,
                        "optim_digest": record.optim_digest},
        "torch": torch.__version__,
    }
    np.savez_compressed(OUT / "cfg1_step.npz", meta=np.array(json.dumps(meta)), **arrays)

    # --- the reference suite's own config: 3 AdamW iterations ---------------------------
    small = TrainConfig(model_dim=16, num_layers=4, num_heads=4, batch_size=4, micro_batch_size=2, seed=1234,
                        tp=2, pp=2, dp=2, iterations=3)
    records = run_reference(small, vocab_size=32, sequence_length=8)
    model = ReferenceTransformer(small, vocab_size=32, sequence_length=8)  # unseeded: names/shapes only
    out = {
        "config": dict(model_dim=16, num_layers=4, num_heads=4, batch_size=4, seed=1234, vocab=32, seq=8,
                       iterations=3),
        "tokens": [[list(row) for row in r.tokens] for r in records],
        "records": [{"loss": r.loss, "param_digest": r.param_digest, "optim_digest": r.optim_digest}
                    for r in records],
        "param_shapes": {n: list(p.shape) for n, p in model.named_parameters()},
        "token_stream_check": [t.tolist() for t in _token_stream(32, 8, 4, 2, 1234)],
        "torch": torch.__version__,
    }
    (OUT / "ref_records.json").write_text(json.dumps(out, indent=1))
    print("wrote", OUT / "cfg1_step.npz", "and", OUT / "ref_records.json")


if __name__ == "__main__":
    main()
