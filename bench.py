"""Throughput of the decoder-LM forward+backward hot path on one MI355X.

Default workload: one TP=4 rank's shard of a GPT-1.3B-shape block (d_model 2048,
4 of 16 heads local with head_dim 128, column-parallel QKV 2048->1536 and FC1
2048->2048, row-parallel out-proj 512->2048 and FC2 2048->2048 emitting partial
sums), seq 2048, micro-batch 4, bf16 with fp32 accumulation; input activations
N(0,1), upstream gradients N(0, 1e-2), weights N(0, 0.02).  A step is one
forward + backward of that shard with fresh parameter gradients.

    python bench.py [--steps K] [--warmup W] [--workload NAME] [--no-graph]

Prints ONE JSON line.  `value` is tokens/s of the whole job (one GPU).  The
timed region replays a HIP graph of the step (captured after the warm-up and
checked bit-for-bit against an eager step) unless --no-graph is given.  The
roofline object is measured in a separate eager pass with HIP events around
each launch of the dominant kernel.  The CPU baseline is the oracle's torch-CPU
restatement of the same step, timed on a bounded sample on this host.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT / "resihp-reproduction_amd"), str(ROOT)):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "train tokens/sec/GPU (fwd+bwd) per shard; MFMA util % and HBM GB/s"
PEAK_BF16 = 2.5e15  # MI355X dense bf16 MFMA FLOP/s
PEAK_HBM = 8.0e12  # bytes/s


def _log(msg):
    print(msg, file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------
# workloads
# ---------------------------------------------------------------------------
class Workload:
    name = ""
    tokens = 0
    flops = 0.0
    config: dict = {}

    def setup(self, dev):
        raise NotImplementedError

    def step(self):
        raise NotImplementedError

    def outputs(self):
        """Tensors whose values identify a step's result (for the graph-vs-eager check)."""
        raise NotImplementedError

    def zero_grads(self):
        for p in self.params():
            p.grad = None

    def extra(self, dev) -> dict:
        """Additional measured legs of this workload, merged into the JSON line."""
        return {}

    def release(self):
        """Drop the last step's outputs, and with them its autograd graph."""
        self.out = None
        self.loss = None

    def params(self):
        return []

    def cpu_sample(self, budget_s: float) -> dict:
        raise NotImplementedError


def _block_fwd_flops(tokens, d, dl, ff, batch, heads_local, head_dim, seq):
    gemm = 2.0 * tokens * (d * 3 * dl + dl * d + d * ff + ff * d)
    attn = 4.0 * batch * heads_local * head_dim * seq * (seq + 1) / 2
    return gemm, attn


class ShardBlock(Workload):
    """One TP rank's shard of one decoder block (middle pipeline stage)."""

    def __init__(self, name, d=2048, heads=16, tp=4, rank=2, seq=2048, batch=4, layers=1):
        self.name, self.d, self.heads, self.tp, self.rank = name, d, heads, tp, rank
        self.seq, self.batch, self.layers = seq, batch, layers
        self.tokens = seq * batch
        dl, ff = d // tp, 4 * d // tp
        g, a = _block_fwd_flops(self.tokens, d, dl, ff, batch, heads // tp, d // heads, seq)
        self.gemm_flops_fwd, self.attn_flops_fwd = g * layers, a * layers
        self.flops = 3.0 * (self.gemm_flops_fwd + self.attn_flops_fwd)
        self.config = {"workload": name, "d_model": d, "heads_total": heads, "heads_local": heads // tp,
                       "head_dim": d // heads, "tp_size": tp, "tp_rank": rank, "seq_len": seq, "micro_batch": batch,
                       "layers": layers, "tokens_per_step": self.tokens,
                       "gemms": {"qkv": [self.tokens, 3 * dl, d], "out": [self.tokens, d, dl],
                                 "fc1": [self.tokens, ff, d], "fc2": [self.tokens, d, ff]},
                       "parallelism": f"one TP={tp} rank on 1 GPU, no collectives (row-parallel partial sums)"}

    def _state(self):
        """This rank's shard of seeded synthetic block weights: matrices N(0, 0.02) drawn from one
        torch.Generator(seed 0) in parameter order, LayerNorm gamma = 1 / beta = 0, cut along the
        reference's shard dims (q/k/v/fc1 rows, out/fc2 columns), bf16."""
        import torch

        from resihp.parallel.reshard import shard_dims

        g = torch.Generator().manual_seed(0)
        d, f = self.d, 4 * self.d
        full = {}
        for gid in range(self.layers):
            p = f"layers.{gid}."
            full[p + "attn_norm.weight"] = torch.ones(d)
            full[p + "attn_norm.bias"] = torch.zeros(d)
            for n in ("q_proj", "k_proj", "v_proj", "out_proj"):
                full[p + f"attn.{n}.weight"] = torch.randn(d, d, generator=g) * 0.02
            full[p + "mlp_norm.weight"] = torch.ones(d)
            full[p + "mlp_norm.bias"] = torch.zeros(d)
            full[p + "mlp.fc1.weight"] = torch.randn(f, d, generator=g) * 0.02
            full[p + "mlp.fc2.weight"] = torch.randn(d, f, generator=g) * 0.02
        layout = shard_dims(range(self.layers))
        out = {}
        for k, v in full.items():
            dim = layout[k]
            if dim is not None and self.tp > 1:
                v = torch.chunk(v, self.tp, dim)[self.rank].contiguous()
            out[k] = v.to(torch.bfloat16)
        return out

    def setup(self, dev):
        import torch

        from resihp.config import TrainConfig
        from resihp.parallel.tp import TensorParallelStage

        cfg = TrainConfig(model_dim=self.d, num_layers=self.layers, num_heads=self.heads, batch_size=self.batch,
                          micro_batch_size=self.batch, seed=0, tp=self.tp, pp=1, dp=1, iterations=1)
        local = {k: v.to(dev) for k, v in self._state().items()}
        self.stage = TensorParallelStage(cfg, vocab_size=8 * self.tp, sequence_length=self.seq,
                                         layer_ids=range(self.layers), is_first=False, is_last=False,
                                         local_state=local, tp_rank=self.rank, tp_size=self.tp)
        g = torch.Generator().manual_seed(1)
        self.x = torch.randn(self.batch, self.seq, self.d, generator=g).to(dev, torch.bfloat16).requires_grad_(True)
        self.dy = (torch.randn(self.batch, self.seq, self.d, generator=g) * 1e-2).to(dev, torch.bfloat16)

    def params(self):
        return list(self.stage.parameters()) + [self.x]

    def step(self):
        self.out = self.stage(hidden=self.x)
        self.out.backward(self.dy)

    def outputs(self):
        return [self.out] + [p.grad for p in self.params()]

    def cpu_sample(self, budget_s):
        import torch

        from oracle import torch_ref

        st = {k: v.float().requires_grad_(True) for k, v in self._state().items()}
        g = torch.Generator().manual_seed(1)
        mb = self.batch
        x = torch.randn(mb, self.seq, self.d, generator=g).requires_grad_(True)
        dy = torch.randn(mb, self.seq, self.d, generator=g) * 1e-2

        def one():
            out = torch_ref.shard_forward(st, num_heads=self.heads, tp_rank=self.rank, tp_size=self.tp,
                                          vocab_size=8 * self.tp, layer_ids=range(self.layers), is_first=False,
                                          is_last=False, hidden=x)
            out.backward(dy)

        sec = _median_time(one, budget_s)
        return {"tokens": mb * self.seq, "seconds": sec,
                "sample": f"fwd+bwd of the same shard at micro-batch {mb} (seq {self.seq}, {self.layers} layer(s)), "
                          f"fp32, oracle torch-CPU restatement; median of 3 after 1 warm-up"}


class GPT2Small(Workload):
    """The full GPT-2-small-shape LM: 12 layers, d 768, 12 heads, FFN 3072, vocab 50257, seq 1024, batch 8."""

    def __init__(self, name="gpt2_small_lm", layers=12, d=768, heads=12, vocab=50257, seq=1024, batch=8):
        self.name, self.layers, self.d, self.heads, self.vocab = name, layers, d, heads, vocab
        self.seq, self.batch = seq, batch
        self.tokens = seq * batch
        g, a = _block_fwd_flops(self.tokens, d, d, 4 * d, batch, heads, d // heads, seq)
        self.flops = 3.0 * (layers * (g + a) + 2.0 * self.tokens * d * vocab)
        self.config = {"workload": name, "layers": layers, "d_model": d, "heads": heads, "ffn": 4 * d,
                       "vocab": vocab, "seq_len": seq, "batch": batch, "tokens_per_step": self.tokens,
                       "parallelism": "single GPU, whole model"}

    def setup(self, dev):
        import torch

        from resihp.config import TrainConfig
        from resihp.model import ReferenceTransformer

        cfg = TrainConfig(model_dim=self.d, num_layers=self.layers, num_heads=self.heads, batch_size=self.batch,
                          micro_batch_size=self.batch, seed=0, tp=1, pp=1, dp=1, iterations=1)
        torch.manual_seed(0)
        self.model = ReferenceTransformer(cfg, vocab_size=self.vocab, sequence_length=self.seq)
        with torch.no_grad():
            for n, p in self.model.named_parameters():
                if "norm" not in n:
                    p.normal_(0.0, 0.02)
        self.model = self.model.to(dev, torch.bfloat16)
        g = torch.Generator().manual_seed(1)
        self.tok = torch.randint(0, self.vocab, (self.batch, self.seq), generator=g).to(dev)

    def params(self):
        return list(self.model.parameters())

    def step(self):
        from resihp.reference import next_token_loss

        self.loss = next_token_loss(self.model(self.tok), self.tok, self.vocab)
        self.loss.backward()

    def outputs(self):
        return [self.loss] + [p.grad for p in self.params()]

    def cpu_sample(self, budget_s):
        import torch

        from oracle import torch_ref

        st = torch_ref.synthetic_state(self.d, self.layers, self.vocab, self.seq, std=0.02, seed=0)
        st = {k: v.requires_grad_(True) for k, v in st.items()}
        bsz = 2  # a quarter of the batch keeps the sample near 10 s
        tok = torch.randint(0, self.vocab, (bsz, self.seq), generator=torch.Generator().manual_seed(1))

        def one():
            logits = torch_ref.model_forward(st, tok, self.heads, range(self.layers))
            torch_ref.next_token_loss(logits, tok, self.vocab).backward()

        sec = _median_time(one, budget_s)
        return {"tokens": bsz * self.seq, "seconds": sec,
                "sample": f"fwd+bwd of the whole LM at batch {bsz} of {self.batch} (seq {self.seq}), fp32, oracle "
                          f"torch-CPU restatement; median of 3 after 1 warm-up"}


class GPT2SmallFused(GPT2Small):
    """GPT-2-small with the LM head fused into the cross-entropy (no [8, 1024, 50257] logits or
    logit-gradient tensors; the backward recomputes the logits in vocabulary chunks)."""

    def __init__(self):
        super().__init__(name="gpt2_small_lm_fused_head")
        self.flops += 2.0 * self.tokens * self.d * self.vocab  # the backward's logit recompute
        self.config["lm_head"] = "fused with the cross-entropy (logits recomputed in the backward)"

    def step(self):
        self.loss = self.model.next_token_loss(self.tok)
        self.loss.backward()


class PPStage(ShardBlock):
    """One 1F1B pipeline stage: 6 of 24 layers (d 2048, 16 heads, FFN 8192), 8 micro-batches of 2x2048."""

    def __init__(self, name="pp_stage_1f1b"):
        super().__init__(name, d=2048, heads=16, tp=1, rank=0, seq=2048, batch=2, layers=6)
        self.micro = 8
        self.tokens = self.micro * self.batch * self.seq
        self.flops *= self.micro
        self.config.update({"micro_batches": self.micro, "stage_index": 1, "num_stages": 4,
                            "tokens_per_step": self.tokens, "parallelism": "one PP stage (1F1B order) on 1 GPU"})

    def setup(self, dev):
        import torch

        super().setup(dev)
        g = torch.Generator().manual_seed(2)
        self.xs = [torch.randn(self.batch, self.seq, self.d, generator=g).to(dev, torch.bfloat16).requires_grad_(True)
                   for _ in range(self.micro)]
        self.dys = [(torch.randn(self.batch, self.seq, self.d, generator=g) * 1e-2).to(dev, torch.bfloat16)
                    for _ in range(self.micro)]

    def params(self):
        return list(self.stage.parameters()) + self.xs

    def step(self):
        from resihp.parallel.pp import run_1f1b

        run_1f1b(self.stage, stage_index=1, num_stages=4, inputs=self.xs, grads=self.dys)

    def outputs(self):
        return [p.grad for p in self.params()]

    def cpu_sample(self, budget_s):
        import torch

        from oracle import torch_ref

        st = {k: v.float().requires_grad_(True) for k, v in self._state().items()}
        g = torch.Generator().manual_seed(2)
        x = torch.randn(self.batch, self.seq, self.d, generator=g).requires_grad_(True)
        dy = torch.randn(self.batch, self.seq, self.d, generator=g) * 1e-2

        def one():
            out = torch_ref.shard_forward(st, num_heads=self.heads, tp_rank=0, tp_size=1, vocab_size=8,
                                          layer_ids=range(self.layers), is_first=False, is_last=False, hidden=x)
            out.backward(dy)

        sec = _median_time(one, budget_s)
        return {"tokens": self.batch * self.seq, "seconds": sec,
                "sample": f"one micro-batch ({self.batch}x{self.seq}) of the {self.layers}-layer stage, fwd+bwd, fp32, "
                          f"oracle torch-CPU restatement; median of 3 after 1 warm-up"}


class ReshardShard(ShardBlock):
    """The TP=2 rank-1 shard of a d2048 / FFN 8192 block after a TP4 -> TP2 reshard: the step is
    the shard's fwd+bwd; the pack (repack_shards of one layer's four TP4 shards of every matrix
    into both TP2 shards, on device) is measured as its own HBM-bound leg."""

    def extra(self, dev):
        return {"reshard_pack": reshard_pack_leg(dev)}


def reshard_pack_leg(dev, reps=10):
    """TP4 -> TP2 re-slice of one d2048 / FFN 8192 layer (q, k, v, fc1 split on dim 0; out, fc2 on
    dim 1) into both new ranks' shards: one batched copy launch (RepackPlan), checked bit for bit
    against torch.cat / torch.chunk, timed with a cold cache (a 1 GiB buffer, larger than L2 plus
    the 256 MB Infinity Cache, is written before every pack)."""
    import torch

    from resihp.parallel.reshard import RepackPlan

    d, ff = 2048, 8192
    g = torch.Generator().manual_seed(3)
    mats = {"q": ((d, d), 0), "k": ((d, d), 0), "v": ((d, d), 0), "fc1": ((ff, d), 0), "out": ((d, d), 1),
            "fc2": ((d, ff), 1)}
    shards = {n: [t.contiguous() for t in torch.chunk((torch.randn(*shape, generator=g) * 0.02).to(dev, torch.bfloat16),
                                                      4, dim)] for n, (shape, dim) in mats.items()}
    plan = RepackPlan([(shards[n], mats[n][1]) for n in mats], (0, 1), 2)

    def pack():
        outs = plan.run()
        return [x for pair in zip(outs[0], outs[1]) for x in pair]

    out = pack()
    k = 0
    for n in mats:
        full = torch.cat(shards[n], mats[n][1])
        for r in range(2):
            if not torch.equal(out[k], torch.chunk(full, 2, mats[n][1])[r]):
                raise RuntimeError(f"reshard pack of {n} rank {r} differs from torch.cat/chunk")
            k += 1
    moved = 2 * sum(t.numel() * t.element_size() for t in out)  # each byte read once, written once
    del out
    flush = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    evs = []
    for _ in range(reps):
        flush.fill_(1)
        ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
        ev[0].record()
        pack()
        ev[1].record()
        evs.append(ev)
    torch.cuda.synchronize()
    us = sorted(a.elapsed_time(b) for a, b in evs)[reps // 2] * 1e3
    gbps = moved / us / 1e3
    return {"bytes_per_launch": moved, "mean_us": round(us, 2), "GB/s": round(gbps, 1),
            "hbm_frac": round(gbps * 1e9 / PEAK_HBM, 4), "bit_exact": True, "launches_per_step": 1,
            "what": "TP4->TP2 pack (RepackPlan, one launch) of one d2048/FFN8192 layer, both new ranks; "
                    "cold cache (1 GiB written before each pack), median of 10"}


def xent_leg(dev, reps=5):
    """Next-token cross-entropy with its gradient (rh_xent_fwd writing dlogits) at GPT-2-small's
    rows: logits [8, 1024, 50257] bf16 (row stride 50264), targets uniform in [0, 50257)."""
    import torch

    from resihp import ops, profiling

    batch, seq, vocab = 8, 1024, 50257
    g = torch.Generator(device="cpu").manual_seed(5)
    buf = torch.empty(batch * seq, 50264, dtype=torch.bfloat16, device=dev)
    buf[:, :vocab] = (torch.randn(batch * seq, vocab, generator=g) * 2.0).to(dev, torch.bfloat16)
    logits = buf[:, :vocab].view(batch, seq, vocab).requires_grad_(True)
    tokens = torch.randint(0, vocab, (batch, seq), generator=g).to(dev)
    ops.next_token_loss(logits, tokens, vocab)
    torch.cuda.synchronize()
    with profiling.record() as events:
        for _ in range(reps):
            ops.next_token_loss(logits, tokens, vocab)
    torch.cuda.synchronize()
    (label, k), = profiling.summary(events).items()
    return {"bytes_per_launch": k["bytes_per_launch"], "mean_us": round(k["mean_ms"] * 1e3, 2),
            "GB/s": round(k["gbps"], 1), "hbm_frac": round(k["gbps"] * 1e9 / PEAK_HBM, 4), "launches_per_step": 1,
            "what": f"{label} at GPT-2-small rows (8x1024 tokens, vocab 50257, bf16), mean of {reps}"}


def adamw_leg(dev, reps=10):
    """One resihp.optim.AdamW step over the fp32 parameters of one TP=4 rank's GPT-1.3B layer (q, k, v
    512x2048, out 2048x512, fc1 and fc2 2048x2048 shards, two LayerNorms: 10 tensors, 12.6 M values)
    -- rh_adamw_multi, one launch; 28 bytes per value (param, grad, exp_avg, exp_avg_sq read; param
    and both moments written).  Cold cache (a 1 GiB buffer written before every step), median."""
    import torch

    from resihp.optim import AdamW

    d, dl, ff = 2048, 512, 2048
    shapes = [(dl, d)] * 3 + [(d, dl), (ff, d), (d, ff)] + [(d,)] * 4
    g = torch.Generator().manual_seed(11)
    params = []
    for shp in shapes:
        t = torch.nn.Parameter((torch.randn(*shp, generator=g) * 0.02).to(dev))
        t.grad = (torch.randn(*shp, generator=g) * 1e-3).to(dev)
        params.append(t)
    opt = AdamW(params, lr=1e-3)
    opt.step()
    torch.cuda.synchronize()
    numel = sum(t.numel() for t in params)
    moved = 28 * numel
    flush = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    evs = []
    for _ in range(reps):
        flush.fill_(1)
        ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
        ev[0].record()
        opt.step()
        ev[1].record()
        evs.append(ev)
    torch.cuda.synchronize()
    us = sorted(a.elapsed_time(b) for a, b in evs)[reps // 2] * 1e3
    gbps = moved / us / 1e3
    return {"bytes_per_launch": moved, "mean_us": round(us, 2), "GB/s": round(gbps, 1),
            "hbm_frac": round(gbps * 1e9 / PEAK_HBM, 4), "launches_per_step": 1,
            "what": f"AdamW step (rh_adamw_multi, one launch) over one TP4 GPT-1.3B layer's fp32 parameters "
                    f"({len(params)} tensors, {numel} values); cold cache, median of {reps}"}


WORKLOADS = {
    "tp4_shard_gpt1.3b_block": lambda: ShardBlock("tp4_shard_gpt1.3b_block"),
    "gpt2_small_lm": GPT2Small,
    "gpt2_small_lm_fused_head": GPT2SmallFused,
    "pp_stage_1f1b": PPStage,
    "tp2_shard_after_reshard": lambda: ReshardShard("tp2_shard_after_reshard", d=2048, heads=16, tp=2, rank=1,
                                                    seq=2048, batch=2),
}


# ---------------------------------------------------------------------------
# measurement
# ---------------------------------------------------------------------------
def _measured_traffic(workload: str, kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 counter summary of this
    workload (profiles/<workload>_counters.md, line `traffic_bytes_per_launch <kernel> = N`):
    FETCH_SIZE + WRITE_SIZE of a --pmc run, each scaled by what the same counter reads for a
    copy of known size.  The summary records the sources digest of the library it measured
    (`library_sources_sha256 = ...`); a summary of other sources, or one that does not cover this
    kernel, gives (None, reason)."""
    path = ROOT / "profiles" / f"{workload}_counters.md"
    if not path.exists():
        return None, "no counter summary for this workload"
    key = f"traffic_bytes_per_launch {kernel} ="
    stamp, value = None, None
    for line in path.read_text().splitlines():
        line = line.strip().strip("`")
        if line.startswith("library_sources_sha256 ="):
            stamp = line.split("=", 1)[1].strip()
        if line.startswith(key):
            value = float(line[len(key):].strip())
    from resihp.profiling import library_sources_digest

    if stamp != library_sources_digest():
        return None, "counter summary measured other library sources"
    if value is None:
        return None, "counter summary does not cover this kernel"
    return value, f"profiles/{path.name}"


def _cpu_info() -> dict:
    """Threads to use for the CPU baseline and what they are: the physical cores (distinct
    package/core ids) of this process's affinity set, capped at the CPU share a GPU job gets here
    (OMP_NUM_THREADS when set), and the CPU model name."""
    try:
        cpus = sorted(os.sched_getaffinity(0))
    except AttributeError:
        cpus = list(range(os.cpu_count() or 1))
    cores = set()
    for c in cpus:
        topo = Path(f"/sys/devices/system/cpu/cpu{c}/topology")
        try:
            cores.add((topo.joinpath("physical_package_id").read_text().strip(),
                       topo.joinpath("core_id").read_text().strip()))
        except OSError:
            cores.add(("?", str(c)))
    physical = max(1, len(cores))
    share = os.environ.get("OMP_NUM_THREADS", "")
    use = min(physical, int(share)) if share.isdigit() and int(share) > 0 else physical
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"threads": use, "physical_cores_in_affinity": physical, "logical_cpus_in_affinity": len(cpus),
            "model": model}


def _median_time(fn, budget_s: float) -> float:
    """1 warm-up call, then the median of 3 timed calls (fewer if one call exceeds the budget)."""
    t0 = time.perf_counter()
    fn()
    times = []
    for _ in range(3):
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
        if time.perf_counter() - t0 > budget_s:
            break
    return sorted(times)[len(times) // 2]


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="tp4_shard_gpt1.3b_block", choices=sorted(WORKLOADS))
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra-legs", action="store_true",
                    help="skip the standalone cross-entropy and reshard-pack bandwidth legs")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="first copy MIB MiB with the library's copy kernel (copy_kernel<16>): a transfer of "
                         "known size that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings")
    args = ap.parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build computes one rank's shard per GPU with no collectives "
              f"(--gpus {args.gpus} is not supported)", file=sys.stderr)
        return 2

    import torch

    from resihp import profiling

    dev = torch.device("cuda:0")
    if args.copy_calibration > 0:
        from resihp.parallel.reshard import device_cat

        src = torch.empty(args.copy_calibration * (1 << 20) // 2, dtype=torch.bfloat16, device=dev).view(-1, 4096)
        src.fill_(1.0)
        for _ in range(3):
            device_cat([src], 0)
        torch.cuda.synchronize()
        _log(f"[bench] copy calibration: 3 copies of {args.copy_calibration} MiB (copy_kernel<16>)")
        del src
    wl = WORKLOADS[args.workload]()
    _log(f"[bench] workload {wl.name}: setup")
    wl.setup(dev)
    for _ in range(max(1, args.warmup)):
        wl.zero_grads()
        wl.step()
    torch.cuda.synchronize()
    _log(f"[bench] warm-up done ({args.warmup} steps)")

    use_graph = not args.no_graph
    graph = None
    if use_graph:
        eager = [t.detach().clone() for t in wl.outputs()]
        # A live output keeps its autograd graph -- and the AccumulateGrad nodes bound to the
        # stream it ran on -- alive; capture must start with none of them left.
        wl.release()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                wl.zero_grads()
                wl.step()
                wl.release()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        wl.zero_grads()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            wl.step()
        for _ in range(3):  # every replay must equal the eager step
            graph.replay()
            torch.cuda.synchronize()
            for a, b in zip(wl.outputs(), eager):
                if not torch.equal(a, b):
                    raise RuntimeError("graph replay differs from the eager step")
        _log("[bench] HIP graph captured; replays match the eager step bit for bit")

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        if graph is not None:
            graph.replay()
        else:
            wl.zero_grads()
            wl.step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms = elapsed / args.steps * 1e3
    tokens_per_s = wl.tokens * args.steps / elapsed
    tflops = wl.flops / (ms * 1e-3) / 1e12
    _log(f"[bench] timed {args.steps} steps: {ms:.3f} ms/step, {tokens_per_s:.4g} tokens/s, {tflops:.1f} TFLOP/s")

    # per-kernel roofline: eager steps with HIP events around every GEMM / attention launch
    wl.release()
    with profiling.record() as events:
        for _ in range(min(args.steps, 5)):
            wl.zero_grads()
            wl.step()
    torch.cuda.synchronize()
    kernels = profiling.summary(events)
    n_steps = min(args.steps, 5)
    # dominant = the MFMA kernel with the most time per step (the split-K reduce is a separate,
    # bandwidth-bound kernel with no FLOPs of its own)
    dominant = max((k for k in kernels if kernels[k]["flops"] > 0), key=lambda k: kernels[k]["total_ms"])
    dk = kernels[dominant]
    achieved = dk["tflops"]
    traffic, traffic_src = _measured_traffic(wl.name, dominant)
    roofline = {"bound": "mfma", "kernel": dominant, "achieved": round(achieved, 2), "peak": PEAK_BF16 / 1e12,
                "unit": "TFLOP/s", "frac": round(achieved * 1e12 / PEAK_BF16, 4), "traffic": traffic,
                "traffic_source": traffic_src, "timing": "HIP events around each launch, 5 eager steps",
                "launches_per_step": dk["launches"] // n_steps, "mean_launch_us": round(dk["mean_ms"] * 1e3, 2),
                "flops_per_launch": dk["flops_per_launch"]}
    per_kernel = {k: {"launches_per_step": v["launches"] // n_steps, "mean_us": round(v["mean_ms"] * 1e3, 2),
                      "tflops": round(v["tflops"], 1)} for k, v in sorted(kernels.items()) if v["flops"] > 0}
    # bandwidth-bound kernels of the step: algorithmic bytes (inputs read once, outputs written
    # once) over the HIP-event duration, against the 8 TB/s HBM peak
    hbm = {k: {"launches_per_step": v["launches"] // n_steps, "mean_us": round(v["mean_ms"] * 1e3, 2),
               "bytes_per_launch": int(v["bytes_per_launch"]), "GB/s": round(v["gbps"], 1),
               "hbm_frac": round(v["gbps"] * 1e9 / PEAK_HBM, 4)}
           for k, v in sorted(kernels.items()) if v["bytes"] > 0}
    _log("[bench] per-kernel: " + json.dumps(per_kernel))
    _log("[bench] bandwidth kernels: " + json.dumps(hbm))
    if args.workload == "tp4_shard_gpt1.3b_block" and not args.no_extra_legs:
        # the path's other bandwidth kernels, measured in this run at their own workloads' sizes
        hbm["xent_fwd (+ dlogits), GPT-2-small rows"] = xent_leg(dev)
        hbm["reshard_pack, TP4->TP2 d2048/FFN8192 layer"] = reshard_pack_leg(dev)
        hbm["adamw_multi, one TP4 GPT-1.3B layer (fp32)"] = adamw_leg(dev)
        _log("[bench] extra bandwidth legs done")

    cpu = None
    if not args.no_cpu_baseline:
        info = _cpu_info()
        torch.set_num_threads(info["threads"])
        _log(f"[bench] CPU baseline on {info['threads']} threads of {info['model']} (budget {args.cpu_seconds}s)")
        sample = wl.cpu_sample(args.cpu_seconds)
        cpu = {"value": round(sample["tokens"] / sample["seconds"], 2), "unit": "tokens/s", "cores": info["threads"],
               "kind": "port", "sample": sample["sample"], "cpu_model": info["model"],
               "physical_cores_in_affinity": info["physical_cores_in_affinity"], "torch": torch.__version__}

    line = {
        "metric": METRIC,
        "value": round(tokens_per_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) activations, N(0,1e-2) upstream grads, N(0,0.02) weights)",
        "config": dict(wl.config, graph=use_graph),
        "tflops": round(tflops, 2),
        "mfma_frac_step": round(tflops * 1e12 / PEAK_BF16, 4),
        "algorithmic_flops_per_step": wl.flops,
        "roofline": roofline,
        "kernels": per_kernel,
        "hbm": hbm,
        "cpu_baseline": cpu,
        "device": torch.cuda.get_device_name(0),
    }
    line.update(wl.extra(dev))
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
