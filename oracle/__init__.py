"""CPU oracle for the decoder-LM forward/backward step -- TEST INFRASTRUCTURE ONLY.

Nothing in the product (the ``resihp`` package or ``libresihp_hip.so``) imports
this package.  Only ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline
leg of ``bench.py`` use it, and only as the checker / the timed CPU baseline.

* :mod:`oracle.torch_ref` -- op-for-op restatement of the reference math on torch
  CPU tensors (fp32 or fp64) with torch autograd: the module form of
  resihp/model.py:48-137, the shard form of resihp/parallel/tp.py:222-273, the
  loss of resihp/reference.py:41-50, the AdamW constants of reference.py:20-38,
  the TP layout / cat / chunk of resihp/parallel/reshard.py:41-123 and the 1F1B
  order of resihp/planner/pp.py:36-77.
* :mod:`oracle.numpy_ref` -- an independent fp64 numpy restatement of the same
  forward with a hand-derived backward (no autograd), used to pin torch_ref.

How each part is pinned (tests/test_oracle.py):
* seeded init, loss, logits, all gradients and the post-AdamW step records:
  golden vectors written from the reference itself (tests/golden/);
* GEMM / attention / LayerNorm / GELU / cross-entropy / embedding: the
  independent numpy restatement in fp64 and central finite differences, plus
  closed forms (zero LM head -> loss = ln V; softmax rows sum to 1; gradient
  rows of the loss sum to 0; attention row 0 equals v_0);
* TP shard math: a TP=1 shard equals the full model; the sum of the partial
  outputs over all ranks equals the full model's (what the reference's
  all-reduce would produce);
* cat / chunk: torch.cat / torch.chunk and round trips;
* 1F1B order: the schedule literals of the reference's own tests.
"""
