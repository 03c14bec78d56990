"""Pipeline-stage boundary tensors on the device: chunk routing, bf16 slabs and reassembly.

Restates the scatter/gather boundary of ``PipelineRuntime`` (resihp/parallel/pp.py:57-80,
211-295).  A stage's output activation (and the gradient of its input) is replicated across its
TP group; exactly one copy crosses the hop, cut into ``N = max(U, D)`` equal contiguous chunks of
the flattened tensor, chunk ``k`` travelling from ``up[k*U//N]`` to ``down[k*D//N]``.  Each
receiver collects its chunks -- a contiguous run, its ``1/D`` share -- in one slab, and the
receiving stage rebuilds the whole tensor from its members' slabs in TP-rank order (the
reference all-gathers them and ``torch.cat``s, pp.py:283-295).

What one GPU shows of it (the P2P transfers and the intra-stage all-gather are collectives):

* the routing tables (:func:`scatter_routing`, :func:`my_chunks`) -- pure, as in the reference;
* the send side as zero-copy views of the flat activation (:func:`scatter_send_chunks`);
* the receive slab in the activation's own dtype -- bf16 for a bf16 model, where the reference's
  slab is fp32 (pp.py:271) and would double the bytes on the link and in the gather;
* the reassembly of a stage's slabs into the boundary tensor by ONE batched copy launch
  (:func:`reconstruct`, ``rh_copy2d_batch``) instead of a ``torch.cat``;
* :func:`exchange`, the whole hop with every rank's slab on this GPU: every chunk of every
  sender copied into its receiver's slab slot by one batched launch -- what the hop's P2P
  transfers deliver, byte for byte.
"""

from __future__ import annotations

import math

import torch

from .. import _hip as H
from .reshard import _copy_segments


def scatter_routing(up_members, down_members) -> tuple[tuple[int, int], ...]:
    """The ``(sender, receiver)`` pair of each chunk of one hop (pp.py:57-80): ``N = max(U, D)``
    chunks, chunk ``k`` from ``up[k*U//N]`` to ``down[k*D//N]``.  Pure."""
    up, down = tuple(up_members), tuple(down_members)
    if not up or not down:
        raise ValueError("both stages of a hop need at least one member")
    n = max(len(up), len(down))
    return tuple((up[k * len(up) // n], down[k * len(down) // n]) for k in range(n))


def my_chunks(rank: int, up_members, down_members) -> tuple[tuple[int, int], ...]:
    """``(chunk index, peer rank)`` of every chunk ``rank`` carries on this hop (pp.py:213-229):
    the sender side if ``rank`` is in the upstream stage, else the receiver side."""
    sending = rank in tuple(up_members)
    if not sending and rank not in tuple(down_members):
        raise ValueError(f"rank {rank} is in neither stage of the hop")
    return tuple((k, recv if sending else send)
                 for k, (send, recv) in enumerate(scatter_routing(up_members, down_members))
                 if (send if sending else recv) == rank)


def _width(numel: int, up_members, down_members) -> int:
    n = max(len(tuple(up_members)), len(tuple(down_members)))
    if numel % n:
        raise ValueError(f"a boundary tensor of {numel} elements does not split into {n} equal chunks")
    return numel // n


def scatter_send_chunks(tensor: torch.Tensor, rank: int, up_members, down_members) -> list:
    """``[(peer, chunk)]`` this upstream rank sends (pp.py:242-260): contiguous views of the
    flattened ``tensor`` -- no copy, the send reads the activation in place."""
    flat = tensor.detach().reshape(-1)
    if not flat.is_contiguous():
        raise ValueError("the boundary tensor must be contiguous")
    width = _width(flat.numel(), up_members, down_members)
    return [(peer, flat[k * width:(k + 1) * width]) for k, peer in my_chunks(rank, up_members, down_members)]


def gather_slab(shape, dtype, device, rank: int, up_members, down_members):
    """A slab for this downstream rank's chunks and the slot each peer's chunk lands in
    (pp.py:262-281), in ``dtype`` (the activation's dtype; the reference allocates fp32)."""
    width = _width(math.prod(shape), up_members, down_members)
    mine = my_chunks(rank, up_members, down_members)
    slab = torch.empty(len(mine) * width, dtype=dtype, device=device)
    return slab, [(peer, slab[i * width:(i + 1) * width]) for i, (_k, peer) in enumerate(mine)]


def reconstruct(shares: list, shape) -> torch.Tensor:
    """The boundary tensor from the receiving stage's slabs in TP-rank order (pp.py:283-295:
    ``torch.cat(all_gather(slab)).view(shape)``).  At degree 1 the slab already is the tensor
    (a view, no copy); otherwise one batched copy launch writes every share to its place."""
    if len(shares) == 1:
        return shares[0].view(shape)
    H.require_gpu(*shares)
    first = shares[0]
    for s in shares:
        if s.dtype != first.dtype or s.dim() != 1 or s.numel() != first.numel() or not s.is_contiguous():
            raise ValueError("slabs must be contiguous, of one dtype and one size")
    if first.numel() * len(shares) != math.prod(shape):
        raise ValueError(f"{len(shares)} slabs of {first.numel()} elements do not fill {tuple(shape)}")
    out = torch.empty(tuple(shape), dtype=first.dtype, device=first.device)
    nbytes = first.numel() * first.element_size()
    base = out.data_ptr()
    _copy_segments([(s.data_ptr(), base + i * nbytes, nbytes, nbytes, 1, nbytes) for i, s in enumerate(shares)], out)
    return out


def exchange(tensor: torch.Tensor, up_members, down_members, *, backward: bool = False) -> dict:
    """One hop with every rank on this GPU: ``{receiver: slab}`` after the chunks of the replicated
    ``tensor`` were copied into their receivers' slab slots by one batched launch -- the bytes the
    hop's P2P transfers deliver.  Forward, the downstream members receive; ``backward=True`` sends
    the gradient of the boundary back over the same rank pairs (pp.py:301-337), so the upstream
    members receive the chunks they sent."""
    H.require_gpu(tensor)
    up, down = tuple(up_members), tuple(down_members)
    if set(up) & set(down):
        raise ValueError("adjacent stages own disjoint ranks")
    flat = tensor.detach().reshape(-1)
    if not flat.is_contiguous():
        raise ValueError("the boundary tensor must be contiguous")
    routing = scatter_routing(up, down)
    width = _width(flat.numel(), up, down)
    end = 0 if backward else 1
    nbytes = width * tensor.element_size()
    slabs, segs = {}, []
    for r in (up if backward else down):
        ks = [k for k, pair in enumerate(routing) if pair[end] == r]  # ascending: a contiguous run
        slab = torch.empty(len(ks) * width, dtype=tensor.dtype, device=tensor.device)
        for i, k in enumerate(ks):
            segs.append((flat[k * width:].data_ptr(), slab[i * width:].data_ptr(), nbytes, nbytes, 1, nbytes))
        slabs[r] = slab
    _copy_segments(segs, tensor)
    return slabs
