"""TP shard layout and the bit-exact on-device re-slice.

Restates the layout tables and pure functions of resihp/parallel/reshard.py:36-123
-- ``ReshardError``, ``shard_dims``, ``reconstruct_full`` (peer shards, else the
checkpoint, else ``ReshardError``), ``local_slice`` (``torch.chunk`` semantics:
chunk = ceil(size / new_size), short last chunk) and ``shard_logical_state`` --
with the concatenation and slicing done by the HIP copy kernels on the GPU
(``rh_reshard_pack`` / ``rh_reshard_unpack`` / ``rh_copy2d_batch``).  Results
are byte-identical to ``torch.cat`` / ``torch.chunk``.

``repack_shards`` builds a rank's shard under a new TP degree straight from the
old shards (TP4 -> TP2: new shard r = cat(old[2r], old[2r+1])) without
materialising the full tensor; it handles any old/new degree pair by copying
each overlapping piece.

The distributed driver ``reshard_tp_state`` (an ``all_gather_object`` of CPU
shards, reshard.py:126-243) is a collective and is not part of this package.
"""

from __future__ import annotations

import ctypes

import torch

from .. import _hip as H


class ReshardError(RuntimeError):
    """Raised when a logical tensor is available from neither peers nor checkpoint."""


_GLOBAL_SHARD_DIMS = {
    "token_embedding.weight": 0,
    "position_embedding.weight": None,
    "final_norm.weight": None,
    "final_norm.bias": None,
    "lm_head.weight": 0,
}
_LAYER_SHARD_DIMS = {
    "attn_norm.weight": None,
    "attn_norm.bias": None,
    "attn.q_proj.weight": 0,
    "attn.k_proj.weight": 0,
    "attn.v_proj.weight": 0,
    "attn.out_proj.weight": 1,
    "mlp_norm.weight": None,
    "mlp_norm.bias": None,
    "mlp.fc1.weight": 0,
    "mlp.fc2.weight": 1,
}
_SHARDED_FIELDS = ("param", "exp_avg", "exp_avg_sq")
_REPLICATED_FIELDS = ("step",)


def shard_dims(layer_ids) -> dict[str, int | None]:
    """Logical name -> shard dim (``None`` = replicated) for the whole model."""
    dims = dict(_GLOBAL_SHARD_DIMS)
    for gid in layer_ids:
        for suffix, dim in _LAYER_SHARD_DIMS.items():
            dims[f"layers.{gid}.{suffix}"] = dim
    return dims


# ---------------------------------------------------------------------------
# device copies
# ---------------------------------------------------------------------------
def _split_shape(shape, dim: int) -> tuple[int, int, int]:
    outer = 1
    for s in shape[:dim]:
        outer *= s
    inner = 1
    for s in shape[dim + 1:]:
        inner *= s
    return outer, shape[dim], inner


def _copy_segments(segs: list[tuple[int, int, int, int, int, int]], like: torch.Tensor) -> None:
    if not segs:
        return
    arr = (H.rh_copy2d * len(segs))()
    for i, (src, dst, src_ld, dst_ld, rows, row_bytes) in enumerate(segs):
        arr[i].src, arr[i].dst = src, dst
        arr[i].src_ld_bytes, arr[i].dst_ld_bytes = src_ld, dst_ld
        arr[i].rows, arr[i].row_bytes = rows, row_bytes
    H.call("rh_copy2d_batch", arr, len(segs), H.stream_of(like))


def device_cat(parts: list[torch.Tensor], dim: int) -> torch.Tensor:
    """``torch.cat(parts, dim)`` by the HIP copy kernels (bit-exact)."""
    H.require_gpu(*parts)
    first = parts[0]
    for p in parts:
        if p.dtype != first.dtype or p.dim() != first.dim():
            raise ValueError("shards must share dtype and rank")
        for d in range(first.dim()):
            if d != dim and p.shape[d] != first.shape[d]:
                raise ValueError(f"shard shapes {tuple(first.shape)} and {tuple(p.shape)} differ off dim {dim}")
    parts = [p.contiguous() for p in parts]
    total = sum(p.shape[dim] for p in parts)
    shape = list(first.shape)
    shape[dim] = total
    out = torch.empty(shape, dtype=first.dtype, device=first.device)
    es = first.element_size()
    if first.dim() == 2:
        n = len(parts)
        src = (ctypes.c_void_p * n)(*[p.data_ptr() for p in parts])
        ext = (ctypes.c_int64 * n)(*[p.shape[dim] for p in parts])
        rows, cols = first.shape if dim == 1 else (0, first.shape[1])
        H.call("rh_reshard_pack", src, ext, n, rows, cols, dim, es, out.data_ptr(), H.stream_of(out))
        return out
    outer, _, inner = _split_shape(shape, dim)
    segs, off = [], 0
    for p in parts:
        e = p.shape[dim]
        if e and outer and inner:
            segs.append((p.data_ptr(), out.data_ptr() + off * inner * es, e * inner * es, total * inner * es, outer,
                         e * inner * es))
        off += e
    _copy_segments(segs, out)
    return out


def device_narrow(full: torch.Tensor, dim: int, start: int, length: int) -> torch.Tensor:
    """``full.narrow(dim, start, length).contiguous().clone()`` by the HIP copy kernels."""
    H.require_gpu(full)
    full = full.contiguous()
    shape = list(full.shape)
    shape[dim] = length
    out = torch.empty(shape, dtype=full.dtype, device=full.device)
    es = full.element_size()
    if full.dim() == 2 and length > 0:
        rows, cols = full.shape
        dst = (ctypes.c_void_p * 2)(None, out.data_ptr())
        ext = (ctypes.c_int64 * 2)(start, length)
        H.call("rh_reshard_unpack", full.data_ptr(), rows, cols, dim, es, 2, dst, ext, H.stream_of(out))
        return out
    outer, size, inner = _split_shape(list(full.shape), dim)
    if length and outer and inner:
        _copy_segments([(full.data_ptr() + start * inner * es, out.data_ptr(), size * inner * es, length * inner * es,
                         outer, length * inner * es)], out)
    return out


def device_clone(t: torch.Tensor) -> torch.Tensor:
    H.require_gpu(t)
    t = t.contiguous()
    out = torch.empty_like(t)
    nbytes = t.numel() * t.element_size()
    if nbytes:
        _copy_segments([(t.data_ptr(), out.data_ptr(), nbytes, nbytes, 1, nbytes)], out)
    return out


def _chunk_bounds(size: int, new_size: int) -> list[tuple[int, int]]:
    """Start/stop of every piece ``torch.chunk(size, new_size)`` returns."""
    if new_size < 1:
        raise ValueError("chunk expects `chunks` to be greater than 0")
    step = -(-size // new_size) if size else 0
    if step == 0:
        return [(0, 0)] * new_size if size == 0 else []
    return [(s, min(s + step, size)) for s in range(0, size, step)]


# ---------------------------------------------------------------------------
# the reference's pure functions, on the device
# ---------------------------------------------------------------------------
def reconstruct_full(name, shard_dim, old_size, contributions, checkpoint=None):
    """Rebuild one full logical tensor from peer shards (reshard.py:84-104).

    Returns ``(full_tensor, source)`` with ``source`` in ``{"peer", "checkpoint"}``.
    """
    if shard_dim is None:
        if contributions:
            first = min(contributions)
            return contributions[first], "peer"
    elif all(index in contributions for index in range(old_size)):
        parts = [contributions[index] for index in range(old_size)]
        return device_cat(parts, shard_dim), "peer"
    if checkpoint is not None and name in checkpoint:
        return checkpoint[name], "checkpoint"
    raise ReshardError(f"logical tensor {name} unavailable from peers and checkpoint")


def local_slice(full, shard_dim, new_rank, new_size):
    """This rank's contiguous ``torch.chunk`` shard of ``full`` (reshard.py:107-111)."""
    if shard_dim is None:
        return device_clone(full.detach())
    bounds = _chunk_bounds(full.shape[shard_dim], new_size)
    start, stop = bounds[new_rank]  # IndexError past the last chunk, as torch.chunk(...)[i]
    return device_narrow(full.detach(), shard_dim, start, stop - start)


def shard_logical_state(full_state, *, layout, tp_rank, tp_size):
    """Cut a full logical state down to one rank's shards (reshard.py:114-123)."""
    return {name: local_slice(full_state[name], dim, tp_rank, tp_size) for name, dim in layout.items()}


def repack_shards(old_shards: list, shard_dim, new_rank: int, new_size: int) -> torch.Tensor:
    """Rank ``new_rank``'s shard under degree ``new_size``, built from the old degree's shards.

    Equal to ``local_slice(torch.cat(old_shards, shard_dim), shard_dim, new_rank, new_size)``
    byte for byte, but copies only the pieces that land in the new shard.
    """
    if shard_dim is None:
        return device_clone(old_shards[0].detach())
    H.require_gpu(*old_shards)
    old = [s.detach().contiguous() for s in old_shards]
    total = sum(s.shape[shard_dim] for s in old)
    start, stop = _chunk_bounds(total, new_size)[new_rank]
    pieces, off = [], 0
    for s in old:
        e = s.shape[shard_dim]
        lo, hi = max(start, off), min(stop, off + e)
        if hi > lo:
            pieces.append(s if (lo == off and hi == off + e) else device_narrow(s, shard_dim, lo - off, hi - lo))
        off += e
    if len(pieces) == 1:
        piece = pieces[0]
        return device_clone(piece) if any(piece is o for o in old) else piece
    return device_cat(pieces, shard_dim)



class RepackPlan:
    """A prepared re-slice: for every (old_shards, shard_dim) item and every rank in `new_ranks`,
    the destination tensor is allocated and the copy list built once; ``run()`` is then ONE
    batched copy launch (rh_copy2d_batch) for every piece of every tensor -- a whole layer's
    TP re-slice as a single HBM-bound kernel.  ``outs[r]`` are rank r's new shards, byte-identical
    to ``repack_shards(shards, dim, r, new_size)`` (so to local_slice of the torch.cat)."""

    def __init__(self, items: list, new_ranks, new_size: int):
        self.outs = {}
        segs = []
        self._like = None
        olds = []
        for old_shards, shard_dim in items:
            old = [t.detach().contiguous() for t in old_shards]
            H.require_gpu(*old)
            if shard_dim is not None:
                for t in old:
                    for d in range(t.dim()):
                        if d != shard_dim and t.shape[d] != old[0].shape[d]:
                            raise ValueError(f"shard shapes {tuple(old[0].shape)} and {tuple(t.shape)} differ "
                                             f"off dim {shard_dim}")
            olds.append((old, shard_dim))
            self._like = old[0]
        for r in new_ranks:
            outs = []
            for old, shard_dim in olds:
                es = old[0].element_size()
                if shard_dim is None:
                    out = torch.empty_like(old[0])
                    if out.numel():
                        nb = out.numel() * es
                        segs.append((old[0].data_ptr(), out.data_ptr(), nb, nb, 1, nb))
                    outs.append(out)
                    continue
                total = sum(t.shape[shard_dim] for t in old)
                start, stop = _chunk_bounds(total, new_size)[r]
                shape = list(old[0].shape)
                shape[shard_dim] = stop - start
                out = torch.empty(shape, dtype=old[0].dtype, device=old[0].device)
                outer, _, inner = _split_shape(shape, shard_dim)
                off = 0
                for t in old:
                    e = t.shape[shard_dim]
                    lo, hi = max(start, off), min(stop, off + e)
                    if hi > lo and outer and inner:
                        segs.append((t.data_ptr() + (lo - off) * inner * es,
                                     out.data_ptr() + (lo - start) * inner * es,
                                     e * inner * es, (stop - start) * inner * es, outer, (hi - lo) * inner * es))
                    off += e
                outs.append(out)
            self.outs[r] = outs
        self._olds = olds  # the sources stay alive as long as the plan
        self._n = len(segs)
        self._arr = (H.rh_copy2d * max(1, self._n))()
        for i, (src, dst, src_ld, dst_ld, rows, row_bytes) in enumerate(segs):
            self._arr[i].src, self._arr[i].dst = src, dst
            self._arr[i].src_ld_bytes, self._arr[i].dst_ld_bytes = src_ld, dst_ld
            self._arr[i].rows, self._arr[i].row_bytes = rows, row_bytes

    def run(self) -> dict:
        if self._n:
            H.call("rh_copy2d_batch", self._arr, self._n, H.stream_of(self._like))
        return self.outs


def repack_many(items: list, new_rank: int, new_size: int) -> list:
    """``[repack_shards(shards, dim, new_rank, new_size) for shards, dim in items]`` as one batched
    copy launch (see RepackPlan)."""
    if not items:
        return []
    return RepackPlan(items, (new_rank,), new_size).run()[new_rank]
