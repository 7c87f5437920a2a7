"""Group-quantizer bookkeeping and same-shape layer batching.

Drop-in for gptq_utils/common_utils.py:13-85 of the reference (its multi-GPU
helpers ``partition_layers`` / ``broadcast_quantized_param`` are not part of
this single-GPU build).  Names, signatures and results are the reference's;
``fake_quantize_grouped`` runs all groups in one HIP launch.
"""
import copy
from dataclasses import dataclass

import torch

from . import _lib


def make_group_quantizers(quantizer, columns, groupsize):
    """gptq_utils/common_utils.py:13-16: a deep copy of ``quantizer`` per
    ``groupsize``-column group (one for ``groupsize == -1``).

    For a WeightQuantizer the copies' buffers are cloned together: one tensor
    per buffer name holding every copy's value, unbound into per-copy views
    (each an independent tensor of the original's shape, as a clone is), so a
    14336-column layer's 112 copies cost two tensor operations instead of 224.
    """
    from .quant_utils import WeightQuantizer
    count = 1 if groupsize == -1 else -(-columns // groupsize)
    if type(quantizer) is not WeightQuantizer or count == 1:
        return [copy.deepcopy(quantizer) for _ in range(count)]
    bufs = quantizer._buffers
    per_copy = {n: (None if b is None else
                    b.detach().unsqueeze(0).expand(count, *b.shape).clone().unbind(0))
                for n, b in bufs.items()}
    out = []
    for i in range(count):
        q = quantizer.__deepcopy__({}, clone_buffers=False)
        q.__dict__["_buffers"] = {n: (None if v is None else v[i]) for n, v in per_copy.items()}
        out.append(q)
    return out


def merge_group_quantizers(quantizers, start, end, groupsize):
    """gptq_utils/common_utils.py:19-30: one quantizer holding rows
    [start, end) of every group's (rows, 1) parameters side by side, i.e. a
    per-layer (R, C/g) scale and zero with ``weight_groupsize = groupsize``."""
    merged = copy.deepcopy(quantizers[0])
    for attr in ("scale", "zero"):
        setattr(merged, attr, torch.cat([getattr(q, attr)[start:end] for q in quantizers],
                                        dim=1).clone())
    merged.weight_groupsize = groupsize
    merged._ready = all(q.ready() for q in quantizers)
    return merged


def fake_quantize_grouped(quantizers, weight, groupsize):
    """gptq_utils/common_utils.py:33-44: round-to-nearest of ``weight``
    (B, R, C) with group k's quantizer on columns [k·g, (k+1)·g) (all columns
    with ``groupsize == -1``).

    One ``g2ptq_fake_quantize`` launch over a (B·R, groups) parameter table,
    the per-element arithmetic of each group's ``fake_quantize``."""
    B, R, C = weight.shape
    rows = B * R
    groups = len(quantizers)
    width = C if groupsize == -1 else groupsize
    if groups != -(-C // width):
        raise ValueError(f"{groups} quantizers for {C} columns in groups of {width}")
    q0 = quantizers[0]
    if not all(q.ready() for q in quantizers):
        raise RuntimeError("fake_quantize_grouped: every group quantizer must be fitted")
    scale = torch.cat([q.scale.reshape(rows, 1) for q in quantizers], dim=1).float().contiguous()
    zero = torch.cat([q.zero.reshape(rows, 1) for q in quantizers], dim=1).float().contiguous()
    x = weight.reshape(rows, C).float().contiguous()
    out = torch.empty_like(x)
    _lib.call("g2ptq_fake_quantize", _lib.stream_ptr(x.device), _lib.ptr(x), rows, C, C,
              width, _lib.ptr(scale), _lib.ptr(zero), groups, q0.bits, _lib.ptr(out), C, None, 0,
              None)
    return out.view(B, R, C).to(weight.dtype)


@dataclass(eq=False)
class ChunkSpec:
    """gptq_utils/common_utils.py:47-57: names of same-shaped linears quantized
    by one instance, and their common (rows, columns)."""
    chunk_names: tuple
    rows: int
    columns: int

    @property
    def num_layers(self):
        return len(self.chunk_names)


def build_chunk_specs(subset, layer_bsz, group_key_fn=None):
    """gptq_utils/common_utils.py:60-85: the linears of ``subset`` (name →
    module) bucketed by weight shape (and ``group_key_fn(name)`` when given),
    buckets in order of first appearance, each cut into chunks of at most
    ``layer_bsz`` names in insertion order."""
    buckets = {}
    for name, module in subset.items():
        shape = tuple(module.weight.shape)
        key = shape if group_key_fn is None else (shape, group_key_fn(name))
        buckets.setdefault(key, (shape, []))[1].append(name)
    return [ChunkSpec(chunk_names=tuple(names[i:i + layer_bsz]), rows=shape[0], columns=shape[1])
            for shape, names in buckets.values()
            for i in range(0, len(names), layer_bsz)]
