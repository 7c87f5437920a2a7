"""Group-quantizer bookkeeping and same-shape layer batching.

Drop-in for gptq_utils/common_utils.py:13-85 of the reference (the multi-GPU
helpers ``partition_layers`` / ``broadcast_quantized_param`` are not part of
this single-GPU build).
"""
import copy
from collections import defaultdict
from dataclasses import dataclass

import torch


def make_group_quantizers(quantizer, columns, groupsize):
    """gptq_utils/common_utils.py:13-16 — one independent quantizer per group."""
    num_groups = 1 if groupsize == -1 else (columns + groupsize - 1) // groupsize
    return [copy.deepcopy(quantizer) for _ in range(num_groups)]


def merge_group_quantizers(quantizers, start, end, groupsize):
    """gptq_utils/common_utils.py:19-30 — per-layer (rows, C/g) scale/zero."""
    result = copy.deepcopy(quantizers[0])
    result.scale = torch.cat([q.scale[start:end] for q in quantizers], dim=1).clone()
    result.zero = torch.cat([q.zero[start:end] for q in quantizers], dim=1).clone()
    result.weight_groupsize = groupsize
    result._ready = all(q.ready() for q in quantizers)
    return result


def fake_quantize_grouped(quantizers, weight, groupsize):
    """gptq_utils/common_utils.py:33-44 — RTN of ``weight (B, R, C)`` group by group."""
    flat_rows = weight.shape[0] * weight.shape[1]
    width = weight.shape[-1] if groupsize == -1 else groupsize
    out = []
    for g, quantizer in enumerate(quantizers):
        start = g * width
        end = min(start + width, weight.shape[-1])
        q = quantizer.fake_quantize(weight[:, :, start:end].reshape(flat_rows, end - start))[0]
        out.append(q.reshape(*weight.shape[:2], end - start))
    return torch.cat(out, dim=-1)


@dataclass(eq=False)
class ChunkSpec:
    """gptq_utils/common_utils.py:47-57 — same-shaped modules quantized as one batch."""
    chunk_names: tuple
    rows: int
    columns: int

    @property
    def num_layers(self):
        return len(self.chunk_names)


def build_chunk_specs(subset, layer_bsz, group_key_fn=None):
    """gptq_utils/common_utils.py:60-85 — group by weight shape, chunk by ``layer_bsz``."""
    groups = defaultdict(list)
    for name, module in subset.items():
        key = module.weight.shape
        if group_key_fn is not None:
            key = (key, group_key_fn(name))
        groups[key].append(name)
    specs = []
    for names in groups.values():
        rows, columns = subset[names[0]].weight.shape
        for s in range(0, len(names), layer_bsz):
            specs.append(ChunkSpec(chunk_names=tuple(names[s:s + layer_bsz]), rows=rows,
                                   columns=columns))
    return specs
