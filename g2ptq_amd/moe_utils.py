"""MoE expert stacking for the checkpoint.

Drop-in for ``MoEMixin.stack_experts`` (utils/models/mixins.py:93-144 of the
reference), which ``ptq.py:133`` calls before saving a quantized MoE model:
per layer, the per-expert ``gate_proj``/``up_proj``/``down_proj`` tensors
become 3-D tensors on the experts container,

    gate_up_proj[_packed|_scale] = stack_e(cat(gate_e, up_e))   (E, 2·I, ·)
    down_proj[_packed|_scale]    = stack_e(down_e)              (E, H, ·)

(``weight_packed=True``: the compressed-tensors buffers ``weight_packed`` /
``weight_scale`` and the ``*_shape`` tensors; otherwise the weights), and the
per-expert modules are dropped.  Every stacked tensor is written by one HIP
launch (``g2ptq_concat``) instead of a cat per expert plus a stack.
"""
from types import MethodType

import torch
from torch import nn

from . import _lib


def stack_cat(groups):
    """``torch.stack([torch.cat(g, dim=0) for g in groups], dim=0)`` for GPU
    tensors, in one launch."""
    parts = [t for g in groups for t in g]
    if not parts:
        raise RuntimeError("stack expects a non-empty TensorList")
    first = parts[0]
    for t in parts:
        if not t.is_cuda or t.device != first.device:
            raise RuntimeError("stack_cat: every tensor must be on the same GPU")
        if t.dtype != first.dtype:
            raise RuntimeError(f"Expected object of scalar type {first.dtype} but got {t.dtype}")
        if t.dim() != first.dim() or t.shape[1:] != first.shape[1:]:
            raise RuntimeError(f"Sizes of tensors must match except in dimension 0. Expected "
                               f"{tuple(first.shape[1:])} but got {tuple(t.shape[1:])}")
    rows = [sum(t.shape[0] for t in g) for g in groups]
    if len(set(rows)) != 1:
        raise RuntimeError(f"stack expects each tensor to be equal size, but got "
                           f"{[rows[0], *first.shape[1:]]} at entry 0 and "
                           f"{[next(r for r in rows if r != rows[0]), *first.shape[1:]]}")
    srcs = [t.contiguous() for t in parts]
    out = torch.empty((len(groups), rows[0], *first.shape[1:]), dtype=first.dtype,
                      device=first.device)
    sizes = [t.numel() * t.element_size() for t in srcs]
    offs = [0]
    for n in sizes:
        offs.append(offs[-1] + n)
    table = torch.tensor([t.data_ptr() for t in srcs] + offs, dtype=torch.int64).to(first.device)
    n = len(srcs)
    _lib.call("g2ptq_concat", _lib.stream_ptr(first.device), table.data_ptr(),
              table.data_ptr() + 8 * n, n, max(sizes), _lib.ptr(out))
    return out


def _stacked_forward(self, hidden_states, top_k_index, top_k_weights):
    # The reference's stacked forward (mixins.py:262-287) reads
    # ``self.gate_up_proj[e].weight`` of a tensor and cannot run either: the
    # stacked layout is what the checkpoint stores, not what the model executes.
    raise NotImplementedError("stacked experts are the checkpoint layout; run the model "
                              "before stack_experts")


def stack_experts(experts, weight_packed=False):
    """utils/models/mixins.py:93-144 (``MoEMixin.stack_experts``)."""
    num_experts = experts.num_experts
    gate_proj = [experts[i].gate_proj for i in range(num_experts)]
    up_proj = [experts[i].up_proj for i in range(num_experts)]
    down_proj = [experts[i].down_proj for i in range(num_experts)]

    def param(groups):
        return nn.Parameter(stack_cat(groups), requires_grad=False)

    if weight_packed:
        experts.gate_up_proj_packed = param(
            [(gate_proj[i].weight_packed, up_proj[i].weight_packed) for i in range(num_experts)])
        experts.down_proj_packed = param([(down_proj[i].weight_packed,) for i in range(num_experts)])
        experts.gate_up_proj_scale = param(
            [(gate_proj[i].weight_scale, up_proj[i].weight_scale) for i in range(num_experts)])
        experts.down_proj_scale = param([(down_proj[i].weight_scale,) for i in range(num_experts)])
        intermediate_dim = int(gate_proj[0].weight_shape[0])
        hidden_dim = int(gate_proj[0].weight_shape[1])
        experts.gate_up_proj_shape = torch.tensor((num_experts, 2 * intermediate_dim, hidden_dim))
        experts.down_proj_shape = torch.tensor((num_experts, hidden_dim, intermediate_dim))
    else:
        experts.gate_up_proj = param(
            [(gate_proj[i].weight, up_proj[i].weight) for i in range(num_experts)])
        experts.down_proj = param([(down_proj[i].weight,) for i in range(num_experts)])

    for i in range(num_experts):
        del experts._modules[str(i)]
    experts.forward = MethodType(_stacked_forward, experts)
