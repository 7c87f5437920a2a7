"""Calibration capture feeding ``add_batch``.

Drop-ins for the caches the reference's drivers hook into a block's forward
and backward passes:

- ``FPInputsCache`` (gptq_utils/gptaq_utils.py:442-555): the full-precision
  input of every quantizable linear, the X_fp stream of ``GPTAQ.add_batch``;
  linears that receive the identical tensor share one host buffer when
  offloaded.  Kept on the device (the 288 GB of HBM hold the inputs of a
  block at the benchmark sizes) unless ``offload_inps``.
- ``SaliencyCache`` (gptq_utils/g2ptq_utils.py:586-681): per batch, the mean
  of grad² over G channel groups of each linear's output gradient, the
  saliency of ``G2PTQ`` / ``GPTQGuided``; ``g2ptq_group_mean_square``.
- ``GradientCache`` (:684-766): the per-token running mean of each linear's
  weight gradient, ``G2PTQ``'s gradients; ``g2ptq_running_mean_update``.

Hook wiring, autograd and the loss-weighted summaries stay in torch; the
per-batch reductions run in the HIP library.
"""
import contextlib
import functools
import gc

import numpy as np
import torch

from . import _lib

_DTYPE_CODE = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


def _cleanup():
    """utils/memory_utils.cleanup_memory: collect garbage and return cached blocks."""
    gc.collect()
    if torch.cuda.is_available():
        torch.cuda.empty_cache()


def _dtype_code(t):
    code = _DTYPE_CODE.get(t.dtype)
    if code is None:
        raise NotImplementedError(f"calibration statistics of {t.dtype} tensors")
    return code


def _module(full, name):
    return full.get(name, full.get(name + ".module", None))


class FPInputsCache:
    """gptq_utils/gptaq_utils.py:442-555."""

    def __init__(self, sequential, modules, nsamples, seqlen, dtype, offload_inps=False,
                 shared_input_groups=None):
        self.fp_cache = {}
        self.fp_buffers = {}
        self.cursor = {}
        self.names = []
        for names in sequential:
            self.names += names
        self.handles = []
        self.offload_inps = offload_inps
        # group_key -> [remaining members, destination slice, source identity]
        self._pending = {}
        for name in self.names:
            self.fp_cache[name] = []
        self.groups, self.group_of = self._build_shared_input_groups(shared_input_groups)
        if not self.offload_inps:
            return
        total_tokens = nsamples * seqlen
        pin = torch.cuda.is_available()
        for group_key, group in self.groups.items():
            in_features = {_module(modules, n).weight.shape[1] for n in group}
            assert len(in_features) == 1, (
                f"shared-input group {group} disagrees on in_features {in_features}; "
                f"get_shared_input_groups grouped modules that cannot share an input tensor")
            # page-locked, so the write-back below is a DMA at link speed
            self.fp_buffers[group_key] = torch.zeros(total_tokens, in_features.pop(), dtype=dtype,
                                                     pin_memory=pin)
            self.cursor[group_key] = 0

    def _build_shared_input_groups(self, shared_input_groups):
        """gptaq_utils.py:481-493: the layer's groups restricted to this cache's names."""
        in_cache = set(self.names)
        groups, group_of = {}, {}
        for group in (shared_input_groups or ()):
            members = tuple(n for n in group if n in in_cache)
            if not members:
                continue
            groups[members[0]] = members
            for name in members:
                group_of[name] = members[0]
        return groups, group_of

    def cache_fp_input(self, m, inp, out, name):
        """gptaq_utils.py:495-532 (forward hook)."""
        inp = inp[0].detach()
        if len(inp.shape) == 3:
            inp = inp.reshape((-1, inp.shape[-1]))
        if not self.offload_inps:
            self.fp_cache[name].append(inp)
            return
        group_key = self.group_of[name]
        group = self.groups[group_key]
        pending = self._pending.get(group_key)
        identity = (inp.data_ptr(), tuple(inp.shape))
        if pending is not None:
            dst = pending[1]
            assert pending[2] == identity, (
                f"shared-input group {group} member {name!r} received a different tensor "
                f"{identity} than the member that fired first {pending[2]}; "
                f"get_shared_input_groups declared them as sharing an input but they do not")
            pending[0] -= 1
        else:
            n = inp.shape[0]
            cursor = self.cursor[group_key]
            buffer = self.fp_buffers[group_key]
            assert cursor + n <= buffer.shape[0], (
                f"FP input buffer for group {group} overflowed ({cursor + n} > {buffer.shape[0]})")
            dst = buffer[cursor:cursor + n]
            dst.copy_(inp.contiguous())
            self.cursor[group_key] = cursor + n
            pending = self._pending[group_key] = [len(group) - 1, dst, identity]
        self.fp_cache[name].append(dst)
        if pending[0] <= 0:
            del self._pending[group_key]

    def add_hook(self, full):
        for name in self.names:
            self.handles.append(_module(full, name).register_forward_hook(
                functools.partial(self.cache_fp_input, name=name)))

    def clear_hook(self):
        for h in self.handles:
            h.remove()
        self.handles = []

    def clear_cache(self):
        self.fp_cache = {}
        self.fp_buffers = {}
        self.cursor = {}
        self._pending = {}
        _cleanup()


def group_mean_square(grad, num_groups):
    """``grad.float().pow(2).view(n, G, -1).mean(-1)`` of a (…, hidden) GPU tensor."""
    if not grad.is_cuda:
        raise RuntimeError("group_mean_square: the gradient must be a GPU tensor")
    g = grad.reshape(-1, grad.shape[-1])
    n_tokens, hidden = g.shape
    group_size = hidden // num_groups
    if group_size * num_groups != hidden:
        raise RuntimeError(f"shape '[{n_tokens}, {num_groups}, {group_size}]' is invalid for "
                           f"input of size {n_tokens * hidden}")
    if g.stride(-1) != 1:
        g = g.contiguous()
    out = torch.empty(n_tokens, num_groups, device=g.device, dtype=torch.float32)
    _lib.call("g2ptq_group_mean_square", _lib.stream_ptr(g.device), _lib.ptr(g), _dtype_code(g),
              n_tokens, hidden, g.stride(0) if n_tokens > 1 else hidden, num_groups,
              _lib.ptr(out))
    return out


class SaliencyCache:
    """gptq_utils/g2ptq_utils.py:586-681."""

    def __init__(self, names, num_groups):
        self.num_groups = num_groups
        self.saliency_cache = {}
        self.outs = {}
        self.names = names
        for name in self.names:
            self.saliency_cache[name] = {}   # loss -> list of per-batch saliency tensors
            self.outs[name] = 0
        self.handles = []
        self.hooks_enabled = False

    def cache_saliency(self, module, inp, out, name):
        self.outs[name] = out

    def grad_hook(self, grad, name, loss_type):
        """:604-618: (n_tokens, G) mean of grad² per channel group."""
        if not self.hooks_enabled:
            return
        self.saliency_cache[name].setdefault(loss_type, []).append(
            group_mean_square(grad, self.num_groups))

    def summarize_saliency(self, loss_weights):
        """:620-640: one list of per-batch tensors, the loss-weighted sum."""
        for name in self.names:
            per_loss = self.saliency_cache[name]
            present = [(l, w) for l, w in loss_weights.items() if l in per_loss]
            if not present:
                self.saliency_cache[name] = []
                continue
            lengths = [len(per_loss[l]) for l, _ in present]
            assert len(set(lengths)) == 1, (
                f"Saliency for '{name}' has mismatched per-loss batch counts: "
                f"{ {l: len(per_loss[l]) for l, _ in present} }")
            self.saliency_cache[name] = [sum(w * per_loss[l][i] for l, w in present)
                                         for i in range(lengths[0])]

    def set_forward_hook(self, full):
        for name in self.names:
            self.handles.append(_module(full, name).register_forward_hook(
                functools.partial(self.cache_saliency, name=name)))

    def backward(self, loss_tensor, loss_type="block", retain_graph=True):
        """:654-672: gradients of the loss w.r.t. the cached outputs."""
        names = [name for name in self.names if isinstance(self.outs[name], torch.Tensor)]
        if not names:
            return
        self.hooks_enabled = True
        try:
            grads = torch.autograd.grad(loss_tensor, [self.outs[name] for name in names],
                                        retain_graph=retain_graph, allow_unused=True)
            for name, grad in zip(names, grads):
                if grad is not None:
                    self.grad_hook(grad, name=name, loss_type=loss_type)
        finally:
            self.hooks_enabled = False

    def clear_hook(self):
        for h in self.handles:
            h.remove()
        self.handles = []
        self.hooks_enabled = False

    def clear_cache(self):
        for name in self.names:
            self.saliency_cache[name] = {}
            self.outs[name] = 0
        _cleanup()


def running_mean_update(cache, grad, n_tokens, index):
    """``cache·(index/(index+1)) + grad.float()/(n_tokens·(index+1))`` in place
    (``cache`` None: a new tensor, the reference's first call on the int 0).
    Returns the cache tensor."""
    if not grad.is_cuda:
        raise RuntimeError("running_mean_update: the gradient must be a GPU tensor")
    g = grad if grad.is_contiguous() else grad.contiguous()
    first = cache is None
    if first:
        cache = torch.empty(g.shape, device=g.device, dtype=torch.float32)
    elif cache.shape != g.shape or not cache.is_contiguous() or cache.dtype != torch.float32:
        raise RuntimeError("running_mean_update: the cache must be a contiguous fp32 tensor "
                           "of the gradient's shape")
    keep = np.float32(index / (index + 1))
    inv_count = np.float32(1.0) / np.float32(n_tokens * (index + 1))
    _lib.call("g2ptq_running_mean_update", _lib.stream_ptr(g.device), _lib.ptr(cache),
              _lib.ptr(g), _dtype_code(g), g.numel(), float(keep), float(inv_count), int(first))
    return cache


class GradientCache:
    """gptq_utils/g2ptq_utils.py:684-766."""

    def __init__(self, names, num_groups):
        self.num_groups = num_groups
        self.gradients_cache = {}
        self.index = {}
        self.current_batch_tokens = {}
        self.names = names
        for name in self.names:
            self.gradients_cache[name] = {}   # loss -> running-mean gradient tensor
            self.index[name] = {}             # loss -> accumulation count
        self.handles = []
        self.hooks_enabled = False

    def forward_hook(self, module, inp, out, name):
        x = inp[0]
        self.current_batch_tokens[name] = x.numel() // x.shape[-1]

    def cache_gradient(self, grad, name, loss_type):
        """:704-714 (weight-gradient hook)."""
        if not self.hooks_enabled:
            return
        n_tokens = self.current_batch_tokens[name]
        index = self.index[name].get(loss_type, 0)
        cache = self.gradients_cache[name].get(loss_type)
        if cache is not None and not isinstance(cache, torch.Tensor):
            cache = None
        self.gradients_cache[name][loss_type] = running_mean_update(cache, grad, n_tokens, index)
        self.index[name][loss_type] = index + 1

    def summarize_gradients(self, loss_weights):
        """:716-724: one tensor per name, the loss-weighted sum (0 when none)."""
        for name in self.names:
            per_loss = self.gradients_cache[name]
            present = [(l, w) for l, w in loss_weights.items() if l in per_loss]
            self.gradients_cache[name] = (sum(w * per_loss[l] for l, w in present)
                                          if present else 0)

    def set_forward_hook(self, full):
        for name in self.names:
            self.handles.append(_module(full, name).register_forward_hook(
                functools.partial(self.forward_hook, name=name)))

    @contextlib.contextmanager
    def set_backward_hook(self, full, loss_type="block"):
        """:736-755: weight-gradient hooks for the duration of one backward."""
        self.hooks_enabled = True
        handles = []
        for name in self.names:
            handles.append(_module(full, name).weight.register_hook(
                functools.partial(self.cache_gradient, name=name, loss_type=loss_type)))
        try:
            yield
        finally:
            for h in handles:
                h.remove()
            self.hooks_enabled = False

    def clear_hook(self):
        for h in self.handles:
            h.remove()
        self.handles = []
        self.hooks_enabled = False

    def clear_cache(self):
        for name in self.names:
            self.gradients_cache[name] = {}
            self.index[name] = {}
        _cleanup()
