"""Calibration capture feeding ``add_batch``.

The reference's drivers hook three caches into a block's forward and backward
passes; these are drop-ins with the same constructors, hook methods and the
attributes the drivers read (``fp_cache``, ``saliency_cache``,
``gradients_cache``):

- ``FPInputsCache`` (gptq_utils/gptaq_utils.py:442-555): the full-precision
  input of every quantizable linear, the X_fp stream of ``GPTAQ.add_batch``.
- ``SaliencyCache`` (gptq_utils/g2ptq_utils.py:586-681): per batch and loss,
  the mean of grad² over G consecutive channel groups of each linear's output
  gradient — the saliencies of ``G2PTQ`` / ``GPTQGuided``.
- ``GradientCache`` (gptq_utils/g2ptq_utils.py:684-766): per loss, the
  per-token running mean of each linear's weight gradient — ``G2PTQ``'s
  gradients.

How they are built here:

- The inputs of a block stay in HBM (288 GB holds a block's calibration
  inputs at the benchmark sizes) unless ``offload_inps``; then each
  shared-input group owns one page-locked host slab that the group's batches
  fill in arrival order through a copy stream, and a member's k-th batch is the
  slab's k-th batch (the member that fires first for a batch copies it, the
  others take the same rows after checking it is the same tensor).
- The per-batch reductions are HIP kernels: ``g2ptq_group_mean_square`` for a
  saliency batch, ``g2ptq_running_mean_update`` (in place) for a gradient.
- Per-loss results live in ``_LossTable`` objects; summarizing folds them with
  the loss weights in the weights' order (w₁·t₁ + w₂·t₂ + …, each product and
  sum rounded once in fp32, as the reference's Python ``sum`` does).
"""
import contextlib
import functools
import gc

import numpy as np
import torch

from . import _lib

_DTYPE_CODE = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


def _release_memory():
    """Drop unreachable tensors and return the allocator's cached blocks
    (what utils/memory_utils.cleanup_memory does for the reference)."""
    gc.collect()
    if torch.cuda.is_available():
        torch.cuda.empty_cache()


def _dtype_code(t):
    code = _DTYPE_CODE.get(t.dtype)
    if code is None:
        raise NotImplementedError(f"calibration statistics of {t.dtype} tensors")
    return code


def _lookup(modules, name):
    """A linear by name; wrapped linears register as ``<name>.module``."""
    m = modules.get(name)
    return m if m is not None else modules.get(name + ".module")


class _Hooks:
    """Handles of registered hooks, removed together."""

    def __init__(self):
        self.handles = []

    def forward(self, modules, names, fn):
        for name in names:
            self.handles.append(_lookup(modules, name).register_forward_hook(
                functools.partial(fn, name=name)))

    def remove(self):
        while self.handles:
            self.handles.pop().remove()


# ---------------------------------------------------------------------------
# Full-precision inputs (GPTAQ's X_fp)
# ---------------------------------------------------------------------------

class _Slab:
    """Token rows of one shared-input group, batch after batch, in a host buffer.

    ``take(k, x, name)`` returns the rows of the group's k-th batch: a member
    asking for a batch nobody has stored yet stores ``x`` (k must be the next
    batch); a member asking for a stored batch gets its rows after a check that
    it received the very tensor the first member did."""

    def __init__(self, members, rows, features, dtype):
        self.members = members
        self.buffer = torch.zeros(rows, features, dtype=dtype,
                                  pin_memory=torch.cuda.is_available())
        self.filled = 0
        self.batches = []      # row views of the buffer, one per batch
        self.origins = []      # (address, shape) of the tensor each batch came from
        self._stream = None
        self._pending = []     # events of the device→host copies in flight

    def take(self, k, x, name):
        origin = (x.data_ptr(), tuple(x.shape))
        if k < len(self.batches):
            if self.origins[k] != origin:
                raise AssertionError(
                    f"shared-input group {self.members} member {name!r} received a different "
                    f"tensor {origin} than the member that fired first {self.origins[k]}; the "
                    "group was declared as sharing one input tensor")
            return self.batches[k]
        n = x.shape[0]
        if self.filled + n > self.buffer.shape[0]:
            raise AssertionError(f"FP input buffer for group {self.members} overflowed "
                                 f"({self.filled + n} > {self.buffer.shape[0]})")
        rows = self.buffer[self.filled:self.filled + n]
        self._store(rows, x)
        self.filled += n
        self.batches.append(rows)
        self.origins.append(origin)
        return rows

    # device→host copies allowed in flight before the oldest is waited for
    # (utils/offload_utils.py:60,114-117 bounds them the same way)
    MAX_INFLIGHT = 2

    def _store(self, rows, x):
        if not x.is_cuda:
            rows.copy_(x)
            return
        # The copy runs on a stream of its own, after the work that produced x,
        # so the forward pass is not held up by the device→host transfer.  x's
        # block stays reserved for the copy stream (record_stream), so the
        # allocator cannot hand it out again before the copy has read it; a
        # caller that writes into x itself must first wait for settle().
        if self._stream is None:
            self._stream = torch.cuda.Stream(device=x.device)
        self._stream.wait_stream(torch.cuda.current_stream(x.device))
        with torch.cuda.stream(self._stream):
            rows.copy_(x, non_blocking=True)
            x.record_stream(self._stream)
            done = torch.cuda.Event()
            done.record(self._stream)
        self._pending.append(done)
        while len(self._pending) > self.MAX_INFLIGHT:
            self._pending.pop(0).synchronize()

    def settle(self):
        """Wait until every stored batch has reached the host buffer."""
        while self._pending:
            self._pending.pop(0).synchronize()


class FPInputsCache:
    """gptq_utils/gptaq_utils.py:442-555: ``fp_cache[name]`` lists the 2-D
    full-precision inputs of linear ``name``, one per calibration batch.
    Kept in HBM as the forward pass produced them, or, with ``offload_inps``,
    copied into host slabs of ``nsamples·seqlen`` rows shared by each
    ``shared_input_groups`` group (tuples of names; names outside this cache
    are ignored, a name in no group forms its own)."""

    def __init__(self, sequential, modules, nsamples, seqlen, dtype, offload_inps=False,
                 shared_input_groups=None):
        self.names = [n for stage in sequential for n in stage]
        self.offload_inps = offload_inps
        self.fp_cache = {n: [] for n in self.names}
        self._hooks = _Hooks()
        self.slabs = {}        # first member's name -> _Slab
        self._slab_of = {}     # name -> its group's _Slab
        if not offload_inps:
            return
        known = set(self.names)
        groups = [tuple(n for n in g if n in known) for g in (shared_input_groups or ())]
        grouped = {n for g in groups for n in g}
        groups = [g for g in groups if g] + [(n,) for n in self.names if n not in grouped]
        for members in groups:
            widths = {_lookup(modules, n).weight.shape[1] for n in members}
            if len(widths) != 1:
                raise AssertionError(
                    f"shared-input group {members} disagrees on in_features {widths}; "
                    "linears of different input widths cannot share an input tensor")
            slab = _Slab(members, nsamples * seqlen, widths.pop(), dtype)
            self.slabs[members[0]] = slab
            for n in members:
                self._slab_of[n] = slab

    @property
    def handles(self):
        return self._hooks.handles

    def cache_fp_input(self, m, inp, out, name):
        """Forward hook of linear ``name``: record this batch's input."""
        x = inp[0].detach()
        x = x.reshape(-1, x.shape[-1])
        batches = self.fp_cache[name]
        if self.offload_inps:
            x = self._slab_of[name].take(len(batches), x, name)
        batches.append(x)

    def add_hook(self, full):
        self._hooks.forward(full, self.names, self.cache_fp_input)

    def clear_hook(self):
        """Remove the hooks; the offloaded batches are on the host afterwards."""
        self._hooks.remove()
        for slab in self.slabs.values():
            slab.settle()

    def clear_cache(self):
        for slab in self.slabs.values():
            slab.settle()
        self.fp_cache = {}
        self.slabs = {}
        self._slab_of = {}
        _release_memory()


# ---------------------------------------------------------------------------
# Per-loss tables and the loss-weighted fold
# ---------------------------------------------------------------------------

class _LossTable:
    """One linear's results per loss type, in the order the losses first appear."""

    def __init__(self):
        self.by_loss = {}

    def __contains__(self, loss):
        return loss in self.by_loss

    def get(self, loss, default=None):
        return self.by_loss.get(loss, default)

    def put(self, loss, value):
        self.by_loss[loss] = value

    def weighted(self, loss_weights):
        """(weight, value) for every loss of ``loss_weights`` present, in its order."""
        return [(w, self.by_loss[l]) for l, w in loss_weights.items() if l in self.by_loss]


def _fold(pairs):
    """w₁·t₁ + w₂·t₂ + … with every product and sum rounded once (no fused
    multiply-add), the arithmetic of the reference's ``sum(w * t ...)``."""
    (w, t), rest = pairs[0], pairs[1:]
    acc = t * w
    for w, t in rest:
        acc = acc + t * w
    return acc


# ---------------------------------------------------------------------------
# Output-gradient saliencies (G2PTQ / GuidedQuant)
# ---------------------------------------------------------------------------

def group_mean_square(grad, num_groups):
    """``grad.float().pow(2).view(n, G, -1).mean(-1)`` of a (…, hidden) GPU
    tensor, in one HIP reduction (n = tokens, G consecutive channel groups)."""
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
    """gptq_utils/g2ptq_utils.py:586-681.  ``saliency_cache[name]`` maps a loss
    type to the list of per-batch (tokens, G) saliencies; after
    ``summarize_saliency`` it is the list of loss-weighted per-batch tensors."""

    def __init__(self, names, num_groups):
        self.names = names
        self.num_groups = num_groups
        self.outs = {n: 0 for n in names}
        self._tables = {n: _LossTable() for n in names}
        self.saliency_cache = {n: self._tables[n].by_loss for n in names}
        self._hooks = _Hooks()
        self.hooks_enabled = False

    @property
    def handles(self):
        return self._hooks.handles

    def cache_saliency(self, module, inp, out, name):
        """Forward hook: keep the linear's output for the backward pass."""
        self.outs[name] = out

    def grad_hook(self, grad, name, loss_type):
        """One batch's output gradient → its (tokens, G) mean of squares."""
        if not self.hooks_enabled:
            return
        table = self._tables[name]
        batches = table.get(loss_type)
        if batches is None:
            batches = []
            table.put(loss_type, batches)
        batches.append(group_mean_square(grad, self.num_groups))

    def backward(self, loss_tensor, loss_type="block", retain_graph=True):
        """Differentiate ``loss_tensor`` w.r.t. every kept output and record
        the saliencies under ``loss_type``."""
        kept = [(n, self.outs[n]) for n in self.names if torch.is_tensor(self.outs[n])]
        if not kept:
            return
        self.hooks_enabled = True
        try:
            grads = torch.autograd.grad(loss_tensor, [o for _, o in kept],
                                        retain_graph=retain_graph, allow_unused=True)
            for (name, _), grad in zip(kept, grads):
                if grad is not None:
                    self.grad_hook(grad, name=name, loss_type=loss_type)
        finally:
            self.hooks_enabled = False

    def summarize_saliency(self, loss_weights):
        """Fold the losses of ``loss_weights`` ({loss: weight}) batch by batch."""
        for name in self.names:
            table = self._tables[name]
            pairs = table.weighted(loss_weights)
            counts = {l: len(table.get(l)) for l in loss_weights if l in table}
            if len(set(counts.values())) > 1:
                raise AssertionError(
                    f"Saliency for '{name}' has mismatched per-loss batch counts: {counts}")
            n = len(pairs[0][1]) if pairs else 0
            self.saliency_cache[name] = [_fold([(w, batches[i]) for w, batches in pairs])
                                         for i in range(n)]

    def set_forward_hook(self, full):
        self._hooks.forward(full, self.names, self.cache_saliency)

    def clear_hook(self):
        self._hooks.remove()
        self.hooks_enabled = False

    def clear_cache(self):
        self._tables = {n: _LossTable() for n in self.names}
        self.saliency_cache = {n: self._tables[n].by_loss for n in self.names}
        self.outs = {n: 0 for n in self.names}
        _release_memory()


# ---------------------------------------------------------------------------
# Weight gradients (G2PTQ)
# ---------------------------------------------------------------------------

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


class _RunningMean:
    """Σ_k grad_k / (n_k · K) over K batches, updated in place on the device."""

    def __init__(self):
        self.value = None
        self.count = 0

    def update(self, grad, n_tokens):
        self.value = running_mean_update(self.value, grad, n_tokens, self.count)
        self.count += 1


class GradientCache:
    """gptq_utils/g2ptq_utils.py:684-766.  ``gradients_cache[name]`` maps a
    loss type to the running per-token mean of the linear's weight gradient;
    after ``summarize_gradients`` it is their loss-weighted sum (0 when none)."""

    def __init__(self, names, num_groups):
        self.names = names
        self.num_groups = num_groups
        self.current_batch_tokens = {}
        self._means = {n: {} for n in names}      # name -> loss -> _RunningMean
        self.gradients_cache = {n: {} for n in names}
        self._hooks = _Hooks()
        self.hooks_enabled = False

    @property
    def handles(self):
        return self._hooks.handles

    @property
    def index(self):
        """Batches accumulated per name and loss."""
        return {n: {l: m.count for l, m in per.items()} for n, per in self._means.items()}

    def forward_hook(self, module, inp, out, name):
        """Forward hook: the batch's token count (rows of the flattened input)."""
        x = inp[0]
        self.current_batch_tokens[name] = x.numel() // x.shape[-1]

    def cache_gradient(self, grad, name, loss_type):
        """Weight-gradient hook: fold this batch into the loss's running mean."""
        if not self.hooks_enabled:
            return
        mean = self._means[name].get(loss_type)
        if mean is None:
            mean = self._means[name][loss_type] = _RunningMean()
        mean.update(grad, self.current_batch_tokens[name])
        self.gradients_cache[name][loss_type] = mean.value

    def summarize_gradients(self, loss_weights):
        for name in self.names:
            pairs = [(w, self._means[name][l].value) for l, w in loss_weights.items()
                     if l in self._means[name]]
            self.gradients_cache[name] = _fold(pairs) if pairs else 0

    def set_forward_hook(self, full):
        self._hooks.forward(full, self.names, self.forward_hook)

    @contextlib.contextmanager
    def set_backward_hook(self, full, loss_type="block"):
        """Weight-gradient hooks on every linear for the duration of one backward."""
        hooks = [_lookup(full, n).weight.register_hook(
            functools.partial(self.cache_gradient, name=n, loss_type=loss_type))
            for n in self.names]
        self.hooks_enabled = True
        try:
            yield
        finally:
            self.hooks_enabled = False
            for h in hooks:
                h.remove()

    def clear_hook(self):
        self._hooks.remove()
        self.hooks_enabled = False

    def clear_cache(self):
        self._means = {n: {} for n in self.names}
        self.gradients_cache = {n: {} for n in self.names}
        _release_memory()
