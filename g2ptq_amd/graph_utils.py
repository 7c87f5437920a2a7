"""Tensor validation and graph replay of block-operator calls.

Drop-in for ``validate_tensors``, ``run_graph`` and ``clear_graph_cache`` of
gptq_utils/graph_utils.py:12-106 (same signatures, exception types and
messages).  The reference uses graphs to amortise the two launches per column
of its Triton block operator.  Here a block operator is one sweep launch, and
``fasterquant(graph=True)`` captures the whole native loop instead
(``_graphs.compensate_graph``); ``run_graph`` keeps the per-block API for the
callers and tests that use it:

- calls are grouped by a *signature*: the operator, the call's name, the
  device, and per parameter either (shape, dtype) of a tensor or the value of
  a constant;
- the first call of a signature runs the operator eagerly on the caller's own
  tensors (that is its result, and it loads every kernel before any capture),
  then records a graph of the same call over private twin tensors — recording
  executes nothing, so the twins need no data yet;
- later calls copy the named inputs into the twins, replay, and copy the named
  outputs back, all enqueued on the current stream.
"""
import torch


def validate_tensors(description, *tensors):
    """gptq_utils/graph_utils.py:12-20: every tensor on the GPU (else
    RuntimeError), on one device and contiguous (else ValueError).  Returns
    the device."""
    if any(t is None or not t.is_cuda for t in tensors):
        raise RuntimeError(f"{description} requires every tensor to be on CUDA.")
    device = tensors[0].device
    if any(t.device != device for t in tensors):
        raise ValueError(f"{description} requires every tensor on the same device.")
    if any(not t.is_contiguous() for t in tensors):
        raise ValueError(f"{description} requires contiguous tensors.")
    return device


class _Replay:
    """A recorded call and the twin tensors its graph reads and writes."""

    def __init__(self, fn, params, device):
        self.twins = {k: torch.empty_like(v) if torch.is_tensor(v) else v
                      for k, v in params.items()}
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            fn(**self.twins)

    def __call__(self, params, inputs, outputs):
        for k in inputs:
            self.twins[k].copy_(params[k])
        self.graph.replay()
        for k in outputs:
            params[k].copy_(self.twins[k])


_REPLAYS = {}


def _signature(fn, name, params, inputs, outputs, device):
    def describe(v):
        return ("tensor", tuple(v.shape), v.dtype) if torch.is_tensor(v) else ("value", v)

    index = device.index if device.index is not None else torch.cuda.current_device()
    items = tuple(sorted((k, describe(v)) for k, v in params.items()))
    return fn, name, index, items, frozenset(inputs), frozenset(outputs)


def run_graph(run_eager, params, *, input_names, output_names, name):
    """``run_eager(**params)`` through a replayed graph; the named outputs are
    written into the caller's tensors, which are returned in order
    (gptq_utils/graph_utils.py:53-101)."""
    tensors = [v for v in params.values() if torch.is_tensor(v)]
    device = validate_tensors(f"CUDA Graph {name}", *tensors)
    sig = _signature(run_eager, name, params, input_names, output_names, device)
    with torch.cuda.device(device):
        replay = _REPLAYS.get(sig)
        if replay is None:
            run_eager(**params)
            _REPLAYS[sig] = _Replay(run_eager, params, device)
        else:
            replay(params, input_names, output_names)
    return tuple(params[k] for k in output_names)


def clear_graph_cache():
    """gptq_utils/graph_utils.py:104-106: drop every recorded graph and its twins."""
    _REPLAYS.clear()
