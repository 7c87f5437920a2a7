"""Tensor validation and HIP-graph capture of compensation calls.

Drop-in for gptq_utils/graph_utils.py:12-106 of the reference.  ``run_graph``
captures ``run_eager(**params)`` into a HIP graph once per (shapes, dtypes,
constants) key and replays it with the current inputs copied in and the
outputs copied out, exactly like the reference's CUDA-graph cache.
"""
import torch

_GRAPH_CACHE = {}


def validate_tensors(description, *tensors):
    """gptq_utils/graph_utils.py:12-20 (same exception types and messages)."""
    if any(t is None or not t.is_cuda for t in tensors):
        raise RuntimeError(f"{description} requires every tensor to be on CUDA.")
    device = tensors[0].device
    if any(t.device != device for t in tensors):
        raise ValueError(f"{description} requires every tensor on the same device.")
    if any(not t.is_contiguous() for t in tensors):
        raise ValueError(f"{description} requires contiguous tensors.")
    return device


def _graph_key(name, run_eager, params, input_names, output_names, device):
    index = device.index if device.index is not None else torch.cuda.current_device()
    tensors = tuple((k, tuple(v.shape), v.dtype) for k, v in params.items()
                    if isinstance(v, torch.Tensor))
    constants = tuple((k, v) for k, v in params.items() if not isinstance(v, torch.Tensor))
    return (name, run_eager, index, tensors, constants, tuple(input_names), tuple(output_names))


def run_graph(run_eager, params, *, input_names, output_names, name):
    """gptq_utils/graph_utils.py:53-101."""
    tensor_params = [v for v in params.values() if isinstance(v, torch.Tensor)]
    device = validate_tensors(f"HIP Graph {name}", *tensor_params)
    key = _graph_key(name, run_eager, params, input_names, output_names, device)
    with torch.cuda.device(device):
        state = _GRAPH_CACHE.get(key)
        if state is None:
            static = {k: (torch.empty_like(v) if isinstance(v, torch.Tensor) else v)
                      for k, v in params.items()}
            for n in input_names:
                static[n].copy_(params[n])
            current = torch.cuda.current_stream(device)
            warm = torch.cuda.Stream(device=device)
            warm.wait_stream(current)
            with torch.cuda.stream(warm):
                run_eager(**static)
            current.wait_stream(warm)
            for n in input_names:
                static[n].copy_(params[n])
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                run_eager(**static)
            state = {"graph": graph, "params": static}
            _GRAPH_CACHE[key] = state
        for n in input_names:
            state["params"][n].copy_(params[n])
        state["graph"].replay()
        for n in output_names:
            params[n].copy_(state["params"][n])
    return tuple(params[n] for n in output_names)


def clear_graph_cache():
    """gptq_utils/graph_utils.py:104-106."""
    _GRAPH_CACHE.clear()
