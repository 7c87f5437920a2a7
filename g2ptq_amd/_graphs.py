"""HIP-graph replay of the native compensation loop (``graph=True``).

The reference captures each 128-column block into a CUDA graph to amortise
its 2·bs per-column launches (gptq_utils/graph_utils.py:53-101).  Here the
whole per-layer loop (find_params, sweeps and tail GEMMs for every block) is
captured once per (variant, shapes, group layout, grid) key and replayed with
inputs copied into, and outputs copied out of, the graph's static buffers.
"""
import torch

from . import _core, _lib

_CACHE = {}


def clear():
    _CACHE.clear()


def compensate_graph(variant, W, U, quantizers, blocksize, groupsize, static_groups, qparam_perm,
                     flags, P=None, Z=None, GH=None, H_diag=None):
    B, R, C = W.shape
    dev = W.device
    q0 = quantizers[0]
    grid, norm, shrink = _core.mse_config(q0)
    hd = _core.hclip_rows(quantizers, H_diag, groupsize, static_groups, B * R, C, dev)
    nhd = hd.shape[0] if hd is not None else 0
    stab, ztab, dynamic = _core.param_tables(quantizers, B * R, groupsize, static_groups, dev)
    colgroup = None
    if groupsize != -1 and static_groups and qparam_perm is not None:
        colgroup = (qparam_perm.to(dev).long() // groupsize).to(torch.int32).contiguous()
    key = (variant, tuple(W.shape), blocksize, groupsize, bool(static_groups), colgroup is not None,
           q0.bits, bool(q0.sym), grid, norm, shrink, nhd, P is not None, Z is not None,
           dev.index if dev.index is not None else torch.cuda.current_device())
    live = {"W": W, "U": U, "P": P, "Z": Z, "GH": GH, "stab": stab, "ztab": ztab,
            "colgroup": colgroup, "flags": flags, "hd": hd}
    state = _CACHE.get(key)
    if state is None:
        static = {k: (v.clone() if v is not None else None) for k, v in live.items()}
        static["Q"] = torch.empty_like(W)
        static["W_int"] = torch.empty_like(W)
        static["Scale"] = torch.empty_like(W)
        nbytes = _lib.query_size("g2ptq_compensate_workspace", variant, B, R, C, blocksize)
        static["ws"] = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=dev)

        def launch():
            _lib.call("g2ptq_compensate", _lib.stream_ptr(), variant, B, R, C, blocksize,
                      _lib.ptr(static["W"]), _lib.ptr(static["U"]), _lib.ptr(static["P"]),
                      _lib.ptr(static["Z"]), _lib.ptr(static["GH"]), q0.bits, int(q0.sym),
                      groupsize, int(bool(static_groups)), grid, norm, shrink,
                      _lib.ptr(static["hd"]), nhd, _lib.ptr(static["colgroup"]),
                      _lib.ptr(static["stab"]),
                      _lib.ptr(static["ztab"]), _lib.ptr(static["Q"]), _lib.ptr(static["W_int"]),
                      _lib.ptr(static["Scale"]), _lib.ptr(static["flags"]),
                      _lib.ptr(static["ws"]), static["ws"].numel())

        current = torch.cuda.current_stream(dev)
        warm = torch.cuda.Stream(device=dev)
        warm.wait_stream(current)
        with torch.cuda.stream(warm):
            launch()
        current.wait_stream(warm)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            launch()
        state = {"graph": graph, "static": static}
        _CACHE[key] = state
    static = state["static"]
    for k, v in live.items():
        if v is not None:
            static[k].copy_(v)
    state["graph"].replay()
    W.copy_(static["W"])
    if GH is not None:
        GH.copy_(static["GH"])
    flags.copy_(static["flags"])
    if dynamic:
        stab.copy_(static["stab"])
        ztab.copy_(static["ztab"])
        for i, q in enumerate(quantizers):
            q.scale = stab[i].view(B * R, 1)
            q.zero = ztab[i].view(B * R, 1)
            q._ready = True
    return static["Q"].clone(), static["W_int"].clone(), static["Scale"].clone()
