"""GPTAQ per-layer quantizer on MI355X.

Drop-in for ``GPTAQ`` and ``run_eager`` of gptq_utils/gptaq_utils.py
(:74-399 of the reference).  The asymmetric-calibration cross term
``dXXT = (2/n)(X_fp − X)ᵀX`` is accumulated in the same MFMA pass as the
Hessian; ``P = α·triu(dXXT·Uᵀ, 1)·U`` and the compensation (``+w̃·P`` inside a
block, ``+Q·P`` in the block tail) run in libg2ptq_hip.so.
"""
import torch

from . import _core, _lib
from ._stage import (KIND_GPTAQ, bump, lazy_counter, single_batch_stager, staged_attr,
                     stager_for)
from .compressed_tensors_utils import compress_layers
from .gptq_utils import _compensate
from .graph_utils import run_graph, validate_tensors


def run_eager(weight, hinv, p, scale, zero, maxq, backend, column_weight=None, int_weight=None,
              error=None):
    """gptq_utils/gptaq_utils.py:74-100 (transposed block layout (B, bs, R))."""
    validate_tensors(f"{backend} GPTAQ", weight, hinv, p, scale, zero, column_weight, int_weight,
                     error)
    _core.check_backend(backend)
    B, bs, R = weight.shape
    _lib.call("g2ptq_block_sweep", _core.stream(), _lib.VARIANT_GPTAQ, B, bs, R, int(maxq),
              _lib.ptr(weight), _lib.ptr(hinv), _lib.ptr(p), _lib.ptr(scale), _lib.ptr(zero),
              None, None, _lib.ptr(column_weight), _lib.ptr(int_weight), _lib.ptr(error), None)
    return weight, int_weight, error


class GPTAQ:
    """gptq_utils/gptaq_utils.py:103-399."""

    def __init__(self, layers, offload_hessians: bool = False):
        self.layers = layers
        self.num_layers = len(layers)
        self.offload_hessians = offload_hessians
        weight = layers[0].weight
        self.dev = weight.device
        self.rows, self.columns = weight.shape
        H_device = "cpu" if offload_hessians else self.dev
        self.H = _core.alloc((self.num_layers, self.columns, self.columns), H_device)
        self.dXXT = _core.alloc((self.num_layers, self.columns, self.columns), H_device)
        self.nsamples = torch.tensor([0] * self.num_layers, device=self.dev)
        self._n = [0] * self.num_layers
        self._n_flushed = [0] * self.num_layers  # samples already folded into H / dXXT
        self._stagers = [None] * self.num_layers
        self.fp_inp = [[] for _ in range(self.num_layers)]

    # Reads of H or dXXT fold the staged calibration tokens into both first.
    H = staged_attr("H")
    dXXT = staged_attr("dXXT")
    nsamples = lazy_counter("nsamples")

    def _flush_staged(self, idx=None):
        stagers = getattr(self, "_stagers", None)
        if not stagers:
            return
        for i in (range(self.num_layers) if idx is None else (idx,)):
            st = stagers[i]
            if st is None or st.k == 0:
                continue
            n, n0 = self._n[i], self._n_flushed[i]
            st.flush(self._H[i], _core.sqrt_scale_sq(n), _core.f32(n0 / n), Dx=self._dXXT[i])
            self._n_flushed[i] = n

    def _maybe_onload_hessian(self):
        """gptaq_utils.py:123-128."""
        return _core.onload_attrs(self, ("H", "dXXT"), enabled=self.offload_hessians,
                                  device=self.dev)

    def add_batch(self, idx, inp, out):
        """gptaq_utils.py:130-148 (``fp_inp[idx]`` is a FIFO of (tokens, C) tensors):
        H and dXXT ← ·n/(n+t) + (2/(n+t))·(XᵀX, (X_fp − X)ᵀX), staged."""
        fp = self.fp_inp[idx][0].to(inp.device, non_blocking=True)
        tmp = 1 if inp.dim() == 2 else inp.shape[0]  # a 2-D input is one sequence
        X, dt = _core.as_tokens(inp)
        Xfp, _ = _core.as_tokens(fp.to(inp.dtype))  # the reference's fp_inp.to(inp)
        if Xfp.shape != X.shape:
            raise ValueError(f"fp_inp shape {tuple(Xfp.shape)} != input {tuple(X.shape)}")
        T = X.shape[0]
        st = stager_for(self, idx, X.device, KIND_GPTAQ, 0, dt)
        if not st.fits(T):
            self._flush_staged(idx)
            if st.can_stage(T):
                st.reserve(T)
        n = self._n[idx] + tmp
        if st.fits(T):
            st.stage(X, Xfp)
        else:
            # a batch larger than the staging budget: update directly
            n0 = self._n_flushed[idx]
            if dt == 0:
                _core.gptaq_update(self._H[idx], self._dXXT[idx], X, Xfp, _core.sqrt_scale_sq(n),
                                   _core.f32(n0 / n))
            else:
                one = single_batch_stager(self.columns, X.device, KIND_GPTAQ, 0, dt, T)
                one.stage(X, Xfp)
                one.flush(self._H[idx], _core.sqrt_scale_sq(n), _core.f32(n0 / n),
                          self._dXXT[idx])
            self._n_flushed[idx] = n
        self._n[idx] = n
        bump(self, "nsamples", idx, tmp)
        del self.fp_inp[idx][0]

    def _run_compensation_block(self, weight, hinv, p, scale, zero, backend, graph):
        """gptaq_utils.py:150-191."""
        quantizer = self.quantizer[0]
        weight = weight.transpose(1, 2).contiguous()
        params = {
            "weight": weight,
            "hinv": hinv.contiguous(),
            "p": p.contiguous(),
            "scale": scale.transpose(1, 2).contiguous(),
            "zero": zero.transpose(1, 2).contiguous(),
            "maxq": quantizer.maxq,
            "backend": backend,
            "column_weight": torch.empty(weight.shape[0], weight.shape[2], dtype=weight.dtype,
                                         device=weight.device),
            "int_weight": torch.empty_like(weight),
            "error": torch.empty_like(weight),
        }
        if graph:
            out = run_graph(run_eager, params,
                            input_names=("weight", "hinv", "p", "scale", "zero"),
                            output_names=("weight", "int_weight", "error"),
                            name="GPTAQ compensation block")
        else:
            out = run_eager(**params)
        return tuple(t.transpose(1, 2).contiguous() for t in out)

    def _run_compensation(self, W, Hinv, P, blocksize, groupsize, static_groups, qparam_perm,
                          backend, graph, H_diag=None):
        """gptaq_utils.py:193-261."""
        _core.check_backend(backend)
        flags = torch.zeros(1, dtype=torch.int32, device=W.device)
        out = _compensate(_lib.VARIANT_GPTAQ, self.quantizer, W, Hinv, blocksize, groupsize,
                          static_groups, qparam_perm, flags, graph, P=P.contiguous(),
                          H_diag=H_diag)
        self._last_flags = flags
        return out

    def fasterquant(self, blocksize=128, percdamp=0.01, groupsize=-1, actorder=False,
                    static_groups=False, alpha=0.25, export_compressed_tensors=False,
                    backend="hip", graph=False):
        """gptaq_utils.py:263-391."""
        _core.check_backend(backend)
        W = _core.stack_weights_f32(self.layers)
        B, R, C = W.shape
        W_flat = W.view(B * R, C)
        flags = torch.zeros(1, dtype=torch.int32, device=self.dev)
        with self._maybe_onload_hessian():
            H = self.H
            self.H = None
            H_diag = _core.hessian_diag(H, self.quantizer[0].hclip)
            _core.fit_static_params(self.quantizer, W_flat, groupsize, static_groups, flags,
                                    H_diag)
            _core.prepare_hessian(H, W, Dx=self.dXXT)
            perm = invperm = None
            if actorder:
                perm, invperm = _core.act_order(H, 0)
                W = _core.permute_cols(W, perm)
                H = _core.permute_sym(H, perm)
                self.dXXT.copy_(_core.permute_sym(self.dXXT, perm))
                if H_diag is not None:
                    H_diag = _core.permute_cols(H_diag, perm)
            Hinv, _ = _core.factor(H, percdamp)
            P = torch.empty_like(Hinv)
            ws = _lib.workspace(B * C * C * 4 + 256, self.dev)
            _lib.call("g2ptq_gptaq_p", _core.stream(), _lib.ptr(self.dXXT), _lib.ptr(Hinv), B, C,
                      _core.f32(alpha), _lib.ptr(P), _lib.ptr(ws), ws.numel())
        Q, W_int, Scale = _compensate(_lib.VARIANT_GPTAQ, self.quantizer, W, Hinv, blocksize,
                                      groupsize, static_groups,
                                      perm if static_groups and actorder else None, flags, graph,
                                      P=P, H_diag=H_diag)
        if actorder:
            Q = _core.permute_cols(Q, invperm)
            W_int = _core.permute_cols(W_int, invperm)
            Scale = _core.permute_cols(Scale, invperm)
        if export_compressed_tensors:
            compress_layers(self.layers, Scale.view(B, R, C), W_int.view(B, R, C),
                            self.quantizer[0].bits, groupsize, C)
        _core.write_back(self.layers, Q, flags)
        _core.finish(flags)

    def free(self):
        """gptaq_utils.py:393-399."""
        self.H = None
        self.Losses = None
        self.dXXT = None
        self.nsamples = None
        self.fp_inp = None
        _lib.release_workspaces()
