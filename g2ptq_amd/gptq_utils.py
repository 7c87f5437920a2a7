"""GPTQ per-layer quantizer on MI355X.

Drop-in for the ``GPTQ`` class and ``run_eager`` of gptq_utils/gptq_utils.py
(:67-359 of the reference): same constructor, attributes and methods, with a
``"hip"`` backend.  ``add_batch`` accumulates the Hessian with the bf16 MFMA
Gram kernel, ``fasterquant`` runs the dampened inverse-Cholesky factor and
the fused lazy-batch compensation in libg2ptq_hip.so.
"""
import collections

import torch

from . import _core, _lib
from ._stage import (DTYPE_BF16, KIND_GPTQ, bump, lazy_counter, single_batch_stager, staged_attr,
                     stager_for)
from .compressed_tensors_utils import compress_layers
from .graph_utils import run_graph, validate_tensors


def run_eager(weight, hinv, scale, zero, maxq, backend, int_weight=None, error=None):
    """gptq_utils/gptq_utils.py:67-90 — one prepared block on the transposed
    layout (B, bs, R); outputs written in place and returned."""
    validate_tensors(f"{backend} GPTQ", weight, hinv, scale, zero, int_weight, error)
    _core.check_backend(backend)
    B, bs, R = weight.shape
    _lib.call("g2ptq_block_sweep", _core.stream(), _lib.VARIANT_GPTQ, B, bs, R, int(maxq),
              _lib.ptr(weight), _lib.ptr(hinv), None, _lib.ptr(scale), _lib.ptr(zero), None, None,
              None, _lib.ptr(int_weight), _lib.ptr(error), None)
    return weight, int_weight, error


class GPTQ:
    """gptq_utils/gptq_utils.py:93-359."""

    def __init__(self, layers, offload_hessians: bool = False):
        self.layers = layers
        self.num_layers = len(layers)
        self.offload_hessians = offload_hessians
        weight = layers[0].weight
        self.dev = weight.device
        self.rows, self.columns = weight.shape
        H_device = "cpu" if offload_hessians else self.dev
        self.H = _core.alloc((self.num_layers, self.columns, self.columns), H_device)
        self.nsamples = torch.tensor([0] * self.num_layers, device=self.dev)
        self._n = [0] * self.num_layers  # host mirror of nsamples (no syncs in add_batch)
        self._n_flushed = [0] * self.num_layers  # samples already folded into H
        self._stagers = [None] * self.num_layers

    # ``H`` reads flush the staged calibration tokens first, so every reader
    # (fasterquant, onload/offload, shared-input copies, callers) sees the
    # Hessian of every batch added so far.
    H = staged_attr("H")
    nsamples = lazy_counter("nsamples")

    def _flush_staged(self, idx=None):
        stagers = getattr(self, "_stagers", None)
        if not stagers:
            return
        src = self.__dict__.setdefault("_gram_src", [None] * self.num_layers)
        flushed = False
        for i in (range(self.num_layers) if idx is None else (idx,)):
            st = stagers[i]
            if st is None or st.k == 0:
                continue
            n, n0 = self._n[i], self._n_flushed[i]
            src[i] = st.flush(self._H[i], _core.sqrt_scale_sq(n), _core.f32(n0 / n))
            self._n_flushed[i] = n
            flushed = True
        if flushed:
            # slots whose Hessians are copies of one Gram result (their own or
            # another stager's, by its serial number): the batched factor
            # factors the first only
            first, alias = {}, {}
            for i, key in enumerate(src):
                if key is not None:
                    if key in first:
                        alias[i] = first[key]
                    else:
                        first[key] = i
            if alias:
                self.__dict__.setdefault("_h_alias", {}).update(alias)

    def _maybe_onload_hessian(self, idx=None):
        """gptq_utils.py:109-113."""
        return _core.onload_attrs(self, ("H",), enabled=self.offload_hessians, device=self.dev)

    def add_batch(self, idx, inp, out):
        """gptq_utils.py:115-126: H ← H·n/(n+t) + (2/(n+t))·XᵀX, t = #sequences.

        A bf16 batch is staged with its source, so that linears fed the same
        input tensors compute their common Gram once (not for the owner of a
        ``SharedInputHessian``, which shares the Hessian itself)."""
        # slot copies made by a shared finalize are stale now
        self.__dict__.pop("_h_alias", None)
        tmp = 1 if inp.dim() == 2 else inp.shape[0]  # a 2-D input is one sequence
        X, dt = _core.as_tokens(inp)
        T = X.shape[0]
        st = stager_for(self, idx, X.device, KIND_GPTQ, 0, dt)
        fits = st.fits(T)
        if not fits:
            self._flush_staged(idx)
            if st.can_stage(T):
                st.reserve(T)
            fits = st.fits(T)
        n = self._n[idx] + tmp
        if fits:
            st.stage(X, share=dt == DTYPE_BF16 and self.__dict__.get("_share_grams", True))
        else:
            # a batch larger than the staging budget: update H directly
            n0 = self._n_flushed[idx]
            if dt == 0:
                _core.hessian_update(self._H[idx], X, _core.sqrt_scale_sq(n), _core.f32(n0 / n))
            else:
                one = single_batch_stager(self.columns, X.device, KIND_GPTQ, 0, dt, T)
                one.stage(X)
                one.flush(self._H[idx], _core.sqrt_scale_sq(n), _core.f32(n0 / n))
            self._n_flushed[idx] = n
        self._n[idx] = n
        bump(self, "nsamples", idx, tmp)

    def _run_compensation_block(self, weight, hinv, scale, zero, backend, graph):
        """gptq_utils.py:128-163 — one block in (B, R, bs) layout."""
        quantizer = self.quantizer[0]
        weight = weight.transpose(1, 2).contiguous()
        params = {
            "weight": weight,
            "hinv": hinv.contiguous(),
            "scale": scale.transpose(1, 2).contiguous(),
            "zero": zero.transpose(1, 2).contiguous(),
            "maxq": quantizer.maxq,
            "backend": backend,
            "int_weight": torch.empty_like(weight),
            "error": torch.empty_like(weight),
        }
        if graph:
            out = run_graph(run_eager, params, input_names=("weight", "hinv", "scale", "zero"),
                            output_names=("weight", "int_weight", "error"),
                            name="GPTQ compensation block")
        else:
            out = run_eager(**params)
        return tuple(t.transpose(1, 2).contiguous() for t in out)

    def _run_compensation(self, W, Hinv, blocksize, groupsize, static_groups, qparam_perm,
                          backend, graph, H_diag=None):
        """gptq_utils.py:165-232: the whole lazy-batch loop, natively.

        ``graph=True`` replays the loop from a HIP graph captured per shape.
        """
        _core.check_backend(backend)
        flags = torch.zeros(1, dtype=torch.int32, device=W.device)
        out = _compensate(_lib.VARIANT_GPTQ, self.quantizer, W, Hinv, blocksize, groupsize,
                          static_groups, qparam_perm, flags, graph, H_diag=H_diag)
        self._last_flags = flags  # device-side failure flags, read by the caller's sync
        return out

    def fasterquant(self, blocksize=128, percdamp=0.01, groupsize=-1, actorder=False,
                    static_groups=False, export_compressed_tensors=False, backend="hip",
                    graph=False):
        """gptq_utils.py:234-353."""
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
            _core.prepare_hessian(H, W)
            perm = invperm = None
            if actorder:
                perm, invperm = _core.act_order(H, 0)
                W = _core.permute_cols(W, perm)
                H = _core.permute_sym(H, perm)
                if H_diag is not None:
                    H_diag = _core.permute_cols(H_diag, perm)
            shared = getattr(self, "_shared_factor", None)
            src = self.__dict__.get("_gram_src")
            if shared is None and src and src[0] is not None and all(x == src[0] for x in src):
                shared = _GramFactors(src[0])
            Hinv, _ = _core.factor(H, percdamp, shared, key=bool(actorder),
                                   alias=self.__dict__.pop("_h_alias", None))
        Q, W_int, Scale = _compensate(_lib.VARIANT_GPTQ, self.quantizer, W, Hinv, blocksize,
                                      groupsize, static_groups,
                                      perm if static_groups and actorder else None, flags, graph,
                                      H_diag=H_diag)
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
        """gptq_utils.py:355-359."""
        self.H = None
        self.Losses = None
        self.nsamples = None
        _lib.release_workspaces()


class _GramFactors:
    """The factor cache of Hessians that are copies of one shared Gram result
    (by its serial number): every slot of an instance holding it, and every
    instance, gets the same prepared Hessian, so the first to factor stores U
    and the others reuse it.  The two most recent results are kept."""
    _cache = collections.OrderedDict()

    def __init__(self, serial):
        self.serial = serial

    def cached_factor(self, ck):
        hit = self._cache.get((self.serial, ck))
        if hit is not None:
            self._cache.move_to_end((self.serial, ck))
        return hit

    def store_factor(self, ck, U, damp):
        self._cache[(self.serial, ck)] = (U, damp)
        while len(self._cache) > 2:
            self._cache.popitem(last=False)


def _compensate(variant, quantizers, W, U, blocksize, groupsize, static_groups, qparam_perm,
                flags, graph, P=None, Z=None, GH=None, H_diag=None):
    if not graph:
        return _core.compensate(variant, W, U, quantizers, blocksize, groupsize, static_groups,
                                qparam_perm, flags, P=P, Z=Z, GH=GH, H_diag=H_diag)
    from ._graphs import compensate_graph
    return compensate_graph(variant, W, U, quantizers, blocksize, groupsize, static_groups,
                            qparam_perm, flags, P=P, Z=Z, GH=GH, H_diag=H_diag)
