"""G2PTQ per-layer quantizer on MI355X.

Drop-in for ``G2PTQ`` and ``run_eager`` of gptq_utils/g2ptq_utils.py
(:97-527 of the reference): saliency-weighted per-row-group Hessians, the
trust-region step β and the gradient-compensated lazy-batch sweep, all in
libg2ptq_hip.so.

The trust region needs ``A⁻¹`` only through ``Grad·A⁻¹`` and ``diag(A⁻¹)``; with
``A⁻¹ = UᵀU`` these are ``(Grad·Uᵀ)·U`` and the column norms of ``U``, so no
explicit inverse is formed, and ``GHinv = Z·U = β·Grad·A⁻¹`` needs no third
product (g2ptq_utils.py:459-476 forms A⁻¹ and three dense products).
"""
import torch

from . import _core, _lib
from .common_utils import fake_quantize_grouped
from ._stage import (KIND_WEIGHTED, bump, lazy_counter, single_batch_stager, staged_attr,
                     stager_for)
from .compressed_tensors_utils import compress_layers
from .gptq_utils import _compensate
from .graph_utils import run_graph, validate_tensors


def run_eager(weight, hinv, scale, zero, z, ghinv, maxq, backend, int_weight=None, error=None,
              weight_raw=None, approx_beta=0.0):
    """gptq_utils/g2ptq_utils.py:97-126 (transposed block layout (B, bs, R));
    ``ghinv`` is updated in place like the reference's block-local clone."""
    tensors = [weight, hinv, scale, zero, z, ghinv, int_weight, error]
    if weight_raw is not None:
        tensors.append(weight_raw)
    validate_tensors(f"{backend} G2PTQ", *tensors)
    _core.check_backend(backend)
    if approx_beta:
        raise NotImplementedError("--approx_grad is only implemented for --gptq_backend torch")
    B, bs, R = weight.shape
    _lib.call("g2ptq_block_sweep", _core.stream(), _lib.VARIANT_G2PTQ, B, bs, R, int(maxq),
              _lib.ptr(weight), _lib.ptr(hinv), None, _lib.ptr(scale), _lib.ptr(zero),
              _lib.ptr(z), _lib.ptr(ghinv), None, _lib.ptr(int_weight), _lib.ptr(error), None)
    return weight, int_weight, error


class G2PTQ:
    """gptq_utils/g2ptq_utils.py:129-527."""

    def __init__(self, layers, saliencies, gradients, num_groups: int,
                 offload_hessians: bool = False, approx_grad_beta: float = 0.0):
        self.layers = layers
        self.num_layers = len(layers)
        self.offload_hessians = offload_hessians
        self.approx_grad_beta = approx_grad_beta
        if approx_grad_beta:
            raise NotImplementedError("--approx_grad is only implemented for --gptq_backend torch")
        weight = layers[0].weight
        self.dev = weight.device
        self.rows, self.columns = weight.shape
        self.num_groups = num_groups
        self.saliencies = []
        for saliency in saliencies:
            self.saliencies.append([s.float() for s in saliency] if saliency is not None else None)
        H_device = "cpu" if offload_hessians else self.dev
        self.gradients = _core.alloc((self.num_layers, self.rows, self.columns), H_device)
        for b, gradient in enumerate(gradients):
            if gradient is not None and isinstance(gradient, torch.Tensor):
                self.gradients[b].copy_(gradient, non_blocking=True)
        self.H = _core.alloc((self.num_layers, self.num_groups, self.columns, self.columns),
                             H_device)
        self.act_square = torch.zeros((self.num_layers, self.columns), device=self.dev)
        self.index = torch.tensor([0] * self.num_layers, device=self.dev)
        self.total_tokens = torch.tensor([0] * self.num_layers, device=self.dev)
        self._k = [0] * self.num_layers
        self._k_flushed = [0] * self.num_layers  # batches already folded into H
        self._tt = [0] * self.num_layers
        self._stagers = [None] * self.num_layers
        assert self.rows % self.num_groups == 0, (
            f"Number of rows ({self.rows}) must be divisible by num_groups ({self.num_groups})")

    # ``H`` reads fold the staged calibration tokens into it first.  Each
    # batch's tokens are staged with their 1/T_b folded in, so a flush after
    # k batches (k₀ of them already in H) is H = (k₀/k)·H + (1/k)·Σ staged,
    # the reference's running per-batch mean.
    H = staged_attr("H")
    index = lazy_counter("index")
    total_tokens = lazy_counter("total_tokens")

    def _flush_staged(self, idx=None):
        stagers = getattr(self, "_stagers", None)
        if not stagers:
            return
        for i in (range(self.num_layers) if idx is None else (idx,)):
            st = stagers[i]
            if st is None or st.k == 0:
                continue
            k, k0 = self._k[i], self._k_flushed[i]
            st.flush(self._H[i], _core.f32(1 / k), _core.f32(k0 / k))
            self._k_flushed[i] = k

    def _maybe_onload_hessian_grad(self, hessian=True, gradients=False):
        """g2ptq_utils.py:172-180."""
        names = ("H",) if hessian else ()
        if gradients:
            names += ("gradients",)
        return _core.onload_attrs(self, names, enabled=self.offload_hessians, device=self.dev)

    @torch.no_grad()
    def add_batch(self, idx, inp, out):
        """g2ptq_utils.py:182-201: H[g] ← H[g]·k/(k+1) + Σ_t s_tg x xᵀ / (T·(k+1))."""
        X, dt = _core.as_tokens(inp)
        n_tokens = X.shape[0]
        sal = self.saliencies[idx][0].to(self.dev).float()
        del self.saliencies[idx][0]
        if sal.shape != (n_tokens, self.num_groups):
            sal = sal.reshape(n_tokens, self.num_groups)
        sal = sal.contiguous()
        tt = self._tt[idx]
        act_beta = _core.f32(tt / (tt + n_tokens))
        tt += n_tokens
        self._tt[idx] = tt
        act_alpha = _core.f32(1 / tt)
        st = stager_for(self, idx, X.device, KIND_WEIGHTED, self.num_groups, dt)
        if not st.fits(n_tokens):
            self._flush_staged(idx)
            if st.can_stage(n_tokens):
                st.reserve(n_tokens)
        k = self._k[idx] + 1
        if st.fits(n_tokens):
            st.stage(X, S=sal, s_scale=_core.f32(1 / n_tokens), act=self.act_square[idx],
                     act_alpha=act_alpha, act_beta=act_beta)
        else:
            # a batch larger than the staging budget: update directly
            k0 = self._k_flushed[idx]
            if dt == 0:
                _core.weighted_update(self._H[idx], X, sal, _core.f32(1 / (n_tokens * k)),
                                      _core.f32(k0 / k), self.act_square[idx], act_alpha,
                                      act_beta)
            else:
                one = single_batch_stager(self.columns, X.device, KIND_WEIGHTED,
                                          self.num_groups, dt, n_tokens)
                one.stage(X, S=sal, s_scale=_core.f32(1 / n_tokens), act=self.act_square[idx],
                          act_alpha=act_alpha, act_beta=act_beta)
                one.flush(self._H[idx], _core.f32(1 / k), _core.f32(k0 / k))
            self._k_flushed[idx] = k
        self._k[idx] = k
        bump(self, "index", idx, 1)
        bump(self, "total_tokens", idx, n_tokens)

    def _run_compensation_block(self, weight, hinv, scale, zero, z, ghinv, backend, graph,
                                weight_raw=None):
        """g2ptq_utils.py:203-250."""
        quantizer = self.quantizer[0]
        weight = weight.transpose(1, 2).contiguous()
        params = {
            "weight": weight,
            "hinv": hinv.contiguous(),
            "scale": scale.transpose(1, 2).contiguous(),
            "zero": zero.transpose(1, 2).contiguous(),
            "z": z.transpose(1, 2).contiguous(),
            "ghinv": ghinv.transpose(1, 2).contiguous(),
            "maxq": quantizer.maxq,
            "backend": backend,
            "int_weight": torch.empty_like(weight),
            "error": torch.empty_like(weight),
        }
        names = ("weight", "hinv", "scale", "zero", "z", "ghinv")
        if graph:
            out = run_graph(run_eager, params, input_names=names,
                            output_names=("weight", "int_weight", "error"),
                            name="G2PTQ compensation block")
        else:
            out = run_eager(**params)
        return tuple(t.transpose(1, 2).contiguous() for t in out)

    def _run_compensation(self, W, Hinv, Z, GHinv, blocksize, groupsize, static_groups,
                          qparam_perm, backend, graph, H_diag=None):
        """g2ptq_utils.py:252-347 (GHinv receives the block-tail updates in place)."""
        _core.check_backend(backend)
        flags = torch.zeros(1, dtype=torch.int32, device=W.device)
        out = _compensate(_lib.VARIANT_G2PTQ, self.quantizer, W, Hinv, blocksize, groupsize,
                          static_groups, qparam_perm, flags, graph, Z=Z.contiguous(), GH=GHinv,
                          H_diag=H_diag)
        self._last_flags = flags
        return out

    def fasterquant(self, blocksize=128, percdamp=0.01, groupsize=-1, actorder=False,
                    static_groups=False, enable_gradient_update=True, alpha=0.0,
                    export_compressed_tensors=False, backend="hip", graph=False):
        """g2ptq_utils.py:349-519."""
        _core.check_backend(backend)
        W = _core.stack_weights_f32(self.layers)
        B, R, C = W.shape
        G = self.num_groups
        Rg = R // G
        W_flat = W.view(B * R, C)
        W_sub = W.view(B * G, Rg, C)
        grads = self.gradients.view(B * G, Rg, C).to(self.dev, copy=True)
        flags = torch.zeros(1, dtype=torch.int32, device=self.dev)
        gradient_step = bool(enable_gradient_update and alpha > 0)
        with self._maybe_onload_hessian_grad():
            H_sub = self.H.view(B * G, C, C)
            H_diag = _core.hessian_diag(H_sub, self.quantizer[0].hclip)
            _core.fit_static_params(self.quantizer, W_flat, groupsize, static_groups, flags,
                                    H_diag)
            _core.prepare_hessian(H_sub, W_sub, Grad=grads)
            Q_sub = None
            if gradient_step:
                if groupsize != -1 and not static_groups:
                    for i, q in enumerate(self.quantizer):
                        q.find_params(W_sub[:, :, i * groupsize:(i + 1) * groupsize]
                                      .reshape(B * R, -1), _flags=flags)
                Q_sub = fake_quantize_grouped(self.quantizer, W_sub, groupsize).contiguous()
            perm = invperm = None
            if actorder:
                perm, invperm = _core.act_order(self.act_square, 1)
                W_sub = _core.permute_cols(W_sub, perm)
                H_sub.copy_(_core.permute_sym(H_sub, perm))
                grads = _core.permute_cols(grads, perm)
                if H_diag is not None:
                    H_diag = _core.permute_cols(H_diag, perm)
            Hinv = self._factor(H_sub, percdamp, bool(actorder))
            if Q_sub is not None and actorder:
                Q_sub = _core.permute_cols(Q_sub, perm)
        if gradient_step:
            beta = torch.empty(B * G * Rg, device=self.dev)
            Z = torch.empty_like(W_sub)
            GH = torch.empty_like(W_sub)
            ws = _lib.workspace(_lib.query_size("g2ptq_trust_region_workspace", B * G, Rg, C),
                                self.dev)
            _lib.call("g2ptq_trust_region", _core.stream(), _lib.ptr(grads), _lib.ptr(Hinv),
                      _lib.ptr(Q_sub), _lib.ptr(W_sub), B * G, Rg, C, _core.f32(alpha), 1,
                      _lib.ptr(beta), _lib.ptr(Z), _lib.ptr(GH), _lib.ptr(ws), ws.numel())
            # the per-row step of the last call, (B·G, R/G), for inspection (the
            # reference keeps it local)
            self._beta = beta.view(B * G, Rg)
            Q, W_int, Scale = _compensate(_lib.VARIANT_G2PTQ, self.quantizer, W_sub, Hinv,
                                          blocksize, groupsize, static_groups,
                                          perm if static_groups and actorder else None, flags,
                                          graph, Z=Z, GH=GH, H_diag=H_diag)
        else:
            # β = 0 ⇒ Z = GHinv = 0 and the G2PTQ sweep reduces, operation for
            # operation, to the GPTQ sweep.
            self._beta = None
            Q, W_int, Scale = _compensate(_lib.VARIANT_GPTQ, self.quantizer, W_sub, Hinv,
                                          blocksize, groupsize, static_groups,
                                          perm if static_groups and actorder else None, flags,
                                          graph, H_diag=H_diag)
        if actorder:
            Q = _core.permute_cols(Q, invperm)
            W_int = _core.permute_cols(W_int, invperm)
            Scale = _core.permute_cols(Scale, invperm)
        Q = Q.view(B, R, C)
        if export_compressed_tensors:
            compress_layers(self.layers, Scale.view(B, R, C), W_int.view(B, R, C),
                            self.quantizer[0].bits, groupsize, C)
        _core.write_back(self.layers, Q, flags)
        _core.finish(flags)

    def _factor(self, H_sub, percdamp, actorder):
        """The dampened inverse-Cholesky factor of the prepared Hessians.

        The α autotune (g2ptq_utils.py:1481-1577) re-runs ``fasterquant`` for
        every α with the Hessians restored in between: U depends on the
        prepared H and the damp only, not on α (only the trust-region β
        does), so it is kept with a copy of the H it came from and reused
        while that H matches exactly (one device comparison instead of a
        factorization).  Not used with offloaded Hessians, whose point is to
        keep C² matrices off the device.
        """
        if self.offload_hessians:
            return _core.factor(H_sub, percdamp)[0]
        key = (percdamp, actorder)
        cache = getattr(self, "_factor_cache", None)
        if cache is not None and cache[0] == key and cache[1].shape == H_sub.shape \
                and torch.equal(cache[1], H_sub):
            return cache[2]
        self._factor_cache = None
        U, _ = _core.factor(H_sub, percdamp)
        self._factor_cache = (key, H_sub.clone(), U)
        return U

    def free(self):
        """g2ptq_utils.py:521-527."""
        self._factor_cache = None
        self.H = None
        self.Losses = None
        self.gradients = None
        self.saliencies = None
        self.act_square = None
        _lib.release_workspaces()
