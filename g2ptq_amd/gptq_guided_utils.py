"""GuidedQuant per-layer quantizer on MI355X.

Drop-in for ``GPTQGuided`` of gptq_utils/gptq_guided_utils.py (:25-219 of the
reference): saliency-weighted per-row-group Hessians (shared MFMA kernel with
G2PTQ) and GPTQ's compensation, inherited unchanged.
"""
import torch

from . import _core, _lib
from ._stage import KIND_WEIGHTED, bump, lazy_counter, single_batch_stager, stager_for
from .compressed_tensors_utils import compress_layers
from .gptq_utils import GPTQ, _compensate


class GPTQGuided(GPTQ):
    """gptq_utils/gptq_guided_utils.py:25-219."""

    index = lazy_counter("index")

    def __init__(self, layers, saliencies, num_groups: int, offload_hessians: bool = False):
        self.layers = layers
        self.num_layers = len(layers)
        self.offload_hessians = offload_hessians
        weight = layers[0].weight
        self.dev = weight.device
        self.rows, self.columns = weight.shape
        self.num_groups = num_groups
        # saliencies: per layer a (N, seq_len, G) tensor
        self.saliencies = [s.float() for s in saliencies]
        H_device = "cpu" if offload_hessians else self.dev
        self.H = _core.alloc((self.num_layers, self.num_groups, self.columns, self.columns),
                             H_device)
        self.act_square = torch.zeros((self.num_layers, self.columns), device=self.dev)
        self.index = torch.tensor([0] * self.num_layers, device=self.dev)
        self._k = [0] * self.num_layers
        self._stagers = [None] * self.num_layers
        assert self.rows % self.num_groups == 0, (
            f"Number of rows ({self.rows}) must be divisible by num_groups ({self.num_groups})")

    def _maybe_onload_hessian(self):
        """gptq_guided_utils.py:53-57."""
        return _core.onload_attrs(self, ("H",), enabled=self.offload_hessians, device=self.dev)

    # ``H`` (inherited staged attribute) reads fold the staged tokens in first:
    # the Hessians are plain sums, so a flush is H += Σ staged.
    def _flush_staged(self, idx=None):
        stagers = getattr(self, "_stagers", None)
        if not stagers:
            return
        for i in (range(self.num_layers) if idx is None else (idx,)):
            st = stagers[i]
            if st is not None and st.k:
                st.flush(self._H[i], 1.0, 1.0)

    @torch.no_grad()
    def add_batch(self, idx, inp, out):
        """gptq_guided_utils.py:59-81: H[g] += Σ_t s_tg x xᵀ; act += Σ x² / T."""
        if inp.dim() == 2:
            inp = inp.unsqueeze(0)
        else:
            assert inp.dim() == 3, "Input must be 2D or 3D. Got %dD." % inp.dim()
        bsz = inp.shape[0]
        k = self._k[idx]
        sal = self.saliencies[idx][k:k + bsz].to(self.dev)
        self._k[idx] = k + bsz
        bump(self, "index", idx, bsz)
        X, dt = _core.as_tokens(inp)
        sal = sal.reshape(-1, sal.shape[-1]).float().contiguous()
        n_tokens = X.shape[0]
        act_alpha = _core.f32(1 / n_tokens)
        st = stager_for(self, idx, X.device, KIND_WEIGHTED, self.num_groups, dt)
        if not st.fits(n_tokens):
            self._flush_staged(idx)
            if st.can_stage(n_tokens):
                st.reserve(n_tokens)
        if st.fits(n_tokens):
            st.stage(X, S=sal, s_scale=1.0, act=self.act_square[idx], act_alpha=act_alpha,
                     act_beta=1.0)
        else:
            # a batch larger than the staging budget: update directly
            if dt == 0:
                _core.weighted_update(self._H[idx], X, sal, 1.0, 1.0, self.act_square[idx],
                                      act_alpha, 1.0)
            else:
                one = single_batch_stager(self.columns, X.device, KIND_WEIGHTED,
                                          self.num_groups, dt, n_tokens)
                one.stage(X, S=sal, s_scale=1.0, act=self.act_square[idx], act_alpha=act_alpha,
                          act_beta=1.0)
                one.flush(self._H[idx], 1.0, 1.0)

    def fasterquant(self, blocksize=128, percdamp=0.01, groupsize=-1, actorder=False,
                    static_groups=False, export_compressed_tensors=False, backend="hip",
                    graph=False):
        """gptq_guided_utils.py:83-211."""
        _core.check_backend(backend)
        W = _core.stack_weights_f32(self.layers)
        B, R, C = W.shape
        G = self.num_groups
        W_flat = W.view(B * R, C)
        W_sub = W.view(B * G, R // G, C)
        flags = torch.zeros(1, dtype=torch.int32, device=self.dev)
        with self._maybe_onload_hessian():
            H = self.H
            self.H = None
            H_sub = H.view(B * G, C, C)
            H_diag = _core.hessian_diag(H_sub, self.quantizer[0].hclip)
            _core.fit_static_params(self.quantizer, W_flat, groupsize, static_groups, flags,
                                    H_diag)
            _core.prepare_hessian(H_sub, W_sub)
            perm = invperm = None
            if actorder:
                perm, invperm = _core.act_order(self.act_square, 1)
                W_sub = _core.permute_cols(W_sub, perm)
                H_sub = _core.permute_sym(H_sub, perm)
                if H_diag is not None:
                    H_diag = _core.permute_cols(H_diag, perm)
            Hinv, _ = _core.factor(H_sub, percdamp)
        Q, W_int, Scale = _compensate(_lib.VARIANT_GPTQ, self.quantizer, W_sub, Hinv, blocksize,
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
        _core.write_back(self.layers, Q.view(B, R, C), flags)
        _core.finish(flags)

    def free(self):
        """gptq_guided_utils.py:213-219."""
        self.H = None
        self.Losses = None
        self.act_square = None
        self.saliencies = None
        self.index = None
        _lib.release_workspaces()
