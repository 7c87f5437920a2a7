"""Hessian de-duplication for linears that receive the same input tensor.

The reference accumulates one Hessian per linear even when several linears
share an input (q/k/v, gate/up; its model specs declare these groups in
utils/models/base.py:209-233 and mixins.py:70-78, and FPInputsCache uses them
to share input copies, gptq_utils/gptaq_utils.py:442-555).  ``SharedInputHessian``
accumulates the group's Hessian once, on its first member, and copies the
result into the other members' slots when calibration ends, so every member
holds exactly the values it would have accumulated itself.

``SharedInputHessian.fasterquant`` quantizes GPTQ members in one compensation
loop over all their rows (rows are independent, the factor is shared), with
the result of every member's own ``fasterquant``.
"""
import copy

import torch


class SharedInputHessian:
    def __init__(self, members):
        """``members``: list of ``(quantizer_instance, layer_index)`` pairs.

        Only plain-Hessian quantizers share: GPTAQ's cross term takes each
        linear's own full-precision input, and the weighted Hessians of G2PTQ
        and GuidedQuant each linear's own saliencies, so their members are
        refused."""
        if not members:
            raise ValueError("SharedInputHessian needs at least one member")
        from .g2ptq_utils import G2PTQ
        from .gptaq_utils import GPTAQ
        from .gptq_guided_utils import GPTQGuided
        for inst, _ in members:
            if isinstance(inst, (GPTAQ, G2PTQ, GPTQGuided)):
                raise ValueError(f"SharedInputHessian shares plain GPTQ Hessians; a "
                                 f"{type(inst).__name__} Hessian depends on more than the input")
        self.members = list(members)
        self._factors = {}
        # the group shares its Hessian itself: its owner's stager need not
        # look for other stagers of the same batches
        self.members[0][0].__dict__["_share_grams"] = False

    # The members' Hessians are bit-identical, and so are their dampened
    # inverse-Cholesky factors: the first member to factor stores it here and
    # the others reuse it (an instance uses the cache only when all of its
    # slots are members).
    def cached_factor(self, percdamp):
        return self._factors.get(percdamp)

    def store_factor(self, percdamp, U, damp):
        self._factors[percdamp] = (U, damp)

    def add_batch(self, inp, out=None):
        owner, idx = self.members[0]
        owner.add_batch(idx, inp, out)

    def finalize(self):
        owner, idx = self.members[0]
        owner.H  # reading H folds any staged calibration tokens into it
        self._factors = {}  # factors of an earlier calibration are stale
        for inst, j in self.members[1:]:
            if inst is owner and j == idx:
                continue
            inst.H[j].copy_(owner.H[idx])
            inst._n[j] = owner._n[idx]
            if hasattr(inst, "_n_flushed"):
                inst._n_flushed[j] = owner._n[idx]
            inst.nsamples[j] = owner.nsamples[idx]
        slots = {}
        for inst, j in self.members:
            slots.setdefault(id(inst), (inst, set()))[1].add(j)
        for inst, js in slots.values():
            if js == set(range(inst.num_layers)):
                inst._shared_factor = self
            # the instance's other member slots now hold copies of its first
            # one: its batched factor need not factor them again (an add_batch
            # on the instance drops the map)
            first = min(js)
            alias = inst.__dict__.get("_h_alias") or {}
            alias.update({j: first for j in js if j != first})
            inst._h_alias = alias

    def fasterquant(self, blocksize=128, percdamp=0.01, groupsize=-1, actorder=False,
                    static_groups=False, export_compressed_tensors=False, backend="hip",
                    graph=False):
        """Every member instance's ``fasterquant`` with these arguments.  GPTQ
        instances whose slots are all members, with dynamic groups, no
        act-order, no hclip and no graph, run as one compensation loop over
        the rows of all of them (the same U, the same per-row arithmetic:
        the weights and fitted group parameters equal the per-instance
        calls'); anything else runs instance by instance."""
        from . import _core, _lib
        from .compressed_tensors_utils import compress_layers
        from .gptq_utils import GPTQ
        insts = []
        for inst, _ in self.members:
            if all(inst is not x for x in insts):
                insts.append(inst)
        kw = dict(blocksize=blocksize, percdamp=percdamp, groupsize=groupsize, actorder=actorder,
                  static_groups=static_groups,
                  export_compressed_tensors=export_compressed_tensors, backend=backend,
                  graph=graph)
        q0 = insts[0].quantizer[0]
        cfg = lambda q: (q.bits, bool(q.sym), bool(q.mse), q.norm, q.grid, q.maxshrink,
                         bool(getattr(q, "hclip", False)))
        joint = (len(insts) > 1 and groupsize > 0 and not static_groups and not actorder
                 and not graph and not getattr(q0, "hclip", False)
                 and all(type(i) is GPTQ and getattr(i, "_shared_factor", None) is self
                         and len(i.quantizer) == len(insts[0].quantizer)
                         and all(cfg(q) == cfg(q0) for q in i.quantizer) for i in insts))
        if not joint:
            for inst in insts:
                inst.fasterquant(**kw)
            return
        _core.check_backend(backend)
        Ws = [_core.stack_weights_f32(inst.layers) for inst in insts]
        C = Ws[0].shape[-1]
        rows = [w.shape[0] * w.shape[1] for w in Ws]
        W = torch.cat([w.view(-1, C) for w in Ws]).unsqueeze(0)
        dev = W.device
        flags = torch.zeros(1, dtype=torch.int32, device=dev)
        with insts[0]._maybe_onload_hessian():
            H = insts[0].H[:1]  # a view: the instances drop their H right after
        for inst in insts:
            inst.H = None
        _core.prepare_hessian(H, W)
        # host work that does not need the factor goes before its status read
        qs = [copy.deepcopy(q) for q in insts[0].quantizer]
        U, _ = _core.factor(H, percdamp, self, key=False)
        Q, W_int, Scale = _core.compensate(_lib.VARIANT_GPTQ, W, U, qs, blocksize, groupsize,
                                           False, None, flags)
        off = 0
        for inst, w, n in zip(insts, Ws, rows):
            B, R = w.shape[0], w.shape[1]
            sl = slice(off, off + n)
            for q, qj in zip(inst.quantizer, qs):
                q._buffers["scale"] = qj.scale[sl]
                q._buffers["zero"] = qj.zero[sl]
                q.__dict__["_ready"] = True
            Qi = Q[0, sl].view(B, R, C)
            if export_compressed_tensors:
                compress_layers(inst.layers, Scale[0, sl].view(B, R, C),
                                W_int[0, sl].view(B, R, C), q0.bits, groupsize, C)
            _core.write_back(inst.layers, Qi, flags)
            off += n
        _core.finish(flags)
