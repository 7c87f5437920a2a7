"""Hessian de-duplication for linears that receive the same input tensor.

The reference accumulates one Hessian per linear even when several linears
share an input (q/k/v, gate/up; its model specs declare these groups in
utils/models/base.py:209-233 and mixins.py:70-78, and FPInputsCache uses them
to share input copies, gptq_utils/gptaq_utils.py:442-555).  ``SharedInputHessian``
accumulates the group's Hessian once, on its first member, and copies the
result into the other members' slots when calibration ends, so every member
holds exactly the values it would have accumulated itself.
"""


class SharedInputHessian:
    def __init__(self, members):
        """``members``: list of ``(quantizer_instance, layer_index)`` pairs."""
        if not members:
            raise ValueError("SharedInputHessian needs at least one member")
        self.members = list(members)
        self._factors = {}

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
