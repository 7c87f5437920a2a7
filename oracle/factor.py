"""Oracle: Hessian preparation, dampening and the inverse-Cholesky factor.

Test infrastructure only.  torch-CPU fp32, the reference's library calls
(``torch.linalg.cholesky`` / ``torch.cholesky_inverse``) in the reference's
order.
"""
import torch


def prepare_hessian(H, W, num_layers=None):
    """gptq_utils/gptq_utils.py:272-277 (in place on H (B,C,C) and W (B,R,C)).

    Returns the per-layer dead-column masks.
    """
    C = H.shape[-1]
    deads = []
    for b in range(H.shape[0]):
        if (H[b] == 0).all():
            H[b] = torch.eye(C).to(H[b])
        dead = torch.diag(H[b]) == 0
        H[b, dead, dead] = 1
        W[b, :, dead] = 0
        deads.append(dead)
    return deads


class LinAlgFailure(Exception):
    pass


def damp_chol_inv_upper(Hb, percdamp=0.01, want_inverse=False):
    """gptq_utils/gptq_utils.py:291-311 (and g2ptq_utils.py:430-450).

    Returns ``(U, damp_percent_used[, Hinv_init])`` with ``U = chol(A⁻¹, upper)``,
    ``A = H + p·mean(diag H)·I``; retries ``p += 0.0015`` while ``0 < p < 1``.
    """
    C = Hb.shape[-1]
    damp_percent = percdamp
    U = Hinv_init = None
    while 1 > damp_percent > 0:
        try:
            damp = damp_percent * torch.mean(torch.diag(Hb))
            diag = torch.arange(C)
            A = Hb.clone()
            A[diag, diag] += damp
            L = torch.linalg.cholesky(A)
            Hinv_init = torch.cholesky_inverse(L)
            U = torch.linalg.cholesky(Hinv_init, upper=True)
            if torch.isnan(U).any().item():
                raise torch._C._LinAlgError
            break
        except torch._C._LinAlgError:
            damp_percent += 0.0015
    if not (0 < damp_percent < 1):
        raise ValueError(f"Quantization: `damp_percent` must between 0 and 1. current is {damp_percent}")
    if want_inverse:
        return U, damp_percent, Hinv_init
    return U, damp_percent


def exact_inv_upper(Hb, damp_percent):
    """fp64 ground truth of the same factor (for accuracy comparisons, not a restatement)."""
    A = Hb.double().clone()
    C = A.shape[-1]
    A[range(C), range(C)] += damp_percent * torch.mean(torch.diag(Hb)).double()
    Ainv = torch.linalg.inv(A)
    Ainv = (Ainv + Ainv.T) / 2
    return torch.linalg.cholesky(Ainv, upper=True), Ainv


def act_order_perm(H):
    """gptq_utils/gptq_utils.py:279-282 — shared permutation, mean diagonal descending."""
    perm = torch.argsort(torch.mean(torch.diagonal(H, dim1=1, dim2=2), dim=0), descending=True,
                         stable=True)
    return perm, torch.argsort(perm)
