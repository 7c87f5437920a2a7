"""Oracle: complete ``fasterquant`` flows (test infrastructure only).

Each function takes the stacked fp32 weights ``W (B, R, C)`` plus the
accumulated statistics, and returns the dequantized weights, integer codes,
per-column scales and the quantizer list, following the reference's
``fasterquant`` step by step (minus offload, export and the write-back).
"""
import torch

from . import compensate, factor, quant


def _configure(bits, sym, columns, groupsize, mse=False, hclip=False):
    q = quant.WeightQuantizer().configure(bits, perchannel=True, sym=sym, mse=mse, hclip=hclip)
    return quant.make_group_quantizers(q, columns, groupsize)


def _hdiag(quantizers, H):
    """gptq_utils/gptq_utils.py:253-257: the undamped diagonal when hclip is on."""
    return torch.diagonal(H, dim1=-2, dim2=-1).clone() if quantizers[0].hclip else None


def _static_params(quantizers, W_flat, groupsize, static_groups, H_diag=None):
    """gptq_utils/gptq_utils.py:259-270."""
    if groupsize == -1 or static_groups:
        for i, qz in enumerate(quantizers):
            if not qz.ready():
                if groupsize == -1:
                    qz.find_params(W_flat, H_diag)
                else:
                    sl = slice(i * groupsize, (i + 1) * groupsize)
                    qz.find_params(W_flat[:, sl], None if H_diag is None else H_diag[:, sl])


def _loop_record(record, perm):
    """The pre-quantization values of a compensation loop, in the loop's column
    order, and the loop order itself (``perm`` maps loop column → column)."""
    return {"X": record["X"], "perm": perm}


def gptq_fasterquant(W, H, bits, sym, blocksize=128, percdamp=0.01, groupsize=-1, actorder=False,
                     static_groups=False, quantizers=None, mse=False, hclip=False,
                     dtype=torch.float32):
    """gptq_utils/gptq_utils.py:234-353 (returns instead of writing layers).

    ``dtype=torch.float64`` (with an fp64 ``H``) runs the same steps in fp64:
    the parity tests' measure of how far fp32 orderings move x/s."""
    W = W.clone().to(dtype)
    H = H.clone()
    B, R, C = W.shape
    if quantizers is None:
        quantizers = _configure(bits, sym, C, groupsize, mse, hclip)
    H_diag = _hdiag(quantizers, H)
    _static_params(quantizers, W.view(B * R, C), groupsize, static_groups, H_diag)
    factor.prepare_hessian(H, W)
    perm = invperm = None
    if actorder:
        perm, invperm = factor.act_order_perm(H)
        if H_diag is not None:
            H_diag = H_diag[:, perm].contiguous()
    Hinv = torch.empty_like(H)
    damps = []
    for b in range(B):
        if actorder:
            W[b] = W[b][:, perm]
            H[b] = H[b][perm][:, perm]
        Hinv[b], d = factor.damp_chol_inv_upper(H[b], percdamp)
        damps.append(d)
    rec = {}
    Q, W_int, Scale = compensate.gptq_compensation(
        W, Hinv, quantizers, blocksize, groupsize, static_groups,
        perm if static_groups and actorder else None, H_diag, record=rec)
    if actorder:
        Q, W_int, Scale = Q[:, :, invperm], W_int[:, :, invperm], Scale[:, :, invperm]
    return {"Q": Q, "W_int": W_int, "Scale": Scale, "quantizers": quantizers, "Hinv": Hinv,
            "damp": damps, "perm": perm, "loop": _loop_record(rec, perm)}


def gptaq_fasterquant(W, H, dXXT, bits, sym, blocksize=128, percdamp=0.01, groupsize=-1,
                      actorder=False, static_groups=False, alpha=0.25, quantizers=None,
                      mse=False, hclip=False, dtype=torch.float32):
    """gptq_utils/gptaq_utils.py:263-391 (``dtype`` as for gptq_fasterquant)."""
    W = W.clone().to(dtype)
    H = H.clone()
    dXXT = dXXT.clone()
    B, R, C = W.shape
    if quantizers is None:
        quantizers = _configure(bits, sym, C, groupsize, mse, hclip)
    H_diag = _hdiag(quantizers, H)
    _static_params(quantizers, W.view(B * R, C), groupsize, static_groups, H_diag)
    deads = factor.prepare_hessian(H, W)
    for b in range(B):
        dXXT[b, :, deads[b]] = 0
    perm = invperm = None
    if actorder:
        perm, invperm = factor.act_order_perm(H)
        if H_diag is not None:
            H_diag = H_diag[:, perm].contiguous()
    Hinv = torch.empty_like(H)
    for b in range(B):
        if actorder:
            W[b] = W[b][:, perm]
            H[b] = H[b][perm][:, perm]
            dXXT[b] = dXXT[b][perm][:, perm]
        Hinv[b], _ = factor.damp_chol_inv_upper(H[b], percdamp)
    P = compensate.gptaq_P(dXXT, Hinv, alpha)
    rec = {}
    Q, W_int, Scale = compensate.gptaq_compensation(
        W, Hinv, P, quantizers, blocksize, groupsize, static_groups,
        perm if static_groups and actorder else None, H_diag, record=rec)
    if actorder:
        Q, W_int, Scale = Q[:, :, invperm], W_int[:, :, invperm], Scale[:, :, invperm]
    return {"Q": Q, "W_int": W_int, "Scale": Scale, "quantizers": quantizers, "Hinv": Hinv, "P": P,
            "perm": perm, "loop": _loop_record(rec, perm)}


def g2ptq_trust_region(gradients_sub, Hinv_init, Hinv, Q_sub, W_sub, alpha, enabled):
    """gptq_utils/g2ptq_utils.py:459-476 — returns ``beta, Z, GHinv``."""
    if enabled:
        eps = torch.finfo(torch.float32).tiny
        GHinv = torch.bmm(gradients_sub, Hinv_init)
        quant_err = Q_sub - W_sub
        diag = torch.diagonal(Hinv_init, dim1=1, dim2=2).unsqueeze(1)
        loss = ((quant_err * GHinv + (quant_err ** 2) / 2) / diag).abs()
        c = (gradients_sub * GHinv).sum(dim=2, keepdim=True) - ((GHinv ** 2) / diag)
        c = c.clamp(min=2 * alpha * loss).clamp(min=eps)
        beta = (1 - torch.sqrt(torch.clamp(1 - (2 * alpha * loss) / c, min=0.0))).mean(-1)
    else:
        beta = torch.zeros((gradients_sub.shape[0], 1)).to(gradients_sub)
    Z = torch.bmm(gradients_sub, Hinv.transpose(1, 2)) * beta.unsqueeze(2)
    GHinv = torch.bmm(Z, Hinv)
    return beta, Z, GHinv


def g2ptq_fasterquant(W, H, gradients, act_square, bits, sym, num_groups, blocksize=128,
                      percdamp=0.01, groupsize=-1, actorder=False, static_groups=False,
                      enable_gradient_update=True, alpha=0.0, quantizers=None, mse=False,
                      hclip=False, dtype=torch.float32):
    """gptq_utils/g2ptq_utils.py:349-519.  ``H`` is (B, G, C, C), mutated like the reference
    (``dtype`` as for gptq_fasterquant)."""
    W = W.clone().to(dtype)
    B, R, C = W.shape
    G = num_groups
    if quantizers is None:
        quantizers = _configure(bits, sym, C, groupsize, mse, hclip)
    W_flat = W.view(B * R, C)
    W_sub = W.contiguous().view(B * G, R // G, C)
    grads = gradients.reshape(B * G, R // G, C).to(dtype).clone()
    H_sub = H.view(B * G, C, C)
    H_diag = _hdiag(quantizers, H_sub)
    _static_params(quantizers, W_flat, groupsize, static_groups, H_diag)
    for b in range(B * G):
        if (H_sub[b] == 0).all():
            H_sub[b] = torch.eye(C)
            grads[b].zero_()
        dead = torch.diag(H_sub[b]) == 0
        H_sub[b, dead, dead] = 1
        W_sub[b, :, dead] = 0
    Q_sub = None
    if enable_gradient_update and alpha > 0:
        if groupsize != -1 and not static_groups:
            for i, qz in enumerate(quantizers):
                qz.find_params(W_sub[:, :, i * groupsize:(i + 1) * groupsize].reshape(B * R, -1))
        Q_sub = quant.fake_quantize_grouped(quantizers, W_sub, groupsize)
    perm = invperm = None
    if actorder:
        perm = torch.argsort(torch.mean(act_square, dim=0), descending=True, stable=True)
        invperm = torch.argsort(perm)
    Hinv_init = torch.empty_like(H_sub)
    Hinv = torch.empty_like(H_sub)
    for b in range(B * G):
        if actorder:
            W_sub[b] = W_sub[b][:, perm]
            H_sub[b] = H_sub[b][perm][:, perm]
            grads[b] = grads[b][:, perm]
        Hinv[b], _, Hinv_init[b] = factor.damp_chol_inv_upper(H_sub[b], percdamp, want_inverse=True)
    if Q_sub is not None and actorder:
        Q_sub = Q_sub[:, :, perm]
    if H_diag is not None and actorder:
        H_diag = H_diag[:, perm].contiguous()
    beta, Z, GHinv = g2ptq_trust_region(grads, Hinv_init, Hinv, Q_sub, W_sub, alpha,
                                        enable_gradient_update and alpha > 0)
    GH0, W_tr = GHinv.clone(), W_sub.clone()
    rec = {}
    Q, W_int, Scale = compensate.g2ptq_compensation(
        W_sub, Hinv, Z, GHinv, quantizers, blocksize, groupsize, static_groups,
        perm if static_groups and actorder else None, H_diag, record=rec)
    if actorder:
        Q, W_int, Scale = Q[:, :, invperm], W_int[:, :, invperm], Scale[:, :, invperm]
    rec["X"] = rec["X"].view(B, R, C)
    return {"Q": Q.view(B, R, C), "W_int": W_int.view(B, R, C), "Scale": Scale.view(B, R, C),
            "quantizers": quantizers, "Hinv": Hinv, "beta": beta, "Z": Z, "GHinv0": GH0,
            "Hinv_init": Hinv_init, "grads": grads, "Q0": Q_sub, "W_sub": W_tr,
            "perm": perm, "loop": _loop_record(rec, perm)}


def guided_fasterquant(W, H, act_square, bits, sym, num_groups, blocksize=128, percdamp=0.01,
                       groupsize=-1, actorder=False, static_groups=False, quantizers=None,
                       mse=False, hclip=False, dtype=torch.float32):
    """gptq_utils/gptq_guided_utils.py:83-211 (``dtype`` as for gptq_fasterquant)."""
    W = W.clone().to(dtype)
    B, R, C = W.shape
    G = num_groups
    if quantizers is None:
        quantizers = _configure(bits, sym, C, groupsize, mse, hclip)
    W_flat = W.view(B * R, C)
    W_sub = W.contiguous().view(B * G, R // G, C)
    H_sub = H.clone().view(B * G, C, C)
    H_diag = _hdiag(quantizers, H_sub)
    _static_params(quantizers, W_flat, groupsize, static_groups, H_diag)
    for b in range(B * G):
        if (H_sub[b] == 0).all():
            H_sub[b] = torch.eye(C)
        dead = torch.diag(H_sub[b]) == 0
        H_sub[b, dead, dead] = 1
        W_sub[b, :, dead] = 0
    perm = invperm = None
    if actorder:
        perm = torch.argsort(torch.mean(act_square, dim=0), descending=True, stable=True)
        invperm = torch.argsort(perm)
        if H_diag is not None:
            H_diag = H_diag[:, perm].contiguous()
    Hinv = torch.empty_like(H_sub)
    for b in range(B * G):
        if actorder:
            W_sub[b] = W_sub[b][:, perm]
            H_sub[b] = H_sub[b][perm][:, perm]
        Hinv[b], _ = factor.damp_chol_inv_upper(H_sub[b], percdamp)
    rec = {}
    Q, W_int, Scale = compensate.gptq_compensation(
        W_sub, Hinv, quantizers, blocksize, groupsize, static_groups,
        perm if static_groups and actorder else None, H_diag, record=rec)
    if actorder:
        Q, W_int, Scale = Q[:, :, invperm], W_int[:, :, invperm], Scale[:, :, invperm]
    rec["X"] = rec["X"].view(B, R, C)
    return {"Q": Q.view(B, R, C), "W_int": W_int.view(B, R, C), "Scale": Scale.view(B, R, C),
            "quantizers": quantizers, "Hinv": Hinv, "perm": perm, "loop": _loop_record(rec, perm)}


def rtn(W, bits, sym, groupsize):
    """gptq_utils/gptq_utils.py:625-644 (RTN with a weight_groupsize quantizer)."""
    B, R, C = W.shape
    qz = quant.WeightQuantizer().configure(bits, perchannel=True, sym=sym, weight_groupsize=groupsize)
    flat = W.reshape(B * R, C).float()
    qz.find_params(flat)
    fq, qi, s = qz.fake_quantize(flat)
    return fq.view(B, R, C), qi.view(B, R, C), qz


def reconstruction_error(W, Q, H):
    """‖WX − QX‖² / (n/2) == tr(ΔW H ΔWᵀ) summed over layers (H = (2/n)·XᵀX)."""
    d = (W.double() - Q.double())
    return torch.einsum("brc,bcd,brd->", d, H.double(), d).item()
