"""Oracle: lazy-batch quantize → error → compensate sweeps (test infrastructure only).

Block functions work on the reference's transposed block layout
``(B, bs, R)``; loop functions work on ``W (B, R, C)`` and a list of oracle
``WeightQuantizer`` objects, exactly like the reference classes.
"""
import torch

from . import quant


# ---------------------------------------------------------------------------
# Block operators (restating the torch backends of ``run_eager``)
# ---------------------------------------------------------------------------

def gptq_block(weight, hinv, scale, zero, int_weight, error, maxq, xq=None):
    """gptq_utils/gptq_utils.py:28-51 (in place on ``weight``/``int_weight``/``error``).

    ``xq`` (optional, the block's shape) receives each column's value at the
    moment it is quantized, for the parity tests' rounding-tie checks."""
    columns = weight.shape[1]
    for column in range(columns):
        w = weight[:, column]
        if xq is not None:
            xq[:, column] = w
        qi, qs, qz = quant.asym_quant(w, scale[:, column], zero[:, column], maxq)
        q = quant.asym_dequant(qi, qs, qz)
        err = (w - q) / hinv[:, column, column].unsqueeze(1)
        weight[:, column].copy_(q)
        int_weight[:, column].copy_(qi)
        error[:, column].copy_(err)
        if column + 1 < columns:
            weight[:, column + 1:].baddbmm_(hinv[:, column, column + 1:].unsqueeze(2),
                                            err.unsqueeze(1), beta=1, alpha=-1)
    return weight, int_weight, error


def gptaq_block(weight, hinv, p, scale, zero, column_weight, int_weight, error, maxq, xq=None):
    """gptq_utils/gptaq_utils.py:28-56."""
    columns = weight.shape[1]
    for column in range(columns):
        column_weight.copy_(weight[:, column])
        if xq is not None:
            xq[:, column] = column_weight
        qi, qs, qz = quant.asym_quant(column_weight, scale[:, column], zero[:, column], maxq)
        q = quant.asym_dequant(qi, qs, qz)
        err = (column_weight - q) / hinv[:, column, column].unsqueeze(1)
        weight[:, column].copy_(q)
        int_weight[:, column].copy_(qi)
        error[:, column].copy_(err)
        if column + 1 < columns:
            weight[:, column + 1:].baddbmm_(
                hinv[:, column, column + 1:].unsqueeze(2), err.unsqueeze(1), beta=1, alpha=-1
            ).baddbmm_(p[:, column, column + 1:].unsqueeze(2), column_weight.unsqueeze(1),
                       beta=1, alpha=1)
    return weight, int_weight, error


def g2ptq_block(weight, hinv, scale, zero, z, ghinv, int_weight, error, maxq, xq=None):
    """gptq_utils/g2ptq_utils.py:34-74 (``approx_beta == 0``)."""
    columns = weight.shape[1]
    for column in range(columns):
        w = weight[:, column]
        if xq is not None:
            xq[:, column] = w
        qi, qs, qz = quant.asym_quant(w, scale[:, column], zero[:, column], maxq)
        q = quant.asym_dequant(qi, qs, qz)
        err = w - q - ghinv[:, column]
        err = err / hinv[:, column, column].unsqueeze(1)
        weight[:, column].copy_(q)
        int_weight[:, column].copy_(qi)
        error[:, column].copy_(err)
        if column + 1 < columns:
            row = hinv[:, column, column + 1:].unsqueeze(2)
            weight[:, column + 1:].sub_(ghinv[:, column + 1:]).baddbmm_(
                row, err.unsqueeze(1), beta=1, alpha=-1)
            ghinv[:, column + 1:].baddbmm_(row, z[:, column].unsqueeze(1), beta=1, alpha=-1)
    return weight, int_weight, error


# ---------------------------------------------------------------------------
# Per-layer lazy-batch loops (``_run_compensation``)
# ---------------------------------------------------------------------------

def _column_quantizers(quantizers, W, i1, i2, groupsize, static_groups, qparam_perm, B, R,
                       H_diag=None):
    """gptq_utils/gptq_utils.py:185-205 — per-column quantizer selection."""
    if groupsize == -1:
        return [quantizers[0]] * (i2 - i1)
    if static_groups:
        idx = range(i1, i2) if qparam_perm is None else qparam_perm[i1:i2].tolist()
        return [quantizers[i // groupsize] for i in idx]
    out = []
    for i in range(i1, i2):
        qz = quantizers[i // groupsize]
        if i % groupsize == 0:
            qz.find_params(W[:, :, i:i + groupsize].reshape(B * R, -1),
                           None if H_diag is None else H_diag[:, i:i + groupsize])
        out.append(qz)
    return out


def _stack_params(cq, shape):
    s = torch.stack([q.scale for q in cq], dim=1).reshape(shape)
    z = torch.stack([q.zero for q in cq], dim=1).reshape(shape)
    return s, z


def _maxq(quantizers):
    return quantizers[0].maxq


def _recorder(record, W):
    """``record`` (a dict or None) receives ``"X"``: every weight's value when it
    was quantized, in the loop's column order (B, R, C)."""
    if record is None:
        return None
    record["X"] = torch.zeros_like(W)
    return record["X"]


def _record_block(X, i1, i2, xt):
    if X is not None:
        X[:, :, i1:i2] = xt.transpose(1, 2)


def gptq_compensation(W, Hinv, quantizers, blocksize=128, groupsize=-1, static_groups=False,
                      qparam_perm=None, H_diag=None, record=None):
    """gptq_utils/gptq_utils.py:165-232 (torch backend, no graph). Mutates W."""
    B, R, C = W.shape
    X = _recorder(record, W)
    Q = torch.zeros_like(W)
    W_int = torch.zeros_like(W)
    Scale = torch.zeros_like(W)
    for i1 in range(0, C, blocksize):
        i2 = min(i1 + blocksize, C)
        W1 = W[:, :, i1:i2].clone()
        cq = _column_quantizers(quantizers, W, i1, i2, groupsize, static_groups, qparam_perm, B, R,
                                H_diag)
        S1, Z1 = _stack_params(cq, W1.shape)
        wt = W1.transpose(1, 2).contiguous()
        it, et, xt = torch.empty_like(wt), torch.empty_like(wt), torch.empty_like(wt)
        gptq_block(wt, Hinv[:, i1:i2, i1:i2].contiguous(), S1.transpose(1, 2).contiguous(),
                   Z1.transpose(1, 2).contiguous(), it, et, _maxq(quantizers), xt)
        _record_block(X, i1, i2, xt)
        Q1, I1, E1 = (t.transpose(1, 2).contiguous() for t in (wt, it, et))
        Q[:, :, i1:i2] = Q1
        W_int[:, :, i1:i2] = I1
        Scale[:, :, i1:i2] = S1
        W[:, :, i2:].baddbmm_(E1, Hinv[:, i1:i2, i2:], beta=1, alpha=-1)
    return Q, W_int, Scale


def gptaq_compensation(W, Hinv, P, quantizers, blocksize=128, groupsize=-1, static_groups=False,
                       qparam_perm=None, H_diag=None, record=None):
    """gptq_utils/gptaq_utils.py:193-261. Mutates W."""
    B, R, C = W.shape
    X = _recorder(record, W)
    Q = torch.zeros_like(W)
    W_int = torch.zeros_like(W)
    Scale = torch.zeros_like(W)
    for i1 in range(0, C, blocksize):
        i2 = min(i1 + blocksize, C)
        W1 = W[:, :, i1:i2].clone()
        cq = _column_quantizers(quantizers, W, i1, i2, groupsize, static_groups, qparam_perm, B, R,
                                H_diag)
        S1, Z1 = _stack_params(cq, W1.shape)
        wt = W1.transpose(1, 2).contiguous()
        it, et, xt = torch.empty_like(wt), torch.empty_like(wt), torch.empty_like(wt)
        cw = torch.empty(wt.shape[0], wt.shape[2], dtype=wt.dtype)
        gptaq_block(wt, Hinv[:, i1:i2, i1:i2].contiguous(), P[:, i1:i2, i1:i2].contiguous(),
                    S1.transpose(1, 2).contiguous(), Z1.transpose(1, 2).contiguous(), cw, it, et,
                    _maxq(quantizers), xt)
        _record_block(X, i1, i2, xt)
        Q1, I1, E1 = (t.transpose(1, 2).contiguous() for t in (wt, it, et))
        Q[:, :, i1:i2] = Q1
        W_int[:, :, i1:i2] = I1
        Scale[:, :, i1:i2] = S1
        W[:, :, i2:].baddbmm_(E1, Hinv[:, i1:i2, i2:], beta=1, alpha=-1).baddbmm_(
            Q1, P[:, i1:i2, i2:], beta=1, alpha=1)
    return Q, W_int, Scale


def g2ptq_compensation(W, Hinv, Z, GHinv, quantizers, blocksize=128, groupsize=-1,
                       static_groups=False, qparam_perm=None, H_diag=None, record=None):
    """gptq_utils/g2ptq_utils.py:252-347 (``approx_grad_beta == 0``). Mutates W and GHinv."""
    B, R, C = W.shape
    X = _recorder(record, W)
    Q = torch.zeros_like(W)
    W_int = torch.zeros_like(W)
    Scale = torch.zeros_like(W)
    D = torch.arange(blocksize - 1, -1, -1).to(GHinv)
    for i1 in range(0, C, blocksize):
        i2 = min(i1 + blocksize, C)
        W1 = W[:, :, i1:i2].clone()
        Z1 = Z[:, :, i1:i2]
        GH1 = GHinv[:, :, i1:i2].clone()
        cq = _column_quantizers(quantizers, W, i1, i2, groupsize, static_groups, qparam_perm, B, R,
                                H_diag)
        S1, Zp1 = _stack_params(cq, W1.shape)
        wt = W1.transpose(1, 2).contiguous()
        it, et, xt = torch.empty_like(wt), torch.empty_like(wt), torch.empty_like(wt)
        g2ptq_block(wt, Hinv[:, i1:i2, i1:i2].contiguous(), S1.transpose(1, 2).contiguous(),
                    Zp1.transpose(1, 2).contiguous(), Z1.transpose(1, 2).contiguous(),
                    GH1.transpose(1, 2).contiguous(), it, et, _maxq(quantizers), xt)
        _record_block(X, i1, i2, xt)
        Q1, I1, E1 = (t.transpose(1, 2).contiguous() for t in (wt, it, et))
        Q[:, :, i1:i2] = Q1
        W_int[:, :, i1:i2] = I1
        Scale[:, :, i1:i2] = S1
        if i2 == C:
            continue
        upd = blocksize * GHinv[:, :, i2:]
        upd.baddbmm_(Z1 * D.reshape(1, 1, -1), Hinv[:, i1:i2, i2:], beta=1, alpha=-1)
        W[:, :, i2:].sub_(upd).baddbmm_(E1, Hinv[:, i1:i2, i2:], beta=1, alpha=-1)
        GHinv[:, :, i2:].baddbmm_(Z[:, :, i1:i2], Hinv[:, i1:i2, i2:], beta=1, alpha=-1)
    return Q, W_int, Scale


def gptaq_P(dXXT, U, alpha=0.25):
    """gptq_utils/gptaq_utils.py:349-352 — ``P = α·triu(dXXT·Uᵀ, 1)·U``."""
    t = torch.bmm(dXXT, U.transpose(1, 2))
    return alpha * torch.bmm(torch.triu(t, diagonal=1), U)
