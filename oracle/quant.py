"""Oracle: weight-quantizer semantics (test infrastructure only).

Restates ``utils/quant_utils.py`` of the reference in torch-CPU fp32.
"""
import copy

import torch


def asym_quant(x, scale, zero, maxq):
    """utils/quant_utils.py:8-12 — ``clamp(round(x/s) + z, -(maxq+1), maxq)``."""
    q = torch.clamp(torch.round(x / scale) + zero, -(maxq + 1), maxq)
    return q, scale, zero


def asym_dequant(q, scale, zero):
    """utils/quant_utils.py:15-16."""
    return scale * (q - zero)


def sym_quant(x, scale, maxq):
    """utils/quant_utils.py:23-26."""
    q = torch.clamp(torch.round(x / scale), -(maxq + 1), maxq)
    return q, scale


def sym_dequant(q, scale):
    """utils/quant_utils.py:29-30."""
    return scale * q


def minmax(x):
    """utils/quant_utils.py:47-57 (clip_ratio == 1)."""
    xmin = x.amin(dim=-1, keepdim=True)
    xmax = x.amax(dim=-1, keepdim=True)
    return torch.minimum(xmin, torch.zeros_like(xmin)), torch.maximum(xmax, torch.zeros_like(xmax))


def params_from_range(xmin, xmax, bits, sym):
    """utils/quant_utils.py:60-68 with the grid of :372-374."""
    maxq = 2 ** (bits - 1) - 1
    minq = -(maxq + 1)
    bit_range = maxq - minq
    if sym:
        scale = torch.maximum(torch.abs(xmin), xmax) / (bit_range / 2)
        zero = torch.zeros_like(scale)
    else:
        scale = (xmax - xmin) / bit_range
        zero = torch.clamp(torch.round(minq - xmin / scale), minq, maxq)
    return scale, zero


def quant_err(fq, x, norm, H_diag=None):
    """utils/quant_utils.py:84-105: sum(|fq - x|^norm) over the last dim, or
    with a Hessian diagonal (blocks, *x.shape[1:]) sum((fq - x)^2 * h), the
    rows of ``x`` splitting into ``blocks`` consecutive equal shares."""
    if H_diag is None:
        return fq.sub_(x).abs_().pow_(norm).sum(-1)
    shape = fq.shape[:-1]
    e = fq.sub_(x).pow_(2)
    e = e.reshape(H_diag.shape[0], -1, *H_diag.shape[1:])
    e.mul_(H_diag.unsqueeze(1))
    return e.sum(-1).reshape(shape)


def find_params(x, bits, sym, mse=False, norm=2.4, grid=50, maxshrink=0.5, H_diag=None):
    """utils/quant_utils.py:377-433 for a per-channel quantizer.

    ``x`` is (rows, cols), or already the canonical (row_groups, col_groups,
    groupsize) view; returns ``scale, zero`` of shape (rows, 1) (resp.
    (row_groups, col_groups)), exactly as ``WeightQuantizer.find_params``
    leaves them (zero rounded again at :428).  ``H_diag`` (hclip) is taken as
    given: the caller reshapes it and drops it when all entries are equal
    (:393-397).
    """
    maxq = 2 ** (bits - 1) - 1
    minq = -(maxq + 1)
    xg = x if x.dim() == 3 else x.flatten(1).unsqueeze(1)   # (rows, 1, cols)  :389
    xmin, xmax = minmax(xg)
    scale, zero = params_from_range(xmin, xmax, bits, sym)
    if mse:                                              # :406-425
        best = torch.full(xg.shape[:-1], float("inf"))
        for i in range(int(maxshrink * grid)):
            for j in range(int(maxshrink * grid)):
                xmin1 = (1 - i / grid) * xmin
                xmax1 = (1 - j / grid) * xmax
                scale1, zero1 = params_from_range(xmin1, xmax1, bits, sym)
                if sym:
                    q, _ = sym_quant(xg, scale1, maxq)
                    fq = sym_dequant(q, scale1)
                else:
                    q, _, _ = asym_quant(xg, scale1, zero1, maxq)
                    fq = asym_dequant(q, scale1, zero1)
                err = quant_err(fq, xg, norm, H_diag)
                better = err < best
                better_k = better.unsqueeze(-1)
                scale = torch.where(better_k, scale1, scale)
                zero = torch.where(better_k, zero1, zero)
                best = torch.where(better, err, best)
    zero = torch.round(zero)
    return scale.squeeze(-1), zero.squeeze(-1)


class WeightQuantizer:
    """Minimal stand-in of utils/quant_utils.py:341-465 (per-channel, no hclip)."""

    def __init__(self):
        self.scale = torch.zeros(1)
        self.zero = torch.zeros(1)
        self._ready = False

    def configure(self, bits, perchannel=True, sym=True, mse=False, norm=2.4, grid=50,
                  maxshrink=0.5, weight_groupsize=-1, hclip=False):
        self.bits, self.perchannel, self.sym, self.mse = bits, perchannel, sym, mse
        self.norm, self.grid, self.maxshrink = norm, grid, maxshrink
        self.weight_groupsize, self.hclip = weight_groupsize, hclip
        self.maxq = 2 ** (bits - 1) - 1
        self.minq = -(self.maxq + 1)
        self.bit_range = self.maxq - self.minq
        self._ready = False
        return self

    def find_params(self, x, H_diag=None):
        """utils/quant_utils.py:377-433 (per-channel or weight_groupsize)."""
        if self.weight_groupsize > 0:
            rows, cols = x.shape
            g = self.weight_groupsize
            xg = x.reshape(rows, cols // g, g)
        else:
            xg = x.flatten(1).unsqueeze(1)
        if self.hclip:                                       # :393-397
            H_diag = H_diag.reshape(H_diag.shape[0], *xg.shape[1:])
            if (H_diag.min() == H_diag.max()).item():
                H_diag = None
        s, z = find_params(xg, self.bits, self.sym, self.mse, self.norm, self.grid,
                           self.maxshrink, H_diag if self.hclip else None)
        self.scale, self.zero = s, z
        # The zero point before its rounding (min/max asym fits only), for the
        # parity tests' tie checks: a value within rounding noise of k + 1/2
        # can round either way on another machine's arithmetic.
        self.zraw = None
        if not self.sym and not self.mse:
            xmin, _ = minmax(xg)
            self.zraw = (self.minq - xmin / s.unsqueeze(-1)).squeeze(-1)
        self._ready = True

    def ready(self):
        return self._ready

    def fake_quantize(self, x):
        """utils/quant_utils.py:435-459; returns (dequantized, codes, scale)."""
        if self.weight_groupsize > 0:
            shape = x.shape
            g = self.weight_groupsize
            xg = x.reshape(shape[0], shape[1] // g, g)
            s, z = self.scale.unsqueeze(-1), self.zero.unsqueeze(-1)
        else:
            xg, s, z = x, self.scale, self.zero
        if self.sym:
            q, _ = sym_quant(xg, s, self.maxq)
            fq = sym_dequant(q, s)
        else:
            q, _, _ = asym_quant(xg, s, z, self.maxq)
            fq = asym_dequant(q, s, z)
        if self.weight_groupsize > 0:
            fq, q = fq.reshape(shape), q.reshape(shape)
        return fq, q, self.scale


def make_group_quantizers(quantizer, columns, groupsize):
    """gptq_utils/common_utils.py:13-16."""
    n = 1 if groupsize == -1 else (columns + groupsize - 1) // groupsize
    return [copy.deepcopy(quantizer) for _ in range(n)]


def merge_group_quantizers(quantizers, start, end, groupsize):
    """gptq_utils/common_utils.py:19-30."""
    out = copy.deepcopy(quantizers[0])
    out.scale = torch.cat([q.scale[start:end] for q in quantizers], dim=1).clone()
    out.zero = torch.cat([q.zero[start:end] for q in quantizers], dim=1).clone()
    out.weight_groupsize = groupsize
    out._ready = all(q.ready() for q in quantizers)
    return out


def fake_quantize_grouped(quantizers, weight, groupsize):
    """gptq_utils/common_utils.py:33-44."""
    flat_rows = weight.shape[0] * weight.shape[1]
    width = weight.shape[-1] if groupsize == -1 else groupsize
    out = []
    for g, quantizer in enumerate(quantizers):
        s = g * width
        e = min(s + width, weight.shape[-1])
        q = quantizer.fake_quantize(weight[:, :, s:e].reshape(flat_rows, e - s))[0]
        out.append(q.reshape(*weight.shape[:2], e - s))
    return torch.cat(out, dim=-1)
