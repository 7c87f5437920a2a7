"""Weight-quantizer grid on MI355X: the drop-in for the weight half of
``utils/quant_utils.py`` of the reference.

``WeightQuantizer`` keeps the reference's attributes and method contract
(``configure`` / ``find_params`` / ``fake_quantize`` / ``ready`` / ``enabled``,
``scale``/``zero`` buffers with the same shapes), but every computation runs
in the HIP library: min/max range fitting, the MSE clip search and
round-to-nearest fake quantization.  Tensors must live on the GPU.

Grid semantics (utils/quant_utils.py:8-68, 372-374): ``maxq = 2^(b-1) - 1``,
``minq = -(maxq + 1)``, ``bit_range = maxq - minq``; ranges always include 0;
symmetric ``s = max(|xmin|, xmax) / (bit_range / 2)``, ``z = 0``; asymmetric
``s = (xmax - xmin) / bit_range``, ``z = clamp(round(minq - xmin / s))``;
``q = clamp(round(x / s) + z, minq, maxq)`` with round-half-to-even and
``x̂ = s·(q - z)``.
"""
import collections

import torch

from . import _lib


def _require_cuda(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError("g2ptq_amd quantizer kernels require GPU tensors")


def _rows_view(x, scale, zero):
    """Flatten ``x`` to (rows, cols) with one (scale, zero) pair per row."""
    x2 = x.reshape(-1, x.shape[-1]).contiguous().float()
    rows = x2.shape[0]
    s = scale.to(torch.float32).expand(*x.shape[:-1], 1).reshape(rows).contiguous()
    z = zero.to(torch.float32).expand(*x.shape[:-1], 1).reshape(rows).contiguous()
    return x2, s, z


def _fake_quant_rows(x, scale, zero, maxq, want_codes=True):
    _require_cuda(x, scale, zero)
    bits = (maxq + 1).bit_length()
    x2, s, z = _rows_view(x, scale, zero)
    q = torch.empty_like(x2)
    codes = torch.empty_like(x2) if want_codes else None
    _lib.call("g2ptq_fake_quantize", _lib.stream_ptr(x.device), _lib.ptr(x2), x2.shape[0],
              x2.shape[1], x2.shape[1], -1, _lib.ptr(s), _lib.ptr(z), 1, bits, _lib.ptr(q),
              x2.shape[1], _lib.ptr(codes), x2.shape[1], None)
    return q.view(x.shape), (codes.view(x.shape) if want_codes else None)


def asym_quant(x, scale, zero, maxq):
    """utils/quant_utils.py:8-12 for a per-row (last-dim broadcast) scale/zero."""
    _, codes = _fake_quant_rows(x, scale, zero, maxq)
    return codes, scale, zero


def asym_dequant(q, scale, zero):
    """utils/quant_utils.py:15-16 (exact: one rounding, like the reference)."""
    return scale * (q - zero)


def asym_quant_dequant(x, scale, zero, maxq):
    return _fake_quant_rows(x, scale, zero, maxq, want_codes=False)[0]


def sym_quant(x, scale, maxq):
    """utils/quant_utils.py:23-26."""
    _, codes = _fake_quant_rows(x, scale, torch.zeros_like(scale), maxq)
    return codes, scale


def sym_dequant(q, scale):
    return scale * q


def sym_quant_dequant(x, scale, maxq):
    return _fake_quant_rows(x, scale, torch.zeros_like(scale), maxq, want_codes=False)[0]


_CONTAINERS = frozenset((dict, collections.OrderedDict, set, list))


class WeightQuantizer(torch.nn.Module):
    """Drop-in for ``utils/quant_utils.py:341-465`` (``WeightQuantizer``)."""

    def __init__(self, shape: int = 1) -> None:
        super().__init__()
        self.register_buffer("scale", torch.zeros(shape))
        self.register_buffer("zero", torch.zeros(shape))
        self._ready = False

    def __deepcopy__(self, memo, clone_buffers=True):
        """An independent copy, as ``copy.deepcopy`` of the module would make,
        without nn.Module's generic deep-copy machinery (make_group_quantizers
        copies one quantizer per group: 112 copies for a 14336-column layer)."""
        new = object.__new__(self.__class__)
        memo[id(self)] = new
        src = self.__dict__
        d = src.copy()  # scalars and flags shared, containers and tensors replaced below
        for k, v in src.items():
            t = type(v)
            if t in _CONTAINERS:
                d[k] = v.copy()
            elif isinstance(v, torch.Tensor):
                d[k] = v.clone()
        if clone_buffers:
            d["_buffers"] = {n: None if b is None else b.clone() for n, b in src["_buffers"].items()}
        object.__setattr__(new, "__dict__", d)
        return new

    def configure(self, bits, perchannel: bool = False, sym: bool = True, mse: bool = False,
                  norm: float = 2.4, grid: int = 50, maxshrink: float = 0.5,
                  weight_groupsize: int = -1, hclip: bool = False) -> None:
        """utils/quant_utils.py:350-375."""
        self.bits = bits
        self.perchannel = perchannel
        self.sym = sym
        self.mse = mse
        self.hclip = hclip
        self.norm = norm
        self.grid = grid
        self.maxshrink = maxshrink
        self.weight_groupsize = weight_groupsize
        self.maxq = 2 ** (bits - 1) - 1
        self.minq = -(self.maxq + 1)
        self.bit_range = self.maxq - self.minq
        self._ready = False

    def find_params(self, x, H_diag=None, _flags=None) -> None:
        """utils/quant_utils.py:377-433 on the GPU.

        ``H_diag`` (needed when ``hclip`` is set) weights the MSE clip search's
        error by the Hessian diagonal: its rows apply to equal consecutive
        shares of the rows of ``x`` (one per layer or saliency group).
        ``_flags`` (int32 device tensor) collects the scale>0 check without a
        host sync; without it the check runs synchronously and raises like the
        reference's device assert would.
        """
        if self.bits == 16:
            return
        _require_cuda(x)
        init_shape = x.shape
        gpr = 1  # column groups per row of x
        if self.weight_groupsize > 0:
            rows, columns = init_shape
            g = self.weight_groupsize
            gpr = columns // g
            xg = x.reshape(rows * gpr, g)
            out_shape = (rows, gpr)
        elif self.perchannel:
            xg = x.flatten(1)
            out_shape = (xg.shape[0], 1)
        else:
            xg = x.reshape(1, -1)
            out_shape = (1, 1)
        hd = self._hdiag(H_diag, xg.shape[0] // gpr, gpr * xg.shape[1], x.device) \
            if self.hclip else None
        xg = xg.float()
        if xg.stride(-1) != 1:
            xg = xg.contiguous()
        rows, cols = xg.shape
        scale = torch.empty(rows, device=x.device, dtype=torch.float32)
        zero = torch.empty(rows, device=x.device, dtype=torch.float32)
        flags = _flags if _flags is not None else torch.zeros(1, dtype=torch.int32, device=x.device)
        stream = _lib.stream_ptr(x.device)
        if self.mse:
            nb = hd.shape[0] if hd is not None else 0
            if hd is not None and (rows // gpr) % nb != 0:
                raise RuntimeError(f"shape '[{nb}, -1, {gpr}, {cols}]' is invalid for input of "
                                   f"size {rows * cols}")
            _lib.call("g2ptq_find_params_mse", stream, _lib.ptr(xg), rows, cols, xg.stride(0),
                      self.bits, int(self.sym), float(self.norm), int(self.grid),
                      float(self.maxshrink), _lib.ptr(hd), gpr * cols, nb, gpr,
                      _lib.ptr(scale), _lib.ptr(zero), 1, _lib.ptr(flags))
        else:
            _lib.call("g2ptq_find_params", stream, _lib.ptr(xg), rows, cols, xg.stride(0),
                      self.bits, int(self.sym), _lib.ptr(scale), _lib.ptr(zero), 1, _lib.ptr(flags))
        self.scale = scale.view(out_shape)
        self.zero = zero.view(out_shape)
        if _flags is None:
            check_flags(flags)
        self._ready = True

    @staticmethod
    def _hdiag(H_diag, row_groups, columns, device):
        """utils/quant_utils.py:393-397: ``H_diag`` as (blocks, columns) fp32 on the
        device, the rows of the search splitting into ``blocks`` equal shares.
        Whether the weights apply (not every entry equal) is decided by the
        kernel, without a host sync."""
        if H_diag is None:
            # the reference reshapes H_diag unconditionally when hclip is set
            raise AttributeError("WeightQuantizer with hclip=True needs H_diag "
                                 "('NoneType' object has no attribute 'shape')")
        nb = H_diag.shape[0]
        if nb == 0 or H_diag.numel() != nb * columns:
            raise RuntimeError(f"shape '[{nb}, {columns}]' is invalid for input of size "
                               f"{H_diag.numel()}")
        return H_diag.to(device=device, dtype=torch.float32).reshape(nb, columns).contiguous()

    def fake_quantize(self, x):
        """utils/quant_utils.py:435-459: returns ``(dequantized, codes, scale)``."""
        x_dtype = x.dtype
        if not (self.ready() and self.bits < 16):
            return None, None, None
        _require_cuda(x)
        shape = x.shape
        x2 = x.reshape(shape[0], -1).float().contiguous()
        rows, cols = x2.shape
        if self.weight_groupsize > 0:
            g = self.weight_groupsize
            ldp = cols // g
        else:
            g = -1
            ldp = 1
        scale = self.scale.float().contiguous()
        zero = self.zero.float().contiguous()
        if g == -1 and scale.numel() == 1 and rows > 1:
            scale = scale.reshape(1).expand(rows).contiguous()
            zero = zero.reshape(1).expand(rows).contiguous()
        fq = torch.empty_like(x2)
        q = torch.empty_like(x2)
        _lib.call("g2ptq_fake_quantize", _lib.stream_ptr(x.device), _lib.ptr(x2), rows, cols, cols,
                  g, _lib.ptr(scale), _lib.ptr(zero), ldp, self.bits, _lib.ptr(fq), cols,
                  _lib.ptr(q), cols, None)
        return fq.view(shape).to(x_dtype), q.view(shape), self.scale

    def enabled(self):
        return self.maxq > 0

    def ready(self):
        return self._ready


def check_flags(flags):
    """Raise the reference's errors for device-side failure flags (one host sync)."""
    v = int(flags.max().item()) if flags.numel() > 1 else int(flags.item())
    if v & _lib.FLAG_BAD_SCALE:
        raise RuntimeError("quantization scale must be positive "
                           "(utils/quant_utils.py: scale.min() > 0 assertion)")
    if v & _lib.FLAG_NAN_OUTPUT:
        raise ValueError("NaN in weights")
