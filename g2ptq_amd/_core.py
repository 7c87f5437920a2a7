"""Host-side steps shared by the GPTQ / GPTAQ / G2PTQ / GuidedQuant classes.

Every numeric step is a call into libg2ptq_hip.so on the current HIP stream;
torch is used only to allocate device memory and to hold tensors.
"""
import contextlib
import logging
import math

import numpy as np
import torch

from . import _lib
from .quant_utils import check_flags

HIP_BACKENDS = ("hip",)
_DTYPE_CODE = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


def check_backend(backend):
    """The reference's backends are ``torch``/``triton``; this build provides ``hip``."""
    if backend not in HIP_BACKENDS:
        raise NotImplementedError(
            f"backend={backend!r} is not provided by g2ptq_amd; use backend='hip' "
            "(every compensation kernel of this package is a HIP kernel)")


def f32(x):
    """Round a Python number to float32 the way a 0-d fp32 tensor op would."""
    return float(np.float32(x))


def stream():
    return _lib.stream_ptr()


def stack_weights_f32(layers):
    """``torch.stack([l.weight for l in layers]).float()`` via the HIP cast kernel."""
    w0 = layers[0].weight
    B = len(layers)
    R, C = w0.shape
    W = torch.empty(B, R, C, device=w0.device, dtype=torch.float32)
    for b, layer in enumerate(layers):
        w = layer.weight.data
        if not w.is_contiguous():
            w = w.contiguous()
        code = _DTYPE_CODE.get(w.dtype)
        if code is None:
            raise TypeError(f"unsupported weight dtype {w.dtype}")
        _lib.call("g2ptq_to_f32", stream(), _lib.ptr(w), _lib.ptr(W[b]), w.numel(), code)
    return W


def write_back(layers, Q, flags):
    """Cast ``Q[b]`` into ``layers[b].weight`` (gptq_utils.py:346-353) with a NaN check."""
    for b, layer in enumerate(layers):
        w = layer.weight.data
        code = _DTYPE_CODE.get(w.dtype)
        if code is None:
            raise TypeError(f"unsupported weight dtype {w.dtype}")
        q = Q[b]
        if w.is_contiguous():
            _lib.call("g2ptq_cast_check", stream(), _lib.ptr(q), _lib.ptr(w), q.numel(), code,
                      _lib.ptr(flags))
        else:
            tmp = torch.empty(w.shape, dtype=w.dtype, device=w.device)
            _lib.call("g2ptq_cast_check", stream(), _lib.ptr(q), _lib.ptr(tmp), q.numel(), code,
                      _lib.ptr(flags))
            w.copy_(tmp)


def as_tokens(inp):
    """Flatten a hook payload to (T, C) contiguous and return it with its
    activation dtype code (0 bf16, 1 fp16, 2 fp32): the reference accepts any
    float input (``inp.float()``, gptq_utils.py:125).  bf16 is staged as is,
    fp16 and fp32 as two and three bf16 planes that sum to it exactly; fp64
    and other types are refused."""
    x = inp if inp.dim() == 2 else inp.reshape(-1, inp.shape[-1])
    code = _DTYPE_CODE.get(x.dtype)
    if code is None:
        raise NotImplementedError(
            f"Hessian accumulation takes bf16, fp16 or fp32 activations (got {x.dtype})")
    if not x.is_contiguous():
        x = x.contiguous()
    if not x.is_cuda:
        raise RuntimeError("Hessian accumulation requires GPU tensors")
    return x, code


def hessian_update(H, X, alpha, beta):
    """H = beta·H + alpha·XᵀX for one layer's (C, C) Hessian."""
    T, C = X.shape
    nbytes = _lib.query_size("g2ptq_hessian_workspace", T, C, 0, 0)
    ws = _lib.workspace(nbytes, X.device)
    _lib.call("g2ptq_hessian_update", stream(), _lib.ptr(X), T, C, C, f32(alpha), f32(beta),
              _lib.ptr(H), C, _lib.ptr(ws), ws.numel())


def gptaq_update(H, Dx, X, Xfp, alpha, beta):
    T, C = X.shape
    nbytes = _lib.query_size("g2ptq_hessian_workspace", T, C, 1, 0)
    ws = _lib.workspace(nbytes, X.device)
    _lib.call("g2ptq_gptaq_update", stream(), _lib.ptr(X), _lib.ptr(Xfp), T, C, C, C, f32(alpha),
              f32(beta), _lib.ptr(H), _lib.ptr(Dx), C, _lib.ptr(ws), ws.numel())


def weighted_update(Hg, X, S, alpha, beta, act, act_alpha, act_beta):
    """Hg (G, C, C) = beta·Hg + alpha·Σ_t S[t,g] x xᵀ; act = act_beta·act + act_alpha·Σ x²."""
    T, C = X.shape
    G = S.shape[1]
    S = S.float().contiguous()
    nbytes = _lib.query_size("g2ptq_hessian_workspace", T, C, 2, G)
    ws = _lib.workspace(nbytes, X.device)
    _lib.call("g2ptq_weighted_hessian_update", stream(), _lib.ptr(X), T, C, C, _lib.ptr(S), G, G,
              f32(alpha), f32(beta), _lib.ptr(Hg), C, C * C, _lib.ptr(act), f32(act_alpha),
              f32(act_beta), _lib.ptr(ws), ws.numel())


def prepare_hessian(H, W, Dx=None, Grad=None):
    """Zero-H → identity, dead columns (gptq_utils.py:272-277 and variants), in place."""
    B, C, _ = H.shape
    R = W.shape[1]
    Rg = Grad.shape[1] if Grad is not None else 0
    nbytes = (B * 8 + 255) // 256 * 256 + (B * C * 4 + 255) // 256 * 256
    ws = _lib.workspace(nbytes, H.device)
    _lib.call("g2ptq_prepare_hessian", stream(), _lib.ptr(H), B, C, _lib.ptr(W), R, _lib.ptr(Dx),
              _lib.ptr(Grad), Rg, _lib.ptr(ws), ws.numel())


def act_order(src, key_mode):
    """Shared permutation (descending key, ties by index) and its inverse, int32 on device."""
    C = src.shape[-1]
    B = src.shape[0]
    perm = torch.empty(C, dtype=torch.int32, device=src.device)
    inv = torch.empty(C, dtype=torch.int32, device=src.device)
    ws = _lib.workspace(C * 4, src.device)
    _lib.call("g2ptq_act_order", stream(), _lib.ptr(src.contiguous()), B, C, key_mode,
              _lib.ptr(perm), _lib.ptr(inv), _lib.ptr(ws), ws.numel())
    return perm, inv


def permute_cols(M, cols):
    """``M[..., cols]`` for a contiguous fp32 tensor (new tensor)."""
    out = torch.empty_like(M)
    C = M.shape[-1]
    _lib.call("g2ptq_permute_cols", stream(), _lib.ptr(M), _lib.ptr(out), M.numel() // C, C,
              _lib.ptr(cols))
    return out


def permute_sym(H, perm):
    """``H[b][perm][:, perm]`` for every b (new tensor)."""
    out = torch.empty_like(H)
    B, C, _ = H.shape
    _lib.call("g2ptq_permute_sym", stream(), _lib.ptr(H), _lib.ptr(out), B, C, _lib.ptr(perm))
    return out


def factor(H, percdamp, shared=None, key=None, alias=None):
    """U[b] = chol((H[b] + p·mean(diag)·I)⁻¹, upper) with the reference's retry loop.

    gptq_utils.py:291-311: on a failed factorization (non-PD pivot or NaN) the
    damp is raised by 0.0015 and the layer is factored again; a damp leaving
    (0, 1) raises ``ValueError``.  Layers that succeed keep their damp.
    ``shared`` (a SharedInputHessian whose members are all of H's slots, so all
    slots hold the same matrix) factors one slot once and reuses the result.
    ``alias`` ({slot: earlier slot holding the same matrix}) factors only the
    other slots and gives each aliased slot its source's U and damp: the
    factor of a slot depends on that slot alone, so the result is the same.
    """
    B, C, _ = H.shape
    if shared is None and alias:
        src = [b for b in range(B) if b not in alias]
        pos = {b: i for i, b in enumerate(src)}
        if len(src) < B and all(alias[b] in pos for b in alias):
            dev = H.device
            Uu, du = factor(H.index_select(0, torch.tensor(src, device=dev)), percdamp)
            at = [pos[alias.get(b, b)] for b in range(B)]
            return Uu.index_select(0, torch.tensor(at, device=dev)), [du[i] for i in at]
    if shared is not None:
        ck = (percdamp, key)
        hit = shared.cached_factor(ck)
        if hit is None:
            U1, d1 = factor(H[:1], percdamp)
            hit = (U1[0], d1[0])
            shared.store_factor(ck, *hit)
        if B == 1:  # the cached factor itself: every later use only reads it
            return hit[0].unsqueeze(0), [hit[1]]
        U = torch.empty_like(H)
        U.copy_(hit[0].unsqueeze(0).expand(B, C, C))
        return U, [hit[1]] * B
    dev = H.device
    U = torch.empty_like(H)
    info = torch.zeros(B, dtype=torch.int32, device=dev)
    skip = torch.zeros(B, dtype=torch.int32, device=dev)
    ws = _lib.workspace(_lib.query_size("g2ptq_factor_workspace", B, C), dev)
    done = [False] * B
    damp_percent = percdamp
    damps = [None] * B
    while 1 > damp_percent > 0:
        _lib.call("g2ptq_inv_chol_upper", stream(), _lib.ptr(H), B, C, f32(damp_percent),
                  _lib.ptr(skip), _lib.ptr(U), _lib.ptr(info), _lib.ptr(ws), ws.numel())
        status = info.cpu().tolist()
        failed = False
        for b in range(B):
            if done[b]:
                continue
            if status[b] == 0:
                done[b] = True
                damps[b] = damp_percent
            else:
                failed = True
        if not failed:
            break
        logging.warning(f"Quantization: Current `damp_percent = {damp_percent:.5f}` is too low, "
                        f"auto-incrementing by `{0.0015:.5f}`")
        damp_percent += 0.0015
        skip = torch.tensor([1 if d else 0 for d in done], dtype=torch.int32, device=dev)
    if not (0 < damp_percent < 1):
        raise ValueError(f"Quantization: `damp_percent` must between 0 and 1. current is {damp_percent}")
    return U, damps


def param_tables(quantizers, BR, groupsize, static_groups, device):
    """(ngroups, B·R) scale/zero tables; pre-filled unless groups are dynamic."""
    ngroups = len(quantizers)
    dynamic = groupsize != -1 and not static_groups
    if dynamic:
        s = torch.empty(ngroups, BR, device=device, dtype=torch.float32)
        z = torch.empty(ngroups, BR, device=device, dtype=torch.float32)
        return s, z, True
    qs = quantizers[:1] if groupsize == -1 else quantizers
    for q in qs:
        if not q.ready():
            raise RuntimeError("quantizer parameters are not fitted (call find_params first)")
    s = torch.stack([q.scale.reshape(-1).float() for q in qs]).contiguous()
    z = torch.stack([q.zero.reshape(-1).float() for q in qs]).contiguous()
    return s, z, False


def mse_config(quantizer):
    if getattr(quantizer, "mse", False):
        return int(quantizer.grid), float(quantizer.norm), float(quantizer.maxshrink)
    return 0, 2.4, 0.5


def hclip_rows(quantizers, H_diag, groupsize, static_groups, rows, C, dev):
    """The (blocks, C) Hessian diagonal the dynamic-group clip searches of the
    compensation loop weight their error with (gptq_utils.py:194-205 passes
    ``H_diag[:, i:i+g]`` to ``find_params``), or None when they use none."""
    q0 = quantizers[0]
    if groupsize == -1 or static_groups or not getattr(q0, "hclip", False):
        return None
    if H_diag is None:
        raise AttributeError("WeightQuantizer with hclip=True needs H_diag "
                             "('NoneType' object has no attribute 'shape')")
    nb = H_diag.shape[0]
    if H_diag.dim() != 2 or H_diag.shape[1] != C or nb == 0 or rows % nb != 0:
        raise RuntimeError(f"H_diag of shape {tuple(H_diag.shape)} does not split {rows} rows "
                           f"of {C} columns")
    if not getattr(q0, "mse", False):
        return None  # only the clip search reads it
    return H_diag.to(device=dev, dtype=torch.float32).contiguous()


def compensate(variant, W, U, quantizers, blocksize, groupsize, static_groups, qparam_perm,
               flags, P=None, Z=None, GH=None, H_diag=None):
    """Native lazy-batch loop (``_run_compensation``); returns (Q, W_int, Scale).

    W (B, R, C) is updated in place with every block tail, like the reference.
    Dynamic group quantizers receive their fitted parameters.  ``H_diag``
    (blocks, C) weights their clip search when the quantizers use ``hclip``.
    """
    B, R, C = W.shape
    dev = W.device
    if blocksize > 128:
        raise ValueError(f"blocksize {blocksize} > 128 is not supported by the HIP sweep")
    for t in (W, U, P, Z, GH):
        if t is not None and (not t.is_cuda or not t.is_contiguous() or t.dtype != torch.float32):
            raise ValueError("compensation operands must be contiguous fp32 GPU tensors")
    stab, ztab, dynamic = param_tables(quantizers, B * R, groupsize, static_groups, dev)
    colgroup = None
    if groupsize != -1 and static_groups and qparam_perm is not None:
        colgroup = (qparam_perm.to(dev).long() // groupsize).to(torch.int32).contiguous()
    grid, norm, shrink = mse_config(quantizers[0])
    hd = hclip_rows(quantizers, H_diag, groupsize, static_groups, B * R, C, dev)
    Q = torch.empty_like(W)
    W_int = torch.empty_like(W)
    Scale = torch.empty_like(W)
    nbytes = _lib.query_size("g2ptq_compensate_workspace", variant, B, R, C, blocksize)
    ws = _lib.workspace(nbytes, dev)
    bits = quantizers[0].bits
    _lib.call("g2ptq_compensate", stream(), variant, B, R, C, blocksize, _lib.ptr(W), _lib.ptr(U),
              _lib.ptr(P), _lib.ptr(Z), _lib.ptr(GH), bits, int(quantizers[0].sym), groupsize,
              int(bool(static_groups)), grid, norm, shrink, _lib.ptr(hd),
              hd.shape[0] if hd is not None else 0, _lib.ptr(colgroup), _lib.ptr(stab),
              _lib.ptr(ztab), _lib.ptr(Q), _lib.ptr(W_int), _lib.ptr(Scale), _lib.ptr(flags),
              _lib.ptr(ws), ws.numel())
    if dynamic:
        scales = stab.view(len(quantizers), B * R, 1).unbind(0)
        zeros = ztab.view(len(quantizers), B * R, 1).unbind(0)
        for q, s_i, z_i in zip(quantizers, scales, zeros):
            # the registered buffers, set directly (nn.Module.__setattr__ per
            # attribute costs more than the rest of this loop)
            q._buffers["scale"] = s_i
            q._buffers["zero"] = z_i
            q.__dict__["_ready"] = True
    return Q, W_int, Scale


def fit_static_params(quantizers, W_flat, groupsize, static_groups, flags, H_diag=None):
    """gptq_utils.py:259-270: fit group params on the unpermuted weights."""
    if groupsize == -1 or static_groups:
        for i, q in enumerate(quantizers):
            if not q.ready():
                if groupsize == -1:
                    q.find_params(W_flat, H_diag, _flags=flags)
                else:
                    sl = slice(i * groupsize, (i + 1) * groupsize)
                    q.find_params(W_flat[:, sl], None if H_diag is None else H_diag[:, sl],
                                  _flags=flags)


def hessian_diag(H, hclip):
    """``torch.diagonal(H, dim1=-2, dim2=-1).clone()`` when hclip is on
    (gptq_utils.py:253-257), else None."""
    if not hclip:
        return None
    return torch.diagonal(H, dim1=-2, dim2=-1).clone()


@contextlib.contextmanager
def onload_attrs(owner, names, enabled=True, device=None):
    """Move ``owner.<name>`` to ``device`` for the duration of the block, then back
    to (pinned) host memory — the effect of offload_utils.onload_attrs
    (utils/offload_utils.py:173-201)."""
    if not enabled:
        yield
        return
    staged = {}
    for n in names:
        host = getattr(owner, n, None)
        if host is not None:
            staged[n] = host
            _swap(owner, n, host.to(device=device, non_blocking=host.is_pinned()))
    try:
        yield
    finally:
        for n in names:
            v = getattr(owner, n, None)
            if v is None or v.device.type == "cpu":
                continue
            host = staged.get(n)
            if host is None or host.shape != v.shape or host.dtype != v.dtype:
                host = torch.empty(v.shape, dtype=v.dtype, pin_memory=True)
            host.copy_(v)
            _swap(owner, n, host)


def _swap(owner, name, value):
    """``owner.<name> = value`` for a copy of the same values on another
    device: the attribute's setter keeps what it derived from the old
    tensor (a shared-input group's cached factor, slot copies)."""
    owner.__dict__["_same_values"] = True
    try:
        setattr(owner, name, value)
    finally:
        owner.__dict__.pop("_same_values", None)


def alloc(shape, device, dtype=torch.float32, pin=False):
    """Zeroed tensor (page-locked when it lives on the host and ``pin``)."""
    pin_memory = bool(pin) and torch.device(device).type == "cpu" and torch.cuda.is_available()
    return torch.zeros(*shape, dtype=dtype, device=device, pin_memory=pin_memory)


def finish(flags):
    """The reference's end-of-fasterquant synchronisation plus its error checks."""
    torch.cuda.synchronize()
    check_flags(flags)


def sqrt_scale_sq(n):
    """alpha matching ``(sqrt(2/n)·x)ᵀ(sqrt(2/n)·x)`` of gptq_utils.py:125-126."""
    s = f32(math.sqrt(f32(2.0 / n)))
    return f32(s * s)
