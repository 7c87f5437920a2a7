"""ctypes binding of ``libg2ptq_hip.so`` (the C ABI declared in include/g2ptq_hip.h).

There is no fallback: if the library is missing or cannot be loaded, every
entry point raises.  Build it with ``python -m g2ptq_amd.build``.
"""
import ctypes
import os

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libg2ptq_hip.so")

FLAG_BAD_SCALE = 1
FLAG_NAN_OUTPUT = 2
FLAG_GROUP_SCALE = 4
VARIANT_GPTQ, VARIANT_GPTAQ, VARIANT_G2PTQ = 0, 1, 2

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_sz = ctypes.c_size_t
_szp = ctypes.POINTER(ctypes.c_size_t)

# name -> argtypes (all functions return int status except the two string ones)
SIGNATURES = {
    "g2ptq_abi_version": [],
    "g2ptq_find_params": [_p, _p, _i64, _i64, _i64, _i32, _i32, _p, _p, _i64, _p],
    "g2ptq_find_params_mse": [_p, _p, _i64, _i64, _i64, _i32, _i32, _f32, _i32, _f32, _p, _i64,
                              _i64, _i64, _p, _p, _i64, _p],
    "g2ptq_fake_quantize": [_p, _p, _i64, _i64, _i64, _i64, _p, _p, _i64, _i32, _p, _i64, _p, _i64, _p],
    "g2ptq_hessian_workspace": [_i64, _i64, _i32, _i64, _szp],
    "g2ptq_hessian_update": [_p, _p, _i64, _i64, _i64, _f32, _f32, _p, _i64, _p, _sz],
    "g2ptq_hessian_stage_rows": [_i64, ctypes.POINTER(ctypes.c_int64)],
    "g2ptq_hessian_stage": [_p, _p, _i64, _i64, _i64, _p, _i64, _i64],
    "g2ptq_hessian_gram_workspace": [_i64, _i64, _szp],
    "g2ptq_hessian_gram": [_p, _p, _i64, _i64, _i64, _f32, _f32, _p, _i64, _p, _sz],
    "g2ptq_gptaq_update": [_p, _p, _p, _i64, _i64, _i64, _i64, _f32, _f32, _p, _p, _i64, _p, _sz],
    "g2ptq_gptaq_stage": [_p, _p, _p, _i64, _i64, _i64, _i64, _p, _i64, _i64],
    "g2ptq_gptaq_gram_workspace": [_i64, _i64, _szp],
    "g2ptq_gptaq_gram": [_p, _p, _i64, _i64, _i64, _f32, _f32, _p, _p, _i64, _p, _sz],
    "g2ptq_weighted_hessian_update": [_p, _p, _i64, _i64, _i64, _p, _i64, _i64, _f32, _f32, _p, _i64,
                                      _i64, _p, _f32, _f32, _p, _sz],
    "g2ptq_weighted_stage": [_p, _p, _i64, _i64, _i64, _p, _i64, _i64, _f32, _p, _i64, _i64, _p, _f32,
                             _f32],
    "g2ptq_weighted_gram_workspace": [_i64, _i64, _i64, _szp],
    "g2ptq_weighted_gram": [_p, _p, _i64, _i64, _i64, _i64, _f32, _f32, _p, _i64, _i64, _p, _sz],
    "g2ptq_hessian_stage_planes": [_i32, _i32, _i64, ctypes.POINTER(ctypes.c_int64)],
    "g2ptq_hessian_stage_height": [_i32, _i32, _i64, _i64, ctypes.POINTER(ctypes.c_int64)],
    "g2ptq_hessian_stage_ex": [_p, _i32, _i32, _p, _p, _i64, _i64, _i64, _i64, _p, _i64, _i64,
                               _f32, _p, _i64, _i64, _p, _f32, _f32],
    "g2ptq_hessian_gram_ex_workspace": [_i32, _i32, _i64, _i64, _i64, _szp],
    "g2ptq_hessian_gram_ex": [_p, _i32, _i32, _p, _i64, _i64, _i64, _i64, _f32, _f32, _p, _i64,
                              _i64, _p, _i64, _p, _sz],
    "g2ptq_prepare_hessian": [_p, _p, _i64, _i64, _p, _i64, _p, _p, _i64, _p, _sz],
    "g2ptq_factor_workspace": [_i64, _i64, _szp],
    "g2ptq_inv_chol_upper": [_p, _p, _i64, _i64, _f32, _p, _p, _p, _p, _sz],
    "g2ptq_block_sweep": [_p, _i32, _i64, _i64, _i64, _i32, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p],
    "g2ptq_compensate_workspace": [_i32, _i64, _i64, _i64, _i64, _szp],
    "g2ptq_compensate": [_p, _i32, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _p, _i32, _i32, _i64, _i32,
                         _i32, _f32, _f32, _p, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _sz],
    "g2ptq_compensate_noalloc": [_p, _i32, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _p, _i32,
                                 _i32, _i64, _i32, _i32, _f32, _f32, _p, _i64, _p, _p, _p, _p, _p,
                                 _p, _p],
    "g2ptq_gptaq_p": [_p, _p, _p, _i64, _i64, _f32, _p, _p, _sz],
    "g2ptq_trust_region": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _f32, _i32, _p, _p, _p, _p, _sz],
    "g2ptq_trust_region_workspace": [_i64, _i64, _i64, _szp],
    "g2ptq_act_order": [_p, _p, _i64, _i64, _i32, _p, _p, _p, _sz],
    "g2ptq_permute_cols": [_p, _p, _p, _i64, _i64, _p],
    "g2ptq_permute_sym": [_p, _p, _p, _i64, _i64, _p],
    "g2ptq_cast_check": [_p, _p, _p, _i64, _i32, _p],
    "g2ptq_to_f32": [_p, _p, _p, _i64, _i32],
    "g2ptq_staged_equal": [_p, _p, _i64, _p, _i64, _i64, _i64, _p],
    "g2ptq_pack_quantized": [_p, _p, _i64, _p, _i64, _i64, _i64, _i32, _i64, _p, _i64, _p, _i32, _i64,
                             _p],
    "g2ptq_concat": [_p, _p, _p, _i64, _i64, _p],
    "g2ptq_group_mean_square": [_p, _p, _i32, _i64, _i64, _i64, _i64, _p],
    "g2ptq_running_mean_update": [_p, _p, _p, _i32, _i64, _f32, _f32, _i32],
    "g2ptq_gemm_f32": [_p, _i64, _i64, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _i32, _p, _i64, _i64,
                       _p, _i64, _i64, _f32, _f32],
}
STRING_FUNCS = ("g2ptq_status_string", "g2ptq_last_error")

_LIB = None


class HipLibraryError(RuntimeError):
    pass


def load():
    """Load the library once; raise if it is missing (no CPU fallback exists)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise HipLibraryError(
            f"{LIB_PATH} not found: build it with `python -m g2ptq_amd.build` "
            "(the quantization path has no non-HIP fallback)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = ctypes.c_int
    for name in STRING_FUNCS:
        fn = getattr(lib, name)
        fn.restype = ctypes.c_char_p
    lib.g2ptq_status_string.argtypes = [ctypes.c_int]
    lib.g2ptq_last_error.argtypes = []
    _LIB = lib
    return lib


def call(name, *args):
    """Call an int-returning entry point and raise on a nonzero status."""
    lib = load()
    status = getattr(lib, name)(*args)
    if status != 0:
        raise_status(name, status)
    return status


def raise_status(name, status):
    """The exception for a nonzero status of entry point ``name``."""
    lib = load()
    detail = lib.g2ptq_last_error().decode(errors="replace")
    kind = lib.g2ptq_status_string(status).decode()
    if status == -1:
        raise ValueError(f"{name}: {kind}: {detail}")
    raise RuntimeError(f"{name}: {kind}: {detail}")


_FAST = None


def fastcall():
    """The CPython fast-call module of the per-batch staging entry points
    (``g2ptq_amd/_fastcall``, built with the library), or None when it is
    not built; it calls the same entry points as ``call``, without ctypes'
    per-argument conversions."""
    global _FAST
    if _FAST is None:
        load()  # the module links against the library loaded here
        try:
            from . import _fastcall
            _FAST = _fastcall
        except ImportError:
            _FAST = False
    return _FAST or None


def query_size(name, *args):
    out = ctypes.c_size_t(0)
    call(name, *args, ctypes.byref(out))
    return out.value


def query_size_i64(name, *args):
    out = ctypes.c_int64(0)
    call(name, *args, ctypes.byref(out))
    return out.value


def ptr(t):
    """Device pointer of a tensor as an integer (None → NULL); every entry
    point declares its pointer arguments ``c_void_p``, which takes either.
    Every kernel reads and writes device memory: a host tensor is refused
    here, as torch refuses to mix devices (an offloaded Hessian outside its
    onload context, a CPU input), before any kernel could touch it."""
    if t is None:
        return None
    if not t.is_cuda:
        raise RuntimeError(f"g2ptq_amd kernels take GPU tensors; got a {t.device} tensor "
                           f"of shape {tuple(t.shape)} (an offloaded Hessian is usable only "
                           "inside its onload context)")
    return t.data_ptr()


def stream_ptr(device=None):
    """The current stream of ``device`` (default: the current device), as an
    integer handle.  The raw device query skips ``torch.cuda.current_device``'s
    lazy-init checks: the callers already hold CUDA tensors."""
    if device is None or device.index is None:
        index = torch._C._cuda_getDevice()
    else:
        index = device.index
    return torch._C._cuda_getCurrentRawStream(index)


_WORKSPACES = {}


def workspace(nbytes, device):
    """A cached uint8 device buffer of at least ``nbytes`` bytes.

    Buffers are cached per (device, current stream) and reused across calls:
    the calls that use one buffer are enqueued on that stream, so stream order
    protects its reuse, and calls on different streams never share one.
    """
    nbytes = max(int(nbytes), 256)
    dev = torch.device(device)
    index = dev.index if dev.index is not None else torch.cuda.current_device()
    key = (index, torch._C._cuda_getCurrentRawStream(index))
    buf = _WORKSPACES.get(key)
    if buf is None or buf.numel() < nbytes:
        _WORKSPACES[key] = None
        buf = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        _WORKSPACES[key] = buf
    return buf


def release_workspaces():
    _WORKSPACES.clear()
