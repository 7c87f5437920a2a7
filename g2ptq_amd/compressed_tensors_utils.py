"""compressed-tensors export of quantized layers.

Drop-in for ``compress`` and ``register_qparam_buffers`` of
utils/compressed_tensors_utils.py (:22-53 of the reference), which stash a
layer's pack-quantized checkpoint tensors (``weight_packed``,
``weight_scale``, ``weight_shape``) for the compressed-tensors saver.  The
reference packs with ``pack_to_int32`` from compressed-tensors 0.18.0
(``requirements.txt:14``; the package is not a dependency here): codes as
int8, offset by 2^(bits−1) to unsigned fields, 32/bits consecutive input
columns per int32 with the first column in the lowest bits.  Packing and the
group-scale extraction run in one HIP launch (``g2ptq_pack_quantized``).
"""
import torch

from . import _core, _lib

Q_PARAMS = ("weight_packed", "weight_scale", "weight_shape")

_DTYPE_CODE = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


def _packed_words(columns, num_bits):
    pf = 32 // num_bits
    return (columns + pf - 1) // pf


def pack_to_int32(value, num_bits):
    """compressed-tensors 0.18.0 ``pack_to_int32(value, num_bits)`` (packed along
    the last dimension) for a 2-D int8 GPU tensor."""
    if value.dtype is not torch.int8:
        raise ValueError("Tensor must be quantized to torch.int8 before packing")
    if num_bits > 8:
        raise ValueError("Packing is only supported for less than 8 bits")
    if num_bits < 1:
        raise ValueError(f"num_bits must be at least 1, got {num_bits}")
    if not value.is_cuda:
        raise RuntimeError("pack_to_int32 runs on the GPU: pass a GPU tensor")
    rows, cols = value.shape
    codes = value.float().contiguous()
    words = _packed_words(cols, num_bits)
    packed = torch.empty(rows, words, dtype=torch.int32, device=value.device)
    _lib.call("g2ptq_pack_quantized", _lib.stream_ptr(value.device), _lib.ptr(codes), cols, None, 0,
              rows, cols, num_bits, 1, _lib.ptr(packed), words, None, 2, 0, None)
    return packed


def compress(layer, Scale, W_int, bits, groupsize):
    """utils/compressed_tensors_utils.py:22-45: stash the layer's packed codes,
    per-group scales (weight dtype) and shape in ``layer._export_qparams``.

    ``Scale`` and ``W_int`` are the compensation's per-element scales and
    integer codes (fp32, any shape with ``weight.numel()`` elements)."""
    weight = layer.weight
    rows, columns = weight.shape
    dtype, dev = weight.dtype, weight.device
    if dtype not in _DTYPE_CODE:
        raise NotImplementedError(f"compressed-tensors export of {dtype} weights")
    if columns % groupsize != 0:
        raise RuntimeError(f"shape '[{rows}, {columns // groupsize}, {groupsize}]' is invalid for "
                           f"input of size {rows * columns}")
    codes = W_int.reshape(rows, columns).float().contiguous()
    scale = Scale.reshape(rows, columns).float().contiguous()
    words = _packed_words(columns, bits)
    packed = torch.empty(rows, words, dtype=torch.int32, device=dev)
    wscale = torch.empty(rows, columns // groupsize, dtype=dtype, device=dev)
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    _lib.call("g2ptq_pack_quantized", _core.stream(), _lib.ptr(codes), columns, _lib.ptr(scale),
              columns, rows, columns, int(bits), int(groupsize), _lib.ptr(packed), words,
              _lib.ptr(wscale), _DTYPE_CODE[dtype], columns // groupsize, _lib.ptr(flags))
    if int(flags.item()) & _lib.FLAG_GROUP_SCALE:
        raise AssertionError("Scales in the same quantization group should be the same.")
    layer._export_qparams = {
        "weight_packed": packed,
        "weight_scale": wscale,
        "weight_shape": torch.tensor(weight.shape).to(dev).contiguous(),
    }


def compress_layers(layers, Scale, W_int, bits, groupsize, columns):
    """The ``export_compressed_tensors`` step of every ``fasterquant``
    (e.g. gptq_utils.py:336-344): ``compress`` per layer of the batch."""
    for b, layer in enumerate(layers):
        compress(layer, Scale[b], W_int[b], bits, columns if groupsize == -1 else groupsize)


def register_qparam_buffers(modules):
    """utils/compressed_tensors_utils.py:48-53: turn the stashed qparams into buffers."""
    for module in modules:
        qparams = module.__dict__.pop("_export_qparams", None)
        if qparams is None:
            continue
        for name, tensor in qparams.items():
            module.register_buffer(name, tensor)
