"""Oracle: compressed-tensors pack-quantized export (test infrastructure only).

Restates ``compress`` of utils/compressed_tensors_utils.py:22-45 and the
packing it calls, ``pack_to_int32`` from compressed-tensors 0.18.0
(requirements.txt:14), which is absent here.  Its published format
("pack-quantized", the uint4b8 / uint8b128 layouts its readers consume): the
int8 code plus 2^(bits−1) as an unsigned bits-wide field, 32 // bits
consecutive input columns per int32 word, the first column in the lowest
bits, columns past the end zero.

Also the MoE expert stacking of the checkpoint (utils/models/mixins.py:93-144).

Parity: no reference test or fixture covers packing, and the library is
absent, so this restatement is pinned by hand-derived known answers of the
format, by an independent bit-by-bit unpacker (round trip) and by the field
layout (tests/test_oracle_pins.py).  The stacking is pinned element by
element against its index map.
"""
import numpy as np
import torch


def pack_to_int32(value, num_bits):
    """compressed-tensors 0.18.0 ``pack_to_int32(value, num_bits)`` (packed_dim=1)."""
    if value.dtype is not torch.int8:
        raise ValueError("Tensor must be quantized to torch.int8 before packing")
    if num_bits > 8:
        raise ValueError("Packing is only supported for less than 8 bits")
    offset = 1 << (num_bits - 1)
    v = (value.numpy().astype(np.int64) + offset) & ((1 << num_bits) - 1)
    pf = 32 // num_bits
    rows, cols = v.shape
    words = -(-cols // pf)
    padded = np.zeros((rows, words * pf), dtype=np.int64)
    padded[:, :cols] = v
    packed = np.zeros((rows, words), dtype=np.int64)
    for i in range(pf):
        packed |= padded[:, i::pf] << (num_bits * i)
    return torch.from_numpy(packed.astype(np.uint32).view(np.int32))


def compress(weight_shape, weight_dtype, Scale, W_int, bits, groupsize):
    """utils/compressed_tensors_utils.py:22-45: the ``_export_qparams`` dict."""
    rows, columns = weight_shape
    quantized_weight = W_int.reshape(weight_shape).to(torch.int8)
    group_scale = Scale.reshape(rows, columns // groupsize, groupsize)
    assert (group_scale == group_scale[..., 0:1]).all(), \
        "Scales in the same quantization group should be the same."
    return {
        "weight_packed": pack_to_int32(quantized_weight, bits).contiguous(),
        "weight_scale": group_scale[:, :, 0].to(weight_dtype).contiguous(),
        "weight_shape": torch.tensor(weight_shape).contiguous(),
    }


def stack_experts(gate, up, down, weight_packed=False):
    """utils/models/mixins.py:93-144 on CPU tensors.

    ``gate``, ``up``, ``down``: per-expert dicts of the modules' tensors
    (``weight``, or ``weight_packed`` / ``weight_scale`` / ``weight_shape``).
    Returns the attributes the reference sets on the experts container.
    """
    E = len(gate)
    if weight_packed:
        out = {
            "gate_up_proj_packed": torch.stack(
                [torch.cat([gate[i]["weight_packed"], up[i]["weight_packed"]], dim=0)
                 for i in range(E)], dim=0),
            "down_proj_packed": torch.stack([down[i]["weight_packed"] for i in range(E)], dim=0),
            "gate_up_proj_scale": torch.stack(
                [torch.cat([gate[i]["weight_scale"], up[i]["weight_scale"]], dim=0)
                 for i in range(E)], dim=0),
            "down_proj_scale": torch.stack([down[i]["weight_scale"] for i in range(E)], dim=0),
        }
        inter = int(gate[0]["weight_shape"][0])
        hidden = int(gate[0]["weight_shape"][1])
        out["gate_up_proj_shape"] = torch.tensor((E, 2 * inter, hidden))
        out["down_proj_shape"] = torch.tensor((E, hidden, inter))
        return out
    return {
        "gate_up_proj": torch.stack([torch.cat([gate[i]["weight"], up[i]["weight"]], dim=0)
                                     for i in range(E)], dim=0),
        "down_proj": torch.stack([down[i]["weight"] for i in range(E)], dim=0),
    }
