"""g2ptq_amd — MI355X-native GPTQ / GPTAQ / G2PTQ per-layer quantization path.

Host classes mirror the reference's per-layer quantizer interface
(gptq_utils/*_utils.py and utils/quant_utils.py of G2PTQ/G2PTQ); every
numeric step runs in the HIP library ``libg2ptq_hip.so`` (gfx950 kernels
behind the C ABI of include/g2ptq_hip.h).
"""
from . import _lib
from .common_utils import (ChunkSpec, build_chunk_specs, fake_quantize_grouped,
                           make_group_quantizers, merge_group_quantizers)
from .g2ptq_utils import G2PTQ
from .gptaq_utils import GPTAQ
from .gptq_guided_utils import GPTQGuided
from .gptq_utils import GPTQ
from .graph_utils import clear_graph_cache, run_graph, validate_tensors
from .quant_utils import WeightQuantizer
from .shared import SharedInputHessian

__all__ = [
    "GPTQ", "GPTAQ", "G2PTQ", "GPTQGuided", "WeightQuantizer", "ChunkSpec", "build_chunk_specs",
    "make_group_quantizers", "merge_group_quantizers", "fake_quantize_grouped", "run_graph",
    "validate_tensors", "clear_graph_cache", "SharedInputHessian",
]


def library_path():
    return _lib.LIB_PATH
