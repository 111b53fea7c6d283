"""MI355X (gfx950) implementation of the GPTQ+ per-linear quantization hot path.

``GPTQPlus``, ``GPTQ`` and ``WeightQuantizer`` are drop-ins for the reference classes of the
same names; all arithmetic runs in the HIP library built by ``gptq_plus_mp_quant_amd.build``.
"""
from .export import dequantize_packed, export_packed, load_packed, save_packed
from .gptq import GPTQ
from .gptq_plus import GPTQPlus, add_batch_shared, fasterquant_shared
from .quant_utils import WeightQuantizer, get_minq_maxq

__all__ = ["GPTQPlus", "GPTQ", "WeightQuantizer", "add_batch_shared", "fasterquant_shared", "get_minq_maxq",
           "export_packed",
           "dequantize_packed", "save_packed", "load_packed"]
__version__ = "0.1.0"
