"""MI355X (gfx950) routed-MoE expert FFN for QuantaWeave.

Drop-in Python surface over the C ABI in include/qwmoe.h:

* ``TopKMoE``, ``SparseSwiGLU``, ``QuantaWeaveConfig``, ``set_moe_kernel``
  (src/quantweave_moe_model.py)
* ``moe_kernels``: ``kernels_available``, ``experts_support_grouped``,
  ``GroupedPlan``, ``grouped_matmul``, ``grouped_swiglu``, ``compute_dtype``,
  ``benchmark`` (src/moe_kernels.py)
* ``QuantizedLinear``, ``quantize_model`` (src/quantization.py)
* ``save_quantized``, ``read_quantized``, ``load_quantized_moe``: the quantised
  on-disk format (src/quantization.py:105-117), read without pickle
* ``MoEDecodeStep``: the routed experts of FastDecoder's one-token step
  (src/fast_decode.py:170-177), capturable in a HIP graph
"""

from . import moe_kernels
from .decode import MoEDecodeStep
from .moe import QuantaWeaveConfig, SparseSwiGLU, TopKMoE, set_moe_kernel
from .quantization import QuantizedLinear, quantize_model
from .checkpoint import load_quantized_moe, read_quantized, save_quantized

__all__ = [
    "QuantaWeaveConfig", "SparseSwiGLU", "TopKMoE", "set_moe_kernel", "QuantizedLinear", "quantize_model",
    "moe_kernels", "MoEDecodeStep", "save_quantized", "read_quantized", "load_quantized_moe",
]
