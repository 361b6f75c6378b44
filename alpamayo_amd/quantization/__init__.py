"""Quantized-Linear modules and converters of the ParoQuant W4A8 path.

Mirrors src/alpamayo_r1/utils/quantization/ of the reference (module and
class names, constructor arguments, buffers and state-dict keys).
"""

from .paroquant_marlin_w4a8 import (  # noqa: F401
    AWQBuffers,
    BF16RotateLinearWrapper,
    MarlinW4A8Linear,
    SharedInputRotateLinears,
    convert_model_to_marlin_w4a8,
    convert_wqlinear_layer,
    dequant_awq,
    dequant_wqlinear,
    load_paroquant_checkpoint,
    pack_awq_int32,
    replace_linears_with_rotate_linear,
    unpack_awq_int32,
    unpack_wqlinear_qweight,
    wqlinear_to_awq,
)
from .qmodule import WQLinear, calculate_zeros_width, pack_intweight  # noqa: F401
from .quantization_utils import pseudo_quantize_tensor  # noqa: F401
from .rotation_linear import RotateLinearInt4, Rotation, check_rotation_pairs  # noqa: F401
from .rotation_utils import apply_rotation_step, quantizer, rotate_tensor  # noqa: F401
