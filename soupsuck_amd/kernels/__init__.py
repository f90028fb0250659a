"""Host-side entry points of the HIP kernels (same names as the reference's solution/kernels)."""

from .add_rmsnorm import add_rms_norm
from .cross_entropy import fused_linear_cross_entropy
from .lora_epilogue import lora_epilogue
from .nf4 import dequantize_nf4
from .nf4_gemm import gemm_f16, nf4_matmul
from .rmsnorm import rms_norm
from .rope import fused_rope
from .swiglu import swiglu, swiglu_fused_backward, swiglu_fused_forward

__all__ = ["add_rms_norm", "fused_linear_cross_entropy", "lora_epilogue", "dequantize_nf4",
           "gemm_f16", "nf4_matmul", "rms_norm", "fused_rope", "swiglu", "swiglu_fused_forward", "swiglu_fused_backward"]
