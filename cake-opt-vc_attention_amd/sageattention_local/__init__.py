"""MI355X (gfx950) implementation of the reference's sageattention_local.vc and .vc_fp8 surfaces."""
from .vc import forward_prepared, kernel_resources, prepare, sage_vc_build_info, sageattn_vc, validate_inputs
from .vc_fp8 import sageattn_vc_fp8

__all__ = ["sageattn_vc", "sageattn_vc_fp8", "prepare", "forward_prepared", "validate_inputs", "kernel_resources",
           "sage_vc_build_info"]
