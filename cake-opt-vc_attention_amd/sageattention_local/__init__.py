"""MI355X (gfx950) implementation of the reference's sageattention_local.vc surface."""
from .vc import forward_prepared, kernel_resources, prepare, sage_vc_build_info, sageattn_vc, validate_inputs

__all__ = ["sageattn_vc", "prepare", "forward_prepared", "validate_inputs", "kernel_resources",
           "sage_vc_build_info"]
