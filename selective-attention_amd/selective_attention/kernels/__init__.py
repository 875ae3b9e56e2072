"""Host launchers of the HIP kernels (replace the reference's triton_kernels/)."""
from .ssu import ssu_forward

__all__ = ["ssu_forward"]
