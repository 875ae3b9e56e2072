"""Host launchers of the HIP kernels (replace the reference's triton_kernels/)."""
from .ssd_scan import ssd_scan_backward, ssd_scan_forward
from .ssu import ssu_forward

__all__ = ["ssd_scan_forward", "ssd_scan_backward", "ssu_forward"]
