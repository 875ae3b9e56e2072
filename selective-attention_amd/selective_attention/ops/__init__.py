from .ssd_scan import SSDScanFn
from .ssu import SSUFn

__all__ = ["SSDScanFn", "SSUFn"]
