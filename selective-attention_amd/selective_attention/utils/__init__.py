from .tensor_utils import check_ndim, check_shape, to_contiguous

__all__ = ["check_ndim", "check_shape", "to_contiguous"]
