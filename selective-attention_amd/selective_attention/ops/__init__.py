from .ssu import SSUFn

__all__ = ["SSUFn"]
