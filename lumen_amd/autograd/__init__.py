"""Reverse-mode autograd over traced graphs (``lumen.autograd``)."""

from lumen_amd.autograd.function import Function, FunctionCtx
from lumen_amd.autograd.transforms import backward, grad, value_and_grad, vjp

__all__ = ["Function", "FunctionCtx", "backward", "grad", "value_and_grad", "vjp"]
