"""``neural_shift_cuda._C``: the HIP library module of neural_shift_cuda_amd.

Importing it raises the library's load error when it has not been built.
"""
import sys as _sys

from neural_shift_cuda_amd import _C as _impl

_sys.modules[__name__] = _impl
