"""Import name of the reference package (``neural_shift_cuda``), served by
``neural_shift_cuda_amd``.

``neural_shift_cuda.ops``, ``neural_shift_cuda.metropolis`` and
``neural_shift_cuda._C`` resolve to the same module objects as their
``neural_shift_cuda_amd`` counterparts, so module-level state (for example
``ops._HAS_CUDA_EXT``) is shared and private helpers such as
``neural_shift_cuda.ops._prep_shifts_for_cuda`` are reachable.
"""
import sys as _sys

import neural_shift_cuda_amd as _impl
from neural_shift_cuda_amd import metropolis, ops  # noqa: F401
from neural_shift_cuda_amd import *  # noqa: F401,F403
from neural_shift_cuda_amd import __all__, __version__  # noqa: F401

_sys.modules[__name__ + ".ops"] = _impl.ops
_sys.modules[__name__ + ".metropolis"] = _impl.metropolis

# model installers: neural_shift_cuda.integration and its patch modules
from neural_shift_cuda_amd import integration  # noqa: E402,F401

_sys.modules[__name__ + ".integration"] = integration
for _name in ("nekde_drunet_attn_patch", "gasd_drunet_attn_patch", "nkd_metropolis_attn_patch",
              "nectr_patch"):
    _sys.modules[f"{__name__}.integration.{_name}"] = getattr(integration, _name)
