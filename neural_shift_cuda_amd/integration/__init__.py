"""Model installers: patch a model class so that its shift-window work runs
on this package's ops (reference neural_shift_cuda/integration/__init__.py).

    from neural_shift_cuda.integration import install_cuda_shift_attn
    install_cuda_shift_attn(NeKDeDRUNetAttn)          # NeKDe, half-plane

    install_cuda_shift_gasd(GASDDRUNetAttn)           # GASD, full window
    install_cuda_shift_metropolis(NeKDeMetropolisDRUNetAttn)
    install_cuda_shift_nectr(NECTR_denoiser)          # official NECTR / nekre

Each installer is idempotent and leaves model math and parameters alone;
``model.use_cuda_shift = False`` restores the class's own methods per
instance.
"""
from .gasd_drunet_attn_patch import install_cuda_shift as install_cuda_shift_gasd
from .nectr_patch import install_cuda_shift as install_cuda_shift_nectr
from .nekde_drunet_attn_patch import install_cuda_shift as install_cuda_shift_attn
from .nkd_metropolis_attn_patch import install_cuda_shift as install_cuda_shift_metropolis

__all__ = [
    "install_cuda_shift_attn",
    "install_cuda_shift_gasd",
    "install_cuda_shift_metropolis",
    "install_cuda_shift_nectr",
]
