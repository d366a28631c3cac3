"""turbo_roformer_amd: the BS-RoFormer transformer stack of LoggeL/turbo-roformer on MI355X (gfx950).

The stack (12 x time attention + FF, freq attention + FF) and the mask head after it (final norm and
per-band MLPs) run as hand-written HIP kernels behind the C ABI in include/trf_hip.h (``libtrf_hip.so``);
STFT, band split, iSTFT and overlap-add stay on the PyTorch host path.
"""

from ._hip import HipUnavailable, support

__all__ = ["HipUnavailable", "support", "__version__"]
__version__ = "0.1.0"
