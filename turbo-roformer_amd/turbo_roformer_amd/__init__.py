"""turbo_roformer_amd: the BS-RoFormer transformer stack of LoggeL/turbo-roformer on MI355X (gfx950).

The stack (12 x time attention + FF, freq attention + FF), the band split before it, the mask head after
it (final norm and per-band MLPs) and the song's Hamming overlap-add run as hand-written HIP kernels behind
the C ABI in include/trf_hip.h (``libtrf_hip.so``); the STFT and iSTFT run through PyTorch on the GPU.
"""

from ._hip import HipUnavailable, support

__all__ = ["HipUnavailable", "support", "__version__"]
__version__ = "0.1.0"
