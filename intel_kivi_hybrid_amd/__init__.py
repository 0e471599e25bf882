"""intel_kivi_hybrid_amd -- KIVI 2-bit KV cache hot path for AMD MI355X (gfx950).

Drop-in for the ``kivi_sycl`` API surface (src/kivi_sycl/__init__.py:24-28 in
the reference): ``KiviCache``, ``generate`` and the compiled-op module ``_C``.
All device work runs in hand-written HIP kernels in ``libkivi_hip.so``,
reached through its C ABI (include/kivi_hip.h); importing the package fails
with ImportError when that library is missing.
"""

from ._version import __version__
from .cache.manager import KiviCache
from .generation.generate import generate

__all__ = ["KiviCache", "generate", "__version__"]
