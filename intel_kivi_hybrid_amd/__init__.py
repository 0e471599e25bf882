"""intel_kivi_hybrid_amd -- KIVI 2-bit KV cache hot path for AMD MI355X (gfx950).

Drop-in for the ``kivi_sycl`` API surface (src/kivi_sycl/__init__.py:24-28 in
the reference): ``KiviCache``, ``generate`` and the compiled-op module ``_C``,
plus ``KiviPackedCache`` / ``generate_packed``: the cache as a
``transformers.Cache`` whose decode attention reads the 2-bit store directly.
All device work runs in hand-written HIP kernels in ``libkivi_hip.so``,
reached through its C ABI (include/kivi_hip.h); using ``KiviCache``,
``generate`` or ``_C`` fails with ImportError when that library is missing.

The public names resolve on first access, so that the build module
(``python -m intel_kivi_hybrid_amd.build``) imports without the library.
"""

from ._version import __version__

__all__ = ["KiviCache", "KiviPackedCache", "generate", "generate_packed", "packed_attention",
           "__version__"]


def __getattr__(name):
    if name == "KiviCache":
        from .cache.manager import KiviCache
        return KiviCache
    if name in ("KiviPackedCache", "packed_attention"):
        from .cache import packed_cache
        return getattr(packed_cache, name)
    if name in ("generate", "generate_packed"):
        from . import generation
        return getattr(generation, name)
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
