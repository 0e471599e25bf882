"""Single import seam for the compiled HIP library (src/kivi_sycl/extension/loader.py:8-19
in the reference).

Every module that launches device work imports ``kivi_native`` from here, so
there is one place that explains a missing build.  There is no fallback: the
package cannot run without ``libkivi_hip.so``.
"""

try:
    from .. import _C as kivi_native
except ImportError as exc:
    raise ImportError(
        "intel_kivi_hybrid_amd._C (the compiled HIP library libkivi_hip.so) was not "
        "found or failed to load.\nBuild it in-place with:\n\n"
        "  python -m intel_kivi_hybrid_amd.build\n"
    ) from exc

__all__ = ["kivi_native"]
