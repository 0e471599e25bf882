"""Test infrastructure only: CPU oracle for the KIVI KV-cache hot path.

Nothing in the product package (``intel_kivi_hybrid_amd``) imports this
package.  Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg use it, as the checker or as the CPU baseline.

* ``oracle.codec``     -- ctypes wrapper over ``libkivi_oracle.so`` (the C
  restatement of the reference codec) and the torch mirror the reference's own
  unit tests use (tests/unit/test_manager_bookkeeping.py:54-66).
* ``oracle.attention`` -- float64 decode attention over dequantised history
  plus fp32 residual (tests/integration/test_attention_fix.py:40-43,91-93 and
  HF ``repeat_kv`` for GQA).
* ``oracle.kivi_cache`` -- restatement of ``KiviCache``
  (src/kivi_sycl/cache/manager.py:14-423) on CPU, driven by the C codec.
"""
