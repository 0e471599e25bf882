"""Writes reference_kat.json: the known answers the reference's own tests and
README state, transcribed as data (nothing here is computed by this build).

Sources (reference checkout):
  packed 228 / scale 1 / zero 1 / exact round trip for [1,2,3,4], G=4:
      tests/integration/test_kivi.py:160-196, test_quantize_simple.py:24-86
  constant 5.0 -> no NaN/Inf, reconstructs 5.0:
      tests/integration/test_kivi.py:256-278, test_roundtrip_kernels.py:79-87
  tie group [0, 0.5, 2.5, 3]: kernel rounding (sycl::round, half away from
      zero, src/csrc/kernels/internal/quant_tile.hpp:64) packs codes
      [0,1,3,3] = 244; the torch mirror (torch.round, half to even,
      tests/unit/test_manager_bookkeeping.py:65) gives [0,0,2,3] = 224
  README cache stats, GPT-2 (12 layers, 12 heads, D=64), G=32, R=64,
      32-token prompt + 199 fed tokens (examples/benchmark.py:74-96):
      378 KB KIVI vs 1386 KB FP32, 3.67x (README.md:17-18)
  reference attention gate: cosine > 0.85 at B=1, H=2, q=3, cache 32, D=64,
      G=32 (tests/integration/test_attention_fix.py:112), README value 0.898
      (README.md:386)
"""
import json
import os

KAT = {
    "packed_228": {
        "input": [1.0, 2.0, 3.0, 4.0], "group_size": 4,
        "packed": [228], "scale": 1.0, "zero": 1.0,
        "dequant": [1.0, 2.0, 3.0, 4.0],
        "source": "tests/integration/test_kivi.py:160-196",
    },
    "packed_228_four_channels": {
        "input": [[1.0, 2.0, 3.0, 4.0]] * 4, "group_size": 4,
        "packed": [228, 228, 228, 228], "scale": [1.0] * 4, "zero": [1.0] * 4,
        "source": "tests/integration/test_quantize_simple.py:24-86",
    },
    "constant_5": {
        "shape": [1, 1, 1, 4], "value": 5.0, "group_size": 4,
        "dequant_value": 5.0,
        "source": "tests/integration/test_kivi.py:256-278",
    },
    "constant_5_roundtrip": {
        "shape": [1, 1, 4, 32], "value": 5.0, "group_size": 32,
        "dequant_value": 5.0,
        "source": "tests/integration/test_roundtrip_kernels.py:79-87",
    },
    "tie_244": {
        "input": [0.0, 0.5, 2.5, 3.0], "group_size": 4,
        "packed_kernel": [244], "packed_mirror": [224],
        "source": "src/csrc/kernels/internal/quant_tile.hpp:64 vs tests/unit/test_manager_bookkeeping.py:65",
    },
    "readme_stats": {
        "B": 1, "H": 12, "D": 64, "G": 32, "R": 64, "layers": 12,
        "prompt_tokens": 32, "fed_tokens": 199,
        "kivi_kb": 378.0, "fp32_kb": 1386.0, "compression": 3.67,
        "source": "README.md:17-18, examples/benchmark.py:109-118",
    },
    "attention_cosine_gate": {
        "B": 1, "H": 2, "q_len": 3, "cache_len": 32, "D": 64, "G": 32,
        "min_cosine": 0.85, "readme_cosine": 0.898,
        "source": "tests/integration/test_attention_fix.py:112, README.md:386",
    },
}

if __name__ == "__main__":
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_kat.json")
    with open(out, "w") as f:
        json.dump(KAT, f, indent=1, sort_keys=True)
    print(out)
