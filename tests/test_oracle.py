"""CPU tests: pin the oracle before trusting it.

Each check is chosen so that a plausible mistake in the C restatement (wrong
rounding mode, fused q*scale+zero, dropped epsilon, wrong bit order, wrong
min/max init) fails one of them:
  * the reference's own known answers (tests/golden/reference_kat.json);
  * an independent float32 + exact-rational implementation over exhaustive
    small groups;
  * the reference's torch mirror on tie-free seeded inputs;
  * invariants: round-trip == dequantize(quantize), |x - x_hat| <= scale/2;
  * get_stats closed form reproducing README.md:17-18.
"""

import itertools
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import codec
from oracle.kivi_cache import closed_form_stats
from tests.conftest import seeded_kv


# ----------------------------------------------------------------------------
# Known answers from the reference's tests.
# ----------------------------------------------------------------------------
def test_kat_packed_228(kat):
    k = kat["packed_228"]
    packed, scales, zeros = codec.quantize_groups(k["input"], k["group_size"])
    assert packed.tolist() == k["packed"]
    assert scales.tolist() == [k["scale"]]
    assert zeros.tolist() == [k["zero"]]
    out = codec.dequantize_groups(packed, scales, zeros, k["group_size"])
    assert out.tolist() == k["dequant"]


def test_kat_four_channels(kat):
    k = kat["packed_228_four_channels"]
    packed, scales, zeros = codec.quantize_groups(np.array(k["input"]), k["group_size"])
    assert packed.tolist() == k["packed"]
    assert scales.tolist() == k["scale"] and zeros.tolist() == k["zero"]


@pytest.mark.parametrize("name", ["constant_5", "constant_5_roundtrip"])
def test_kat_constant(kat, name):
    k = kat[name]
    x = np.full(k["shape"], k["value"], np.float32)
    packed, scales, zeros = codec.quantize_groups(x, k["group_size"])
    assert np.all(packed == 0)
    assert np.all(scales == np.float32(1e-10))          # (max-min)/3 + 1e-10
    assert np.all(zeros == np.float32(k["value"]))
    out = codec.dequantize_groups(packed, scales, zeros, k["group_size"])
    assert np.all(out == np.float32(k["dequant_value"]))
    assert np.all(codec.roundtrip_groups(x, k["group_size"]) == np.float32(k["dequant_value"]))


def test_kat_tie_rounding(kat):
    k = kat["tie_244"]
    packed, _, _ = codec.quantize_groups(k["input"], k["group_size"])
    assert packed.tolist() == k["packed_kernel"]
    # the mirror disagrees exactly here, and count_ties sees it
    mirror = codec.mirror_roundtrip(np.array(k["input"], np.float32), 4)
    mp, ms, mz = codec.quantize_groups(mirror.numpy(), 4)
    assert codec.count_ties(k["input"], 4) == 2
    codes_mirror = [int(round(float(v))) for v in (mirror.numpy() - 0.0)]
    assert codes_mirror == [0, 0, 2, 3]
    assert sum(c << (2 * i) for i, c in enumerate(codes_mirror)) == k["packed_mirror"][0]


# ----------------------------------------------------------------------------
# Independent implementation: numpy float32 for every IEEE step, exact
# rationals for round-half-away, Python's min/max over the set.
# ----------------------------------------------------------------------------
def _independent_group(vals):
    f = np.float32
    xs = [f(v) for v in vals]
    mn = min([f(1e30)] + xs)
    mx = max([f(-1e30)] + xs)
    scale = f(f(f(mx - mn) / f(3.0)) + f(1e-10))
    codes = []
    for x in xs:
        t = f(f(x - mn) / scale)
        q = int((Fraction(float(t)) + Fraction(1, 2)).__floor__())
        codes.append(min(max(q, 0), 3))
    packed = [sum(codes[4 * j + k] << (2 * k) for k in range(4)) for j in range(len(xs) // 4)]
    deq = [f(f(f(q) * scale) + mn) for q in codes]
    return packed, scale, mn, deq


def test_exhaustive_small_groups_match_independent_impl():
    values = [-3.0, -1.0, -0.5, 0.0, 0.25, 0.5, 1.0, 1.5, 2.75]
    groups = np.array(list(itertools.product(values, repeat=4)), np.float32)
    packed, scales, zeros = codec.quantize_groups(groups, 4)
    deq = codec.roundtrip_groups(groups, 4).reshape(-1, 4)
    for i, g in enumerate(groups):
        p, s, z, d = _independent_group(g)
        assert packed[i] == p[0], (g, packed[i], p)
        assert scales[i] == s and zeros[i] == z
        assert deq[i].tolist() == [float(v) for v in d]


def test_random_groups_match_independent_impl():
    rng = np.random.default_rng(7)
    for G in (4, 8, 12, 32):
        x = (rng.standard_normal((64, G)) * rng.choice([1e-3, 1.0, 50.0], (64, 1))).astype(np.float32)
        packed, scales, zeros = codec.quantize_groups(x, G)
        packed = packed.reshape(64, G // 4)
        for i in range(64):
            p, s, z, _ = _independent_group(x[i])
            assert packed[i].tolist() == p and scales[i] == s and zeros[i] == z


# ----------------------------------------------------------------------------
# Invariants and the mirror.
# ----------------------------------------------------------------------------
@pytest.mark.parametrize("G", [4, 8, 16, 32, 64, 128])
def test_roundtrip_equals_quantize_then_dequantize(G):
    x = seeded_kv((3, 5, G * 7), seed=G, kind="key")
    packed, scales, zeros = codec.quantize_groups(x.numpy(), G)
    pair = codec.dequantize_groups(packed, scales, zeros, G)
    fused = codec.roundtrip_groups(x.numpy(), G)
    assert np.array_equal(pair.view(np.uint32), fused.view(np.uint32))


@pytest.mark.parametrize("G,kind", [(32, "key"), (32, "value"), (128, "value"), (8, "key")])
def test_mirror_matches_on_tie_free_inputs(G, kind):
    x = seeded_kv((2, 3, 64, 128), seed=11 + G, kind=kind)
    assert codec.count_ties(x.numpy(), G) == 0
    mirror = codec.mirror_roundtrip(x, G).numpy().reshape(-1)
    ours = codec.roundtrip_groups(x.numpy(), G)
    assert np.array_equal(mirror.view(np.uint32), ours.view(np.uint32))


def test_error_bound_half_scale():
    x = seeded_kv((4, 8, 256), seed=3, kind="key").numpy().reshape(-1)
    G = 32
    packed, scales, zeros = codec.quantize_groups(x, G)
    out = codec.dequantize_groups(packed, scales, zeros, G)
    err = np.abs(out.astype(np.float64) - x).reshape(-1, G).max(axis=1)
    assert np.all(err <= scales.astype(np.float64) * 0.5 * (1 + 1e-5) + 1e-6)
    codes = codec.unpack_codes(packed, G)
    assert codes.max() <= 3


def test_nan_and_large_values():
    x = np.array([np.nan, 1.0, 2.0, 4.0,          # NaN ignored by min/max, coded 0
                  2e30, 3e30, 4e30, 5e30,          # above the 1e30 min init
                  -5e30, -4e30, -3e30, -2e30],     # below the -1e30 max init
                 np.float32)
    packed, scales, zeros = codec.quantize_groups(x, 4)
    assert zeros[0] == 1.0 and codec.unpack_codes(packed[:1], 4)[0] == 0
    assert zeros[1] == np.float32(1e30)             # reference init wins
    assert zeros[2] == np.float32(-5e30)
    assert np.float32(scales[2]) == np.float32(np.float32(np.float32(-1e30) - np.float32(-5e30)) / np.float32(3)) + np.float32(1e-10)


def test_signed_zero_ordering():
    x = np.array([0.0, -0.0, 1.0, 2.0], np.float32)
    _, _, zeros = codec.quantize_groups(x, 4)
    assert zeros[0] == 0 and np.signbit(zeros[0])


# ----------------------------------------------------------------------------
# get_stats closed form == README numbers.
# ----------------------------------------------------------------------------
def test_stats_closed_form_matches_readme(kat):
    k = kat["readme_stats"]
    s = closed_form_stats(k["B"], k["H"], k["D"], k["G"], k["R"],
                          k["prompt_tokens"] + k["fed_tokens"])
    assert s["kivi_bytes"] / 1024 == pytest.approx(k["kivi_kb"], abs=0.05)
    assert s["fp32_bytes"] / 1024 == pytest.approx(k["fp32_kb"], abs=0.05)
    assert s["compression"] == pytest.approx(k["compression"], abs=0.005)


def test_config1_expected_accounting():
    # Benchmark config 1: 12 layers, B=1, H=12, D=64, R=G=32, 200 tokens.
    s = closed_form_stats(1, 12, 64, 32, 32, 200)
    assert s["quantized_tokens"] == 192 and s["residual_tokens"] == 8
    assert s["kivi_bytes"] == 196608 and s["fp32_bytes"] == 1228800
    assert s["compression"] == pytest.approx(6.25)
