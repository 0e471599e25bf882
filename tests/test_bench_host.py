"""bench.py's byte accounting and its one-GPU contract, on the host.

The algorithmic byte counts behind every GB/s figure and `roofline.achieved`
are pinned against the closed forms stated independently for each BASELINE
configuration (per (b, kv head): codes D*T/4 per tensor, key scales and
zeros 8*D*T/Gk, value scales and zeros 8*T*D/Gv, the fp32 window 8*Tr*D, q
and o 8*(Hq/Hkv)*D)."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_attention_bytes_match_the_config_closed_forms():
    # config 3: 656,384 B per (b, head) x 512 pairs
    assert bench.attn_bytes(16, 32, 32, 128, 4096, 128, 32, 32) == 656_384 * 512 == 336_068_608
    # config 4 (Tq = 8064, Tr = 128): 1,167,360 B x 512 pairs
    assert bench.attn_bytes(64, 32, 8, 128, 8064, 128, 32, 32) == 1_167_360 * 512 == 597_688_320
    # the same with a bf16 residual ring: the window's K and V at 2 bytes
    assert bench.attn_bytes(64, 32, 8, 128, 8064, 128, 32, 32, ring_bytes=2) == \
        597_688_320 - 512 * 2 * 128 * 128 * 2 == 564_133_888
    # config 5 (Gv = 128): 13,766,656 B x 32 pairs
    assert bench.attn_bytes(4, 32, 8, 128, 131072, 128, 32, 128) == 13_766_656 * 32


def test_codec_bytes_match_config2():
    n = 8 * 32 * 128 * 4096
    assert bench.quant_bytes(n, 32) == 603_979_776            # 4N + N/4 + 8N/G
    assert 2 * bench.quant_bytes(n, 32) == 1_207_959_552      # K + V
    assert bench.dequant_bytes(n, 32) == bench.quant_bytes(n, 32)
    assert bench.roundtrip_bytes(n) == 2 * 4 * n


def test_decode_flush_bytes():
    # one chunk per (b, kv head): K and V read (2 x G x D fp32), codes
    # written (2 x G x D / 4), key scales and zeros (8 D), value scales and
    # zeros (8 G D / Gv)
    per = 2 * 32 * 128 * 4 + 2 * 32 * 128 // 4 + 8 * 128 + 8 * 32 * 128 // 32
    assert bench.flush_bytes(64, 8, 128, 32, 32) == per * 512 == 18_874_368


def test_store_tokens_accepts_only_states_the_flush_rule_leaves():
    assert bench.store_tokens(8064, 111, 32, 128) == 8175
    assert bench.store_tokens(4096, 127, 32, 128) == 4223
    with pytest.raises(ValueError):
        bench.store_tokens(8064, 95, 32, 128)      # below R - G
    with pytest.raises(ValueError):
        bench.store_tokens(8064, 128, 32, 128)     # a full window would have flushed
    with pytest.raises(ValueError):
        bench.store_tokens(8063, 111, 32, 128)     # not whole chunks


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
