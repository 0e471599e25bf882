"""Host checks of the packed-store format helpers: the code-order
encoder/decoder of intel_kivi_hybrid_amd.store against the matrix-core layout
as include/kivi_hip.h documents it, and the validation of saved
KiviPackedCache files (no device work)."""

import pytest
import torch

from intel_kivi_hybrid_amd.store import decode_codes, encode_codes

SHAPES = [(32, 64), (32, 128), (64, 64), (64, 128), (32, 256)]


def _layout_bit(G, D, key, t, d):
    """(lane, dword, bit) of element (t, d) per the header's description:
    key tile ks*(G/16)+nb: lane l element j = token 16nb + l%16, channel
    32ks + 8(l/16) + j; value tile kt*(D/16)+nb: lane l element j = token
    32kt + 8(l/16) + j, channel 16nb + l%16; tiles 2w and 2w+1 share dword
    w, element j of tile 2w+m at bit 8m + 2(j/2) + 16(j%2)."""
    if key:
        nb, lm = divmod(t, 16)
        ks, rest = divmod(d, 32)
        lq, j = divmod(rest, 8)
        tile = ks * (G // 16) + nb
    else:
        nb, lm = divmod(d, 16)
        kt, rest = divmod(t, 32)
        lq, j = divmod(rest, 8)
        tile = kt * (D // 16) + nb
    lane = lm + 16 * lq
    w, m = divmod(tile, 2)
    return lane, w, 8 * m + 2 * (j // 2) + 16 * (j % 2)


@pytest.mark.parametrize("G,D", SHAPES)
@pytest.mark.parametrize("key", [True, False])
def test_matrix_core_order_matches_header(G, D, key):
    g = torch.Generator().manual_seed(G + D + key)
    np_ = G * D // 1024
    for _ in range(24):
        t = int(torch.randint(0, G, (1,), generator=g))
        d = int(torch.randint(0, D, (1,), generator=g))
        c = torch.zeros(G, D, dtype=torch.uint8)
        c[t, d] = 3
        raw = encode_codes(c, G, D, 1, key)
        words = raw.view(torch.int32).reshape(64, np_).to(torch.int64) & 0xFFFFFFFF
        lane, w, bit = _layout_bit(G, D, key, t, d)
        expect = torch.zeros(64, np_, dtype=torch.int64)
        expect[lane, w] = 3 << bit
        assert torch.equal(words, expect), (t, d)


@pytest.mark.parametrize("layout,G,D", [(0, 4, 8), (0, 32, 128), (0, 16, 64)] +
                         [(1, G, D) for G, D in SHAPES])
@pytest.mark.parametrize("key", [True, False])
def test_encode_decode_round_trip(layout, G, D, key):
    g = torch.Generator().manual_seed(layout * 1000 + G + D)
    c = torch.randint(0, 4, (2, 3, 4, G, D), generator=g, dtype=torch.uint8)
    raw = encode_codes(c, G, D, layout, key)
    assert raw.dtype == torch.uint8 and raw.shape == (2, 3, 4, G * D // 4)
    assert torch.equal(decode_codes(raw, G, D, layout, key), c)


def test_plain_order_is_the_reference_byte_order():
    """Plain keys: [G][D/4], channel 4i+k at bits 2k of byte (t, i); plain
    values: [D][G/4], token 4j+k at bits 2k of byte (d, j)."""
    G, D = 4, 8
    c = torch.zeros(G, D, dtype=torch.uint8)
    c[1, 6] = 2                          # token 1, channel 6
    k = encode_codes(c, G, D, 0, True)   # byte 1*2 + 1, bits 4-5
    assert k.tolist() == [0, 0, 0, 2 << 4, 0, 0, 0, 0]
    v = encode_codes(c, G, D, 0, False)  # byte (d=6, j=0), bits 2-3
    assert v.tolist() == [0, 0, 0, 0, 0, 0, 2 << 2, 0]


def _write(path, meta, tensors=None):
    from safetensors.torch import save_file
    save_file(tensors or {"layers.0.k_scale": torch.zeros(1, 1, 8, 0)}, str(path), metadata=meta)


GOOD = {"format": "kivi-packed-kv", "version": "1", "num_layers": "1", "head_dim": "8",
        "num_kv_heads": "1", "group_size": "4", "value_group_size": "4",
        "residual_length": "8"}


@pytest.mark.parametrize("change,msg", [
    ({"format": "something-else"}, "not a KiviPackedCache file"),
    ({"version": "99"}, "format version"),
    ({"group_size": None}, "incomplete cache metadata"),
    ({"head_dim": "eight"}, "incomplete cache metadata"),
])
def test_load_rejects_bad_files(tmp_path, change, msg):
    from intel_kivi_hybrid_amd.cache.packed_cache import KiviPackedCache
    meta = {k: v for k, v in {**GOOD, **change}.items() if v is not None}
    p = tmp_path / "c.safetensors"
    _write(p, meta)
    with pytest.raises(ValueError, match=msg):
        KiviPackedCache.load(str(p), device="cuda")
