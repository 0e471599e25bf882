"""CPU tests of the decode-attention launch plan, through the C ABI's
workspace-size entry points (host logic only; no GPU work).

A plan with S > 1 splits needs B * Hkv * rows * S * (D + 2) fp32 of split
partials (rows: query rows per kv head of one launch, 1, 2, 4 or 8); an
unsplit plan needs none.  The split count follows the plan's rule, then
at least 2 chunks per wave.  At head_dim 128: the larger of (a) the most
splits whose workgroups fit 512 at once with >= 16 chunks per wave and (b)
enough splits for 256 workgroups; at other head dims ~2048 chunk waves (4
waves per workgroup).  Small batches split deeply while the benchmark
configs keep their plans.
"""

from intel_kivi_hybrid_amd import _native


def _decode_ws(B, Hq, Hkv, D, G, Gv, n_chunks, res_len, splits=0):
    return _native.load().kivi_packed_decode_attention_workspace_size(
        B, Hq, Hkv, D, G, Gv, n_chunks, res_len, splits)


def _splits(ws, B, Hkv, rows, D):
    per = B * Hkv * rows * (D + 2) * 4
    assert ws % per == 0
    return ws // per


def test_benchmark_configs_keep_their_plans():
    assert _decode_ws(64, 32, 8, 128, 32, 32, 252, 128) == 0          # config 4: one split
    assert _decode_ws(16, 32, 32, 128, 32, 32, 128, 128) == 0         # config 3: one split
    ws = _decode_ws(4, 32, 8, 128, 32, 128, 4096, 128)                 # config 5
    assert _splits(ws, 4, 8, 4, 128) == 16


def test_small_batches_split_to_two_chunks_per_wave():
    # one sequence, 8 kv heads: 8 (b, kv-head) pairs; (b) wants 32 splits
    assert _splits(_decode_ws(1, 32, 8, 128, 32, 32, 252, 128), 1, 8, 4, 128) == 32   # 8K
    assert _splits(_decode_ws(1, 32, 8, 128, 32, 32, 63, 128), 1, 8, 4, 128) == 8     # 2K: 2 per wave
    # an explicit split count is kept
    assert _splits(_decode_ws(1, 32, 8, 128, 32, 32, 252, 128, 4), 1, 8, 4, 128) == 4


def test_mid_batches_keep_sixteen_chunks_per_wave_at_head_dim_128():
    # 252 chunks (8K): 4 splits leave 16 chunks per wave
    for B, S in ((2, 16), (4, 8), (8, 4), (12, 4), (16, 4), (24, 2), (32, 2), (48, 1)):
        ws = _decode_ws(B, 32, 8, 128, 32, 32, 252, 128)
        assert (_splits(ws, B, 8, 4, 128) if ws else 1) == S, B
    # 1020 chunks (32K): (a) allows 8 splits at B=8 and 16 at B=2 and 4
    for B, S in ((2, 16), (4, 16), (8, 8), (16, 4)):
        assert _splits(_decode_ws(B, 32, 8, 128, 32, 32, 1020, 128), B, 8, 4, 128) == S, B
    # 60 chunks (2K): no split keeps 16 per wave, so (b): 256 workgroups
    assert _splits(_decode_ws(8, 32, 8, 128, 32, 32, 60, 128), 8, 8, 4, 128) == 4
    assert _decode_ws(32, 32, 8, 128, 32, 32, 60, 128) == 0


def test_other_head_dims_aim_at_2048_waves():
    # head_dim 64, 12/12 heads: 16 sequences -> 192 pairs, 3 splits; 4 -> 11
    assert _splits(_decode_ws(16, 12, 12, 64, 32, 32, 252, 64), 16, 12, 1, 64) == 3
    assert _splits(_decode_ws(4, 12, 12, 64, 32, 32, 252, 64), 4, 12, 1, 64) == 11


def test_window_only_context_is_unsplit():
    # no chunk yet: one split whichever kernel runs, so no workspace
    assert _decode_ws(1, 32, 8, 128, 32, 32, 0, 100) == 0
    assert _decode_ws(1, 32, 8, 128, 32, 32, 0, 100, 8) == 0
    assert _decode_ws(16, 32, 8, 64, 32, 32, 0, 127) == 0


def test_rows_follow_head_groups_and_query_tokens():
    # 12 query heads per kv head: launches of 8 heads (8 rows)
    assert _splits(_decode_ws(1, 24, 2, 128, 32, 32, 252, 128), 1, 2, 8, 128) == 32
    # ratio 3 pads to 4 rows
    ws = _decode_ws(1, 24, 8, 128, 32, 32, 252, 128)
    assert _splits(ws, 1, 8, 4, 128) == 32
    # three query tokens at 4 heads per kv head: 2 tokens per launch, 8 rows
    ws = _native.load().kivi_packed_attention_workspace_size(1, 3, 8, 2, 128, 32, 32, 252, 128, 0)
    assert _splits(ws, 1, 2, 8, 128) == 32
