"""CPU tests of the decode-attention launch plan, through the C ABI's
workspace-size entry points (host logic only; no GPU work).

A plan with S > 1 splits needs B * Hkv * rows * S * (D + 2) fp32 of split
partials (rows: query rows per kv head of one launch, 1, 2, 4 or 8); an
unsplit plan needs none.  The split count follows the plan's rule: aim at
~2048 chunk waves (4 waves per workgroup) with at least 2 chunks per wave,
so small batches split deeply while the benchmark configs keep their plans.
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
    # one sequence, 8 kv heads: 8 (b, kv-head) pairs
    assert _splits(_decode_ws(1, 32, 8, 128, 32, 32, 252, 128), 1, 8, 4, 128) == 32   # 8K
    assert _splits(_decode_ws(1, 32, 8, 128, 32, 32, 63, 128), 1, 8, 4, 128) == 8     # 2K
    # 8 sequences: 64 pairs, 8 splits reach 2048 waves
    assert _splits(_decode_ws(8, 32, 8, 128, 32, 32, 252, 128), 8, 8, 4, 128) == 8
    # an explicit split count is kept
    assert _splits(_decode_ws(1, 32, 8, 128, 32, 32, 252, 128, 4), 1, 8, 4, 128) == 4


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
