"""CPU restatements of the LDS and register layouts of the matrix-core
attention steps (csrc/oc_kernels.h, csrc/oc_prefill.hip), checked against
the properties the kernels rely on (no GPU needed).

1. kperm (the transposed decode step): the K row order that makes the eight
   probabilities lane 16*kg + x holds for a 32-token block (A rows 4kg + i of
   the block's two 16-row halves) the tokens 8kg .. 8kg + 7 in order, the k
   index of the p.V instruction.
2. pf_vtok (the prefill's V stage): a permutation inside each 32-token block
   under which the transposing read of rows 8g .. 8g + 7 hands lane group g
   the tokens 4g + b and 16 + 4g + b, the ones whose scores the lane holds.
3. v_xor / vswz (the 16-bit and fp8 V tiles in LDS): every transposing read
   (16 rows of one column piece for 16-bit, 32 rows for fp8) uses no bank
   slot more than twice, where the unswizzled layout uses one slot 8 (d 64)
   or 16 (d 128) times; and the XOR keeps each chunk inside its row.  The
   prefill's vswz is the same map on 32-byte column pairs (v_xor / 2), over
   the same LDS rows of the same reads.
The restatements are checked to fail on planted slips.
"""

import pytest


def kperm(a):
    return (a & ~31) + 8 * ((a >> 2) & 3) + 4 * ((a >> 4) & 1) + (a & 3)


def pf_vtok(r):
    return (r & ~31) + 16 * ((r >> 2) & 1) + 4 * ((r >> 3) & 3) + (r & 3)


def v_xor(r, d, fp8):
    """16-byte chunk XOR of LDS row r (the decode's V tile)"""
    if fp8:
        return (r >> 1) & 7 if d == 128 else (r >> 2) & 3
    return 2 * ((r & 3) + 4 * ((r >> 3) & 1)) if d == 128 else 2 * (((r & 3) >> 1) + 2 * ((r >> 3) & 1))


def _lane_block_tokens(perm, j, kg):
    """tokens behind the eight probabilities of lane group kg for block j
    (registers c[2j][0..3], c[2j+1][0..3]: A rows 32j + 4kg + i and
    32j + 16 + 4kg + i)"""
    return [perm(32 * j + 4 * kg + i) for i in range(4)] + [perm(32 * j + 16 + 4 * kg + i) for i in range(4)]


@pytest.mark.parametrize("perm,ok", [(kperm, True), (lambda a: a, False),
                                     (lambda a: (a & ~31) + 8 * ((a >> 2) & 3) + 4 * ((a >> 4) & 1) + (3 - (a & 3)),
                                      False)])
def test_kperm_hands_each_lane_its_tokens_in_order(perm, ok):
    good = sorted(perm(a) for a in range(64)) == list(range(64)) and all(
        _lane_block_tokens(perm, j, kg) == list(range(32 * j + 8 * kg, 32 * j + 8 * kg + 8))
        for j in range(2) for kg in range(4))
    assert good == ok


def test_pf_vtok_permutes_blocks_and_matches_the_lanes():
    for blk in range(4):
        rows = range(32 * blk, 32 * blk + 32)
        assert sorted(pf_vtok(r) for r in rows) == list(rows)
    for g in range(4):
        got = sorted(pf_vtok(8 * g + e) % 32 for e in range(8))
        assert got == sorted([4 * g + b for b in range(4)] + [16 + 4 * g + b for b in range(4)])
    # a slip (the two halves swapped in the row order) breaks the match
    slip = lambda r: (r & ~31) + 16 * ((r >> 3) & 1) + 4 * ((r >> 2) & 3) + (r & 3)  # noqa: E731
    assert sorted(slip(8 * 1 + e) % 32 for e in range(8)) != sorted(
        [4 + b for b in range(4)] + [20 + b for b in range(4)])


def _max_slot_use(d, fp8, xor):
    """largest number of lanes' 16-byte pieces on one 16-byte bank slot (of a
    256-byte bank line) over the transposing reads of a 64-token V tile"""
    es = 1 if fp8 else 2
    row_bytes = d * es
    worst = 0
    for tb2 in range(2):
        for nc in range(d // 16):
            for h in range(1 if fp8 else 2):  # 16-bit: two instructions (rows +0, +4)
                if fp8:
                    # ds_read_b64_tr_b8: lanes 2m, 2m + 1 of group kg read 16 bytes of row 32 tb2 + 8 kg + m
                    rows = [32 * tb2 + 8 * kg + m for kg in range(4) for m in range(8)]
                    offs = [16 * (nc ^ xor(r)) for r in rows]
                    width = 16
                else:
                    # ds_read_b64_tr_b16: lanes 4m .. 4m + 3 of group kg read a 32-byte column pair of row
                    # 32 tb2 + 8 kg + 4 h + m
                    rows = [32 * tb2 + 8 * kg + 4 * h + m for kg in range(4) for m in range(4)]
                    offs = [32 * (nc ^ (xor(r) >> 1)) for r in rows]
                    width = 32
                use = {}
                for r, o in zip(rows, offs):
                    for piece in range(0, width, 16):
                        slot = ((r * row_bytes + o + piece) % 256) // 16
                        use[slot] = use.get(slot, 0) + 1
                worst = max(worst, max(use.values()))
    return worst


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("fp8", [False, True])
def test_v_xor_spreads_the_transposing_reads(d, fp8):
    xor = lambda r: v_xor(r, d, fp8)  # noqa: E731
    chunks = d * (1 if fp8 else 2) // 16
    assert all(0 <= (c ^ xor(r)) < chunks for r in range(64) for c in range(chunks))
    # each read is 16 rows x 32 bytes (16-bit) or 32 rows x 16 bytes (fp8) =
    # 512 bytes, at least two passes over a 256-byte line; no slot more than twice
    assert _max_slot_use(d, fp8, xor) <= 2
    assert _max_slot_use(d, fp8, lambda r: 0) >= 8  # unswizzled: one slot many times over
