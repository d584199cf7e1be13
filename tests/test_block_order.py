"""CPU model of the attention kernel's block order (pyasc_amd/csrc/flash_attn_kernels.h:
fa_fwd_body; the head-group size: flash_attn.hip, geometry): for many shapes,
every (batch*head, query block) pair runs exactly once, on the XCD that holds its
head, and causal blocks of one head start heaviest first.  The GPU tests check the
outputs of a few of these shapes; this covers the mapping over many more."""
import itertools

import pytest


def block_coords(heads_total, n_qblocks, head_group, causal, bid):
    # restatement of the kernel's mapping (workgroup bid runs on XCD bid % 8)
    if heads_total % 8 == 0:
        slot = bid >> 3
        per_group = head_group * n_qblocks
        grp = slot // per_group
        r = slot - grp * per_group
        g0 = grp * head_group
        heads_left = (heads_total >> 3) - g0
        assert heads_left >= 1
        gsz = min(heads_left, head_group)
        bh = (bid & 7) + 8 * (g0 + r % gsz)
        qb = r // gsz
    else:
        bh = bid % heads_total
        qb = bid // heads_total
    if causal:
        qb = n_qblocks - 1 - qb
    return bh, qb


def head_group(heads_total, n_qblocks, causal, cus, waves):
    # the launcher's choice
    if not causal:
        return 1
    slots = cus // 8 * (8 // waves)
    g = 2 * ((slots + n_qblocks - 1) // n_qblocks)
    heads_xcd = heads_total // 8
    return max(1, heads_xcd if (g > heads_xcd and heads_xcd > 0) else g)


SHAPES = [(ht, nq) for ht in (1, 3, 8, 16, 24, 40, 56, 128, 136) for nq in (1, 2, 7, 12, 16, 23, 32, 64)]


@pytest.mark.parametrize("heads_total,n_qblocks", SHAPES)
@pytest.mark.parametrize("causal", [False, True])
def test_every_block_once_on_its_xcd(heads_total, n_qblocks, causal):
    for cus, waves in ((256, 8), (256, 4), (304, 8), (80, 4)):
        g = head_group(heads_total, n_qblocks, causal, cus, waves)
        seen = {}
        for bid in range(heads_total * n_qblocks):
            bh, qb = block_coords(heads_total, n_qblocks, g, causal, bid)
            assert 0 <= bh < heads_total and 0 <= qb < n_qblocks
            assert (bh, qb) not in seen, (bh, qb, bid, seen.get((bh, qb)))
            seen[(bh, qb)] = bid
            if heads_total % 8 == 0:
                assert bh % 8 == bid % 8  # the head's K/V stay in one XCD's L2
        assert len(seen) == heads_total * n_qblocks


@pytest.mark.parametrize("heads_total,n_qblocks", [s for s in SHAPES if s[0] % 8 == 0])
def test_causal_heavy_first_within_each_head(heads_total, n_qblocks):
    g = head_group(heads_total, n_qblocks, True, 256, 8)
    last = {}
    for bid in range(heads_total * n_qblocks):
        bh, qb = block_coords(heads_total, n_qblocks, g, True, bid)
        if bh in last:
            assert qb == last[bh] - 1  # each head's blocks start in order of decreasing work
        last[bh] = qb


def test_bench_shape_group_and_order():
    # B4 H32 S4096, 8-wave blocks of 256 queries: 16 blocks per head, 32 slots per XCD
    g = head_group(128, 16, True, 256, 8)
    assert g == 4
    first = [block_coords(128, 16, g, True, bid) for bid in range(0, 8 * 8, 8)]  # XCD 0's first 8
    assert first == [(0, 15), (8, 15), (16, 15), (24, 15), (0, 14), (8, 14), (16, 14), (24, 14)]
