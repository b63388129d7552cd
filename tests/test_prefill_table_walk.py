"""The block-table entries the MFMA prefill kernels read with 16-token blocks, walked on the CPU.

prefill_kernel (csrc/qp_prefill.hip) and prefill_wide_kernel (csrc/qp_prefill_wide.hip) read the table pair of tile
t + 5 one iteration ahead of its copies, through a pointer that steps two entries per tile; the tile kernel's
six-phase unrolled loop of int4 keys reads the 12 entries of tiles it + 5 .. it + 10 at once, in its first iteration,
and its rolled steady loop of int8 keys runs in pairs whose first iteration reads the 4 entries of tiles it + 5, it + 6.
Their steady iterations (that unrolled loop, the tile kernel's rolled steady loop of int8 keys, the wide kernel's
steady loop) take a pair's second entry without checking the split's end, which is only valid when that tile is
followed by another one. This walk restates each kernel's loop structure (prologue and loops, with the `kPfSteadyLead` bound read
from the source) and checks, for every context length mod 32, row blocks of (token, head) pairs at several GQA widths
and the key-split geometry the kernels use, that

* every entry read lies inside the sequence's own row (index < ceil(kend / 16)), so a table whose row holds exactly
  ceil(n / 16) entries is never read past its end;
* tile t reads the entries of its own blocks: 2t + kb / 16, and the next one only when its second 16-key run starts
  before the split's end.

A walk with the bound one tile shorter (the kernel's earlier steady condition) reads one entry past the row, which
the test also checks, so the walk can see the mistake it guards against."""
import re
from pathlib import Path

import pytest

CSRC = Path(__file__).resolve().parents[1] / "vllm-quantpack_amd" / "csrc"
TILE = 32        # keys per tile (kPfKeys)
DECODE_TILE = 32  # split granularity (QP_DECODE_TILE)


def steady_lead() -> int:
    m = re.search(r"constexpr int kPfSteadyLead = (\d+);", (CSRC / "qp_prefill.h").read_text())
    assert m, "kPfSteadyLead not found in qp_prefill.h"
    # both kernels bound their steady loops by it (the tile kernel's unrolled loop by it + 5 + kPfSteadyLead)
    src = (CSRC / "qp_prefill.hip").read_text()
    assert "it + 5 + kPfSteadyLead <= ntiles" in src
    # the unrolled loop's group read, as walked below
    assert "for (int k = 0; k < 12; ++k) tb[k] = tnext[k];" in src and "tnext += 12;" in src
    assert "for (int k = 0; k < 4; ++k) tb[k] = tnext[k];" in src and "tnext += 4;" in src
    assert "it + 1 < nplain && it + 1 + kPfSteadyLead <= ntiles; it += 2" in src
    assert "it + kPfSteadyLead <= ntiles" in (CSRC / "qp_prefill_wide.hip").read_text()
    return int(m.group(1))


def walk(n, qlen, t_first, t_last, split, splits, int4, lead, wide=False):
    """Table indices read by one workgroup (a row block whose (token, head) rows span local tokens t_first..t_last of
    a qlen-token chunk whose last token sees n keys; key split `split` of `splits`), as the kernel reads them (wide:
    prefill_wide_kernel's loops, whose iterations run up to the split's second-to-last tile). Returns (reads,
    expected) lists of (tile, index)."""
    first_pos = n - qlen + t_first
    kend = max(0, min(n, n - qlen + t_last + 1))
    seg = -(-n // (splits * DECODE_TILE)) * DECODE_TILE
    kb = split * seg
    ke = min(kend, kb + seg)
    if splits > 1 and kb >= n:
        return [], []
    ntiles = -(-(ke - kb) // TILE) if ke > kb else 0
    vis_all = first_pos + 1
    nplain = min(ntiles, max(0, (vis_all - kb) // TILE))
    tile_key = lambda t: kb + TILE * t
    reads, state = [], {"tnext": (kb >> 4) + 8, "next_tile": 4}

    def table_ahead(t, steady):
        assert t == state["next_tile"], "the table pointer steps one tile at a time"
        state["next_tile"] += 1
        tn = state["tnext"]
        off1 = 1 if steady else min(1, (ke - 1 - tile_key(t)) >> 4)
        reads.append((t, tn))
        reads.append((t, tn + off1))
        state["tnext"] += 2

    def iteration(it, steady):
        if steady or it + 4 < ntiles:
            if steady or it + 5 < ntiles:
                table_ahead(it + 5, steady)

    if ntiles == 0:
        return [], []
    if ntiles > 4:
        table_ahead(4, False)
    it = 0
    if wide:
        while it + 1 < nplain and it + lead <= ntiles:
            iteration(it, True)
            it += 1
        while it + 1 < ntiles:
            iteration(it, False)
            it += 1
    else:
        if int4:
            while it + 6 <= nplain and it + 5 + lead <= ntiles:
                # iteration it reads tnext .. tnext + 11 in one load: the pairs of tiles it + 5 .. it + 10
                assert state["next_tile"] == it + 5
                tn = state["tnext"]
                reads.extend((it + 5 + k // 2, tn + k) for k in range(12))
                state["tnext"] += 12
                state["next_tile"] += 6
                it += 6
        else:
            while it + 1 < nplain and it + 1 + lead <= ntiles:
                # the pair's first iteration reads tnext .. tnext + 3: the pairs of tiles it + 5, it + 6
                assert state["next_tile"] == it + 5
                tn = state["tnext"]
                reads.extend((it + 5 + k // 2, tn + k) for k in range(4))
                state["tnext"] += 4
                state["next_tile"] += 2
                it += 2
            while it < nplain and it + lead <= ntiles:
                iteration(it, True)
                it += 1
        while it < ntiles:
            iteration(it, False)
            it += 1
    expected = []
    for t in range(4, ntiles):
        b0 = tile_key(t) >> 4
        expected += [(t, b0), (t, b0 + 1 if tile_key(t) + 16 < ke else b0)]
    return reads, expected


def shapes():
    """Chunks of 20 and 64 tokens over contexts of every residue mod 32 around the loops' bounds, one to three key
    splits."""
    for base in (160, 320, 480, 992):
        for r in range(32):
            n = base + r
            for qlen in (20, 64):
                if qlen <= n:
                    for splits in (1, 2, 3):
                        yield n, qlen, splits


def blocks(qlen, G, rows):
    """(t_first, t_last) of each row block of `rows` (token, head) rows over a qlen-token chunk with G heads."""
    for r0 in range(0, qlen * G, rows):
        yield r0 // G, (min(qlen * G, r0 + rows) - 1) // G


# the tile kernel's 192-row blocks at GQA 1, 6 and 8, the wide kernel's 128-row blocks at GQA 16
KERNELS = [dict(int4=True, G=6, rows=192), dict(int4=True, G=8, rows=192), dict(int4=True, G=1, rows=192),
           dict(int4=False, G=6, rows=192), dict(int4=True, wide=True, G=16, rows=128)]
IDS = ["tiles-int4-g6", "tiles-int4-g8", "tiles-int4-g1", "tiles-int8-g6", "wide-g16"]


def out_of_row(lead, int4, G, rows, wide=False):
    bad = []
    for n, qlen, splits in shapes():
        for t_first, t_last in blocks(qlen, G, rows):
            for split in range(splits):
                reads, _ = walk(n, qlen, t_first, t_last, split, splits, int4, lead, wide)
                row = -(-n // 16)
                bad += [(n, qlen, splits, t_first, split, t, i) for t, i in reads if i >= row]
    return bad


@pytest.mark.parametrize("kernel", KERNELS, ids=IDS)
def test_every_table_read_stays_in_the_row(kernel):
    assert out_of_row(steady_lead(), **kernel) == []


@pytest.mark.parametrize("kernel", KERNELS, ids=IDS)
def test_each_tile_reads_its_own_blocks(kernel):
    lead = steady_lead()
    for n, qlen, splits in shapes():
        for t_first, t_last in blocks(qlen, kernel["G"], kernel["rows"]):
            for split in range(splits):
                reads, expected = walk(n, qlen, t_first, t_last, split, splits, kernel["int4"], lead,
                                       kernel.get("wide", False))
                assert reads == expected, (n, qlen, splits, t_first, split)


@pytest.mark.parametrize("kernel", KERNELS, ids=IDS)
def test_a_bound_one_tile_shorter_reads_past_the_row(kernel):
    """The walk catches the mistake it guards against: steady iterations up to the split's last tile read the entry
    after a last tile of 1..16 keys."""
    bad = out_of_row(steady_lead() - 1, **kernel)
    assert bad, "the shorter bound should read past the row"
    assert all((n % 32) in range(1, 17) for n, *_ in bad)
