"""CPU model check of the collect scans' stage sync (flat_collect_kernel, px_collect.hip, and
the collect mode of flat_scan_kernel, px_flat.hip, which reads a stage's first A operands at
the start of the stage instead of after the wait before it: the same order).

The kernels have no barrier per stage. Each wave publishes in LDS the last stage it has
committed to a stage buffer (C). Stage s of a wave with queries:

    MFMAs over buffer s % 3 (its first A operands were read at the end of stage s - 1), and
    the keys of tile s - 1 from norm slot (s - 1) % 4;
    wait until every wave's C >= s + 1;
    read stage s + 1's first A operands from buffer (s + 1) % 3;
    write its part of stage s + 2 to buffer (s + 2) % 3 (wave 0: the norms, to slot
    (s + 2) % 4); C = s + 2.

A wave whose queries are all padding only stages rows: wait until every C >= s + 1; write
its part of stage s + 2; C = s + 2. After the last stage a wave with queries reads norm slot
(nstages - 1) % 4. The prologue writes stages 0 and 1 and sets every C = 1 before its one
barrier.

The fp16 variant of flat_collect_kernel stages two tiles at a time: its stage s holds tiles
2s and 2s + 1 and their norms (slots 2s, 2s + 1 of eight, a pair per stage: pair slot s % 4),
and during stage s a wave also reads the norms of stage s itself (tile 2s's keys, tested
during tile 2s + 1's MFMAs), so its reads are pair slots (s - 1) % 4 and s % 4.

The per-split list scan of lists of 32 (flat_scan_kernel, px_flat.hip) and that kernel's
collect mode use the same waits in another order: stage s reads buffer s % 3 for its MFMAs
and then, in the stage's own epilogue, the keys of tile s from norm slot s % 4 (the list
insertions, or the keys kept for the next stage's tests); after the wait there is no read,
only the write of stage s + 2 (the next stage's A operands are read at its start).

The model runs the eight waves of a workgroup under random interleavings, with every read
an interval that other waves' steps may fall inside, and checks that no wave waits forever,
that every read finds the stage it expects in every wave's part, and that no write lands on
a buffer or slot while a wave is reading it. Broken variants (a wait one stage short, the
write moved before the wait) must be caught.
"""
import random

import pytest

STAGE_BUFS, NORM_BUFS, WAVES = 3, 4, 8


class Violation(AssertionError):
    pass


def _wave_program(s_count, live, c_off=0, write_first=False, pairs=False, lists=False):
    """The steps of one wave: ('read'|'end'|'write'|'set'|'wait', ...) in program order.
    lists: flat_scan_kernel's order (tile s's norms read in stage s's epilogue, no read after
    the wait)."""
    prog = []
    for s in range(s_count):
        if live:
            prog.append(("read", "buf", s % STAGE_BUFS, s))          # MFMAs of stage s
            if lists:
                prog.append(("read", "norm", s % NORM_BUFS, s))      # the stage's epilogue
            elif s > 0:
                prog.append(("read", "norm", (s - 1) % NORM_BUFS, s - 1))
            if pairs:  # two tiles a stage: the first tile's norms, tested during the second
                prog.append(("read", "norm", s % NORM_BUFS, s))
            prog.append(("end",))
        if write_first:
            prog.append(("write", s + 2))
        prog.append(("wait", s + 1 + c_off))
        if live and not lists and s + 1 < s_count:
            prog.append(("read", "buf", (s + 1) % STAGE_BUFS, s + 1))  # next A operands
            prog.append(("end",))
        if not write_first:
            prog.append(("write", s + 2))
        prog.append(("set", s + 2))
    if live and not lists:
        prog.append(("read", "norm", (s_count - 1) % NORM_BUFS, s_count - 1))
        prog.append(("end",))
    return prog


def run_schedule(s_count, live_waves, seed, max_steps=10**6, **variant):
    rnd = random.Random(seed)
    progs = [_wave_program(s_count, w < live_waves, **variant) for w in range(WAVES)]
    pc = [0] * WAVES
    C = [1] * WAVES
    # per buffer or norm slot, the stage of each wave's part (every wave writes its rows
    # of a stage buffer; wave 0 alone writes the norms); None: never written
    held = {("buf", b): [None] * WAVES for b in range(STAGE_BUFS)}
    held.update({("norm", b): [None] * WAVES for b in range(NORM_BUFS)})
    for stage in (0, 1):
        held[("buf", stage)] = [stage] * WAVES
        held[("norm", stage)][0] = stage
    writers = {"buf": range(WAVES), "norm": (0,)}

    def holds(kind, slot, stage):
        return all(held[(kind, slot)][v] == stage for v in writers[kind])

    reading = [[] for _ in range(WAVES)]  # (kind, slot, stage) being read
    for _ in range(max_steps):
        ready = [w for w in range(WAVES) if pc[w] < len(progs[w])]
        if not ready:
            return
        w = rnd.choice(ready)
        op = progs[w][pc[w]]
        if op[0] == "wait":
            if min(C) < op[1]:
                continue  # not yet: another wave moves
        elif op[0] == "read":
            kind, slot, stage = op[1:]
            if not holds(kind, slot, stage):
                raise Violation(f"wave {w} reads {kind} {slot} for stage {stage}, "
                                f"holding {held[(kind, slot)]}")
            reading[w].append((kind, slot, stage))
        elif op[0] == "end":
            for kind, slot, stage in reading[w]:
                if not holds(kind, slot, stage):
                    raise Violation(f"{kind} {slot} overwritten during wave {w}'s read")
            reading[w].clear()
        elif op[0] == "write":
            stage = op[1]
            for kind, slot in (("buf", stage % STAGE_BUFS), ("norm", stage % NORM_BUFS)):
                if w not in writers[kind]:
                    continue
                for v in range(WAVES):
                    if any(r[:2] == (kind, slot) for r in reading[v]):
                        raise Violation(f"wave {w} writes {kind} {slot} while wave {v} reads it")
                held[(kind, slot)][w] = stage
        elif op[0] == "set":
            C[w] = op[1]
        pc[w] += 1
    raise Violation("no progress: a wave waits forever")


@pytest.mark.parametrize("order", ["collect", "pairs", "lists"])
@pytest.mark.parametrize("live_waves", [8, 2, 1])
@pytest.mark.parametrize("stages", [1, 2, 3, 7, 24])
def test_protocol_holds(stages, live_waves, order):
    for seed in range(60):
        run_schedule(stages, live_waves, seed, pairs=order == "pairs", lists=order == "lists")


@pytest.mark.parametrize("variant", [dict(c_off=-1), dict(write_first=True),
                                     dict(c_off=-1, pairs=True), dict(write_first=True, pairs=True),
                                     dict(c_off=-1, lists=True), dict(write_first=True, lists=True)])
def test_broken_variants_are_caught(variant):
    # a wait for C >= s lets a wave read stage s + 1's buffer before every wave has written
    # its part; writing stage s + 2 before the wait overwrites stage s - 1's buffer while a
    # slower wave may still read it
    with pytest.raises(Violation):
        for seed in range(400):
            run_schedule(12, 8, seed, **variant)
