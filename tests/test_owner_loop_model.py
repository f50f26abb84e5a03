"""CPU model of the tile kernel's owner loop: which LDS record slots it reads.

In ``msda_tile_backward`` (muspace_amd/csrc/msda_backward_tiles.hpp, phase D) a
lane group owns one position of the sorted batch and walks its records, slots
``first + stride * r`` for r = 0 .. cnt-1, with NR = 2 records in flight:
register set j holds record r + j; once it is consumed -- its slot is
overwritten with the four corner dot products D_0..D_3, whose float bits are
not a record -- the set is refilled from slot ``min(r + j + NR, cnt - 1)``,
keeping its old (valid) record when ``r + j + NR >= cnt``, and the set's
grad_out row is loaded from the query in the record's id.

An earlier form refilled unconditionally from the clamped slot, which for
some counts re-read the already consumed last slot and took D bits for a
record id: a garbage query and an out-of-range grad_out row, which faulted the
GPU. This model replays both forms over every count a group can hold and
checks that the current one (a) consumes every record exactly once, in order,
(b) never keeps a value read from a consumed slot, and (c) only ever forms
grad_out addresses from real record ids, so the kernel's ``min(q, queries-1)``
clamp on the row address never changes a value.
"""

import pytest

NR = 2  # grad_out rows in flight per group (msda_tile_backward)
CONSUMED = object()  # a slot holding D_0..D_3 instead of a record


def _owner_loop(cnt, first, stride, refill_keeps_old_record=True):
    """Replay one group's loop; returns (consumed order, ids used for rows,
    values kept from consumed slots)."""
    slots = {first + stride * r: ("record", r) for r in range(cnt)}
    consumed, row_ids, bad_keeps = [], [], []

    def read(slot):
        return slots[slot]

    e = [None] * NR
    for j in range(NR):  # prologue
        e[j] = read(first + stride * min(j, cnt - 1))
        row_ids.append(e[j])
    r = 0
    while r < cnt:
        for j in range(NR):
            if r + j < cnt:
                assert e[j] == ("record", r + j), (cnt, r, j, e[j])
                consumed.append(e[j][1])
                slots[first + stride * (r + j)] = CONSUMED
            nx = r + j + NR
            t = read(first + stride * min(nx, cnt - 1))
            if refill_keeps_old_record:
                e[j] = t if nx < cnt else e[j]
            else:
                e[j] = t
            if e[j] is t and t is CONSUMED:
                bad_keeps.append((r, j))
            row_ids.append(e[j])
        r += NR
    return consumed, row_ids, bad_keeps


@pytest.mark.parametrize("stride", [1, 2, 4])
def test_current_refill_never_keeps_a_consumed_slot(stride):
    for cnt in range(1, 129):
        for sub in range(stride):
            consumed, row_ids, bad = _owner_loop(cnt, first=7 + sub, stride=stride)
            assert consumed == list(range(cnt)), cnt
            assert bad == [], (cnt, bad)
            # every grad_out row address comes from a real record of this group:
            # its query is in range, so the row-address clamp is never needed
            assert all(isinstance(i, tuple) and i[0] == "record" and 0 <= i[1] < cnt
                       for i in row_ids), cnt


def test_unconditional_refill_reads_a_consumed_slot():
    """The earlier form fails the same check (the model detects the fault)."""
    failing = [cnt for cnt in range(1, 41)
               if _owner_loop(cnt, first=0, stride=1, refill_keeps_old_record=False)[2]]
    assert failing == list(range(1, 41))
