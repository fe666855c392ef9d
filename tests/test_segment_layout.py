"""Host-side Gram schedules of ``ops.SegmentLayout`` (CPU tables, no kernel).

The grouped split kernel takes every segment of 1 .. 320 rows as a set of two
items (A and G) that must sit on one XCD (one eighth of the launch table) and
write the segment's tile-pair records from its first slot; the tile-pair
kernel takes the longer segments' pairs.  Every record slot must be written
by exactly one of the two launches.
"""

from __future__ import annotations

import numpy as np

from opake_amd import ops

LENGTHS = [[0, 1, 63, 64, 65, 255, 256], [130, 0, 200, 7, 128, 257, 288],
           [256, 300, 2, 0, 64, 321, 1000]]
DIMS = [(64, 96), (128, 40), (32, 256)]


def _npairs(n):
    nt = (n + 127) // 128
    return nt * (nt + 1) // 2


def _table(t, n):
    return t.cpu().numpy().astype(np.int64).reshape(-1, 4)[:n]


def test_split_schedule_covers_every_record_once():
    layout = ops.SegmentLayout(LENGTHS, "cpu", gram_dims=DIMS)
    lens = np.asarray(LENGTHS).reshape(-1)
    first = np.concatenate([[0], np.cumsum([_npairs(n) for n in lens])])
    assert layout.n_items == first[-1]
    short = (lens >= 1) & (lens <= ops.SegmentLayout.SPLIT_MAX_ROWS)
    assert layout.n_sets == int(short.sum())

    sets = _table(layout.set_items, layout.n_set_items)
    assert len(sets) % 8 == 0
    per = len(sets) // 8
    live = sets[sets[:, 0] >= 0]
    assert len(live) == 2 * layout.n_sets
    written = np.zeros(layout.n_items, dtype=int)
    seen = {}
    for idx, (w0, row0, rows, slot) in enumerate(sets):
        if w0 < 0:
            continue
        problem, op, s = w0 & 0xFF, (w0 >> 8) & 1, w0 >> 9
        seen.setdefault(s, []).append((op, idx // per, problem, row0, rows, slot))
    for s, pair in seen.items():
        assert sorted(p[0] for p in pair) == [0, 1], s
        assert pair[0][1:] == pair[1][1:], s  # same XCD, segment and slot
        _, _, problem, row0, rows, slot = pair[0]
        k = np.nonzero(np.cumsum(LENGTHS[problem]) - LENGTHS[problem] == row0)[0]
        v = problem * len(LENGTHS[0]) + [kk for kk in k if LENGTHS[problem][kk] == rows][0]
        assert slot == first[v] and 1 <= rows <= ops.SegmentLayout.SPLIT_MAX_ROWS
        written[slot:slot + _npairs(rows)] += 1
    assert len(seen) == layout.n_sets

    pairs = _table(layout.long_items, layout.n_long_items)
    for w0, row0, rows, slot in pairs:
        if w0 < 0:
            continue
        assert rows > ops.SegmentLayout.SPLIT_MAX_ROWS
        written[slot] += 1
    assert (written == 1).all()

    # The tile-pair schedule of every segment (other dtypes) still covers all.
    every = _table(layout.items, layout.n_launch_items)
    slots = every[every[:, 0] >= 0, 3]
    assert sorted(slots.tolist()) == list(range(layout.n_items))


def test_split_schedule_runs_expensive_items_first_per_xcd():
    lengths = [[240 + (7 * k) % 75 for k in range(16)] for _ in range(4)]
    dims = [(2048, 11264), (5632, 2048), (2048, 11264), (5632, 2048)]
    layout = ops.SegmentLayout(lengths, "cpu", gram_dims=dims)
    sets = _table(layout.set_items, layout.n_set_items)
    per = len(sets) // 8
    for x in range(8):
        part = sets[x * per:(x + 1) * per]
        part = part[part[:, 0] >= 0]
        prob, op = part[:, 0] & 0xFF, (part[:, 0] >> 8) & 1
        k = np.asarray(dims)[prob, op]
        blocks = np.where(part[:, 2] > 288, 55, np.where(part[:, 2] > 256, 45, 36))
        cost = k * blocks
        assert (np.diff(cost) <= 0).all(), x
