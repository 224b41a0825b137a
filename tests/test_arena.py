"""Layout of the stage-window arena (host logic; runs on the CPU)."""
import torch

from morph_amd.arena import ALIGN_LARGE, ALIGN_SMALL, STAGGER, Arena, plan

MiB = 1 << 20


def _spans(arena):
    out = []
    for row in arena.views:
        for t in row:
            out.append((t.data_ptr(), t.data_ptr() + t.numel() * t.element_size()))
    return sorted(out)


def test_large_streams_start_on_2mib_plus_a_64kib_step_per_stream():
    n = 3 * MiB // 4  # 3 MiB of float32: above the 2 MiB threshold
    groups = [[(n, torch.float32)] * 3 + [(n, torch.float16)] for _ in range(2)]
    offsets, total = plan(groups)
    for row in offsets:
        assert [o % ALIGN_LARGE for o in row] == [0, STAGGER, 2 * STAGGER, 3 * STAGGER]
    assert total >= offsets[-1][-1] + 2 * n
    arena = Arena(groups, "cpu")
    for row in arena.views:
        assert [t.data_ptr() % ALIGN_LARGE for t in row] == [0, STAGGER, 2 * STAGGER, 3 * STAGGER]
        assert [t.dtype for t in row] == [torch.float32] * 3 + [torch.float16]
        assert all(t.numel() == n for t in row)


def test_small_streams_pack_densely_and_nothing_overlaps():
    groups = [[(3072, torch.float32)] * 3 + [(3072, torch.bfloat16)] for _ in range(300)]
    groups.append([(MiB, torch.float32)] * 3)  # one large parameter among them
    offsets, total = plan(groups)
    small_bytes = 300 * 3072 * (3 * 4 + 2)
    # no 2 MiB padding per small stream: the small ones fit in their own bytes + alignment
    assert offsets[300][0] <= _round_up(small_bytes + 300 * 4 * ALIGN_SMALL, ALIGN_LARGE)
    arena = Arena(groups, "cpu")
    spans = _spans(arena)
    for (a0, a1), (b0, _) in zip(spans, spans[1:]):
        assert a1 <= b0
    assert spans[-1][1] <= arena.storage.data_ptr() + arena.nbytes
    for row in arena.views[:300]:
        assert all(t.data_ptr() % ALIGN_SMALL == 0 for t in row)


def test_views_are_independent_memory():
    groups = [[(MiB, torch.float32)] * 2]
    arena = Arena(groups, "cpu")
    a, b = arena.views[0]
    a.fill_(1.0)
    b.fill_(2.0)
    assert torch.all(a == 1.0) and torch.all(b == 2.0)


def _round_up(x, a):
    return (x + a - 1) // a * a
