"""One HBM allocation for a stage window's per-parameter streams.

The fused AdamW pass streams, for every element, the master, both moments and
the export copy of the same index at the same time.  On MI355X it runs 2-3%
faster when those streams sit in one allocation, each large stream starting
on a 2 MiB boundary plus a 64 KiB step per stream of its parameter (stream k
of a parameter at 2 MiB * j + k * 64 KiB), than when each is a separate torch
allocation (config-2 window, round-robin in one process, two instances each:
234.5-235.1 us against 240.1-241.7 us per launch; a 4 KiB step was no better
than separate allocations, a 1 MiB step in between).  This mirrors the
reference's stage window, whose state for a parameter is one `[3, N]` float32
record (streamtrain/disk.py:48, 68-69).

The streams of a small parameter (all under 2 MiB) are packed at 256-byte
alignment, so a group of a few hundred norm/bias vectors does not pay 2 MiB of
padding each.
"""
import torch

ALIGN_LARGE = 2 << 20
STAGGER = 64 << 10
ALIGN_SMALL = 256


def align_up(x, a):
    return (x + a - 1) // a * a


def plan(groups):
    """Byte offsets for `groups` (one list of (numel, dtype) streams per parameter).

    Returns (offsets, total_bytes); offsets mirrors the nesting of `groups`.
    """
    off = 0
    offsets = []
    for streams in groups:
        sizes = [int(numel) * torch.empty((), dtype=dtype).element_size()
                 for numel, dtype in streams]
        large = max(sizes, default=0) >= ALIGN_LARGE
        row = []
        for k, nbytes in enumerate(sizes):
            if large:
                off = align_up(off, ALIGN_LARGE) + k * STAGGER
            else:
                off = align_up(off, ALIGN_SMALL)
            row.append(off)
            off += nbytes
        offsets.append(row)
    return offsets, align_up(off, ALIGN_SMALL)


class Arena:
    """Flat views into one device allocation laid out by plan()."""

    def __init__(self, groups, device):
        groups = [list(s) for s in groups]
        offsets, total = plan(groups)
        # The allocator hands out large blocks at 2 MiB-aligned addresses; the
        # extra 2 MiB lets the base move up to the next boundary if it does not.
        self.storage = torch.empty(total + ALIGN_LARGE, dtype=torch.uint8, device=device)
        base = (-self.storage.data_ptr()) % ALIGN_LARGE
        self.views = []
        for streams, row in zip(groups, offsets):
            vs = []
            for (numel, dtype), off in zip(streams, row):
                nbytes = int(numel) * torch.empty((), dtype=dtype).element_size()
                start = base + off
                if start + nbytes > self.storage.numel():
                    raise AssertionError("arena plan exceeds its allocation")
                vs.append(self.storage[start:start + nbytes].view(dtype))
            self.views.append(vs)

    @property
    def nbytes(self):
        return self.storage.numel()
