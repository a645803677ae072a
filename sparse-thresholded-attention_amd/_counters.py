"""Measurement-only counters kept on the device between reads.

The per-query drop-ins expose cumulative statistics of their selection (how often a tile's union
overflowed k_max, how far PQ Stream's positions spread, ...) through get_overflow_stats() /
reset_overflow_stats(), as their reference modules do.  Those numbers must not cost a host sync
per call, so each phase keeps one float64 device vector of running sums and one of running
maxima, each updated by one in-place torch op per call, next to host-side element counts; a read
syncs once.
"""
import torch


class PhaseCounters:
    """Running sums and maxima of per-call device statistics for one phase (prefill / decode)."""

    def __init__(self, sums, maxes=(), counts=("cells",)):
        self.sum_names = tuple(sums)
        self.max_names = tuple(maxes)
        self.count_names = tuple(counts)
        self.clear()

    def clear(self):
        self._sums = None
        self._maxes = None
        self.counts = {n: 0 for n in self.count_names}

    def add(self, counts, sums, maxes=()):
        """counts: {name: int}; sums / maxes: device 0-d tensors in declaration order."""
        for n, c in counts.items():
            self.counts[n] += int(c)
        s = torch.stack([x.to(torch.float64) for x in sums])
        if self._sums is None:
            self._sums = s
        else:
            self._sums.add_(s)
        if self.max_names:
            m = torch.stack([x.to(torch.float64) for x in maxes])
            if self._maxes is None:
                self._maxes = m
            else:
                torch.maximum(self._maxes, m, out=self._maxes)

    def read(self):
        """(counts, sums, maxes) as plain Python dicts; zeros before the first add."""
        sums = self._sums.tolist() if self._sums is not None else [0.0] * len(self.sum_names)
        maxes = self._maxes.tolist() if self._maxes is not None else [0.0] * len(self.max_names)
        return dict(self.counts), dict(zip(self.sum_names, sums)), dict(zip(self.max_names, maxes))


def ratio(a, b):
    return (a / b) if b else 0.0
