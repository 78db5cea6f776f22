"""Rolling-window host-to-device bandwidth estimate (mirrors transfer/bandwidth.py:13-97 of
the reference: fed by every successful transfer, read for observability only).

Throughput is total bytes of the samples inside the window divided by the time since the
oldest of them, in GiB/s (1024**3 bytes, as the reference reports it); fewer than two
samples give 0.0.  ``peak_gbps`` is the largest value seen at a ``record`` since the last
``reset``.
"""
from __future__ import annotations

import collections
import time


class BandwidthMonitor:
    def __init__(self, window_s: float = 5.0):
        if window_s <= 0:
            raise ValueError("window_s must be positive")
        self.window_s = window_s
        self._samples: collections.deque[tuple[float, int]] = collections.deque()
        self._peak_gbps = 0.0

    def record(self, bytes_transferred: int, now: float | None = None) -> None:
        t = time.monotonic() if now is None else now
        self._samples.append((t, int(bytes_transferred)))
        self._trim(t)
        self._peak_gbps = max(self._peak_gbps, self.current_gbps(t))

    def _trim(self, now: float) -> None:
        while self._samples and self._samples[0][0] < now - self.window_s:
            self._samples.popleft()

    def bytes_in_window(self, now: float | None = None) -> int:
        self._trim(time.monotonic() if now is None else now)
        return sum(b for _, b in self._samples)

    def current_gbps(self, now: float | None = None) -> float:
        t = time.monotonic() if now is None else now
        self._trim(t)
        if len(self._samples) < 2:
            return 0.0
        span = t - self._samples[0][0]
        if span <= 0:
            return 0.0
        return sum(b for _, b in self._samples) / span / float(1 << 30)

    def peak_gbps(self) -> float:
        return self._peak_gbps

    def reset(self) -> None:
        self._samples.clear()
        self._peak_gbps = 0.0
