"""The shader clock a timed loop ran at, per XCD, from clock stamps on its stream.

The MI355X runs MFMA-heavy kernels under its power limit, well below the
2.4 GHz its peak figures assume, and the clock it settles at differs from
part to part by several percent. A throughput figure without the clock it was
taken at cannot be told apart from a regression, so bench.py brackets each
timed loop with :class:`ClockWindow`: ``start()`` and ``stop()`` enqueue
``mb_clock_stamp`` on the loop's stream, right before its first launch and
right after its last. Each stamp has a block on every CU read that CU's
shader-clock counter (``s_memtime``) and the constant 100 MHz counter
(``s_memrealtime``). The shader-clock counters of different CUs are not
synchronised (they differ by ~1e8 cycles within one XCD), so the stamps are
paired CU by CU, and for each CU seen in both

    clock = (shader_1 - shader_0) / (real_1 - real_0) * 100 MHz

is its mean shader clock over the loop, kernels and the gaps between them
alike. The CUs of an XCD share its clock; an XCD's figure is the median over
its CUs.

The SMU's metrics table (amdsmi ``current_gfxclks``) cannot serve here: on
MI355X it refreshes about once a second, so a loop of tens of milliseconds
sees one reading, taken at some earlier moment.
"""
from __future__ import annotations

import statistics
from typing import Any

from teamredbench_amd.native import capi


class ClockWindow:
    """Clock stamps before and after a region of work on `stream` (a HIP stream handle)."""

    def __init__(self, torch: Any, lib: capi.NativeLibrary, stream: int, device: str = "cuda:0"):
        self._torch, self._lib, self._stream = torch, lib, stream
        self._stamps = [torch.zeros(4 * capi.CLOCK_BLOCKS, dtype=torch.int64, device=device) for _ in range(2)]

    def start(self) -> None:
        self._lib.clock_stamp(self._stamps[0].data_ptr(), self._stream)

    def stop(self) -> None:
        self._lib.clock_stamp(self._stamps[1].data_ptr(), self._stream)

    def summary(self) -> dict[str, Any]:
        """Per-XCD mean shader clock (MHz) over the region and their mean / min / max; call after the stream
        has been synchronised."""
        before, after = (s.view(-1, 4).cpu().tolist() for s in self._stamps)
        return clock_summary(before, after)


def cu_key(xcd: int, hw_id: int) -> tuple[int, int]:
    """(XCD, CU within it) of a stamp block: HW_ID bits 15:8 hold the CU, shader-array and shader-engine
    ids of the wave."""
    return int(xcd), (int(hw_id) >> 8) & 0xFF


def clock_summary(before: list[list[int]], after: list[list[int]]) -> dict[str, Any]:
    """Per-XCD clocks from two stamps, each a list of [shader, real, xcd, hw_id] per block, paired CU by CU
    (a CU that ran several blocks of one stamp keeps its first). ``cus_paired`` counts the CUs seen in both
    stamps and ``cu_spread_mhz`` is the widest spread of the per-CU clocks within one XCD."""
    def by_cu(stamp: list[list[int]]) -> dict[tuple[int, int], tuple[int, int]]:
        seen: dict[tuple[int, int], tuple[int, int]] = {}
        for shader, real, xcd, hw in stamp:
            seen.setdefault(cu_key(xcd, hw), (int(shader), int(real)))
        return seen

    b, a = by_cu(before), by_cu(after)
    per_xcd: dict[int, list[float]] = {}
    for key in sorted(set(a) & set(b)):
        (s0, r0), (s1, r1) = b[key], a[key]
        if r1 > r0 and s1 >= s0:
            per_xcd.setdefault(key[0], []).append((s1 - s0) / ((r1 - r0) / capi.CLOCK_REALTIME_HZ) / 1e6)
    if not per_xcd:
        return {"available": False, "reason": "no CU appears in both stamps"}
    mhz = {x: statistics.median(v) for x, v in sorted(per_xcd.items())}
    window_s = statistics.median((a[k][1] - b[k][1]) / capi.CLOCK_REALTIME_HZ for k in set(a) & set(b))
    return {
        "available": True,
        "source": "s_memtime / s_memrealtime stamps around the timed loop, paired per CU (mb_clock_stamp)",
        "gfxclk_mhz_mean": round(statistics.fmean(mhz.values()), 1),
        "gfxclk_mhz_min": round(min(mhz.values()), 1),
        "gfxclk_mhz_max": round(max(mhz.values()), 1),
        "gfxclk_mhz_per_xcd": {str(x): round(v, 1) for x, v in mhz.items()},
        "window_s": round(window_s, 6),
        "cus_paired": sum(len(v) for v in per_xcd.values()),
        "cu_spread_mhz": round(max(max(v) - min(v) for v in per_xcd.values()), 1),
    }
