"""Core clock of the GPU over a stretch of work, from ``h3a_clock_sample``.

A benchmark that quotes a fraction of the nominal MFMA peak (defined at the
part's 2.4 GHz peak engine clock) depends on the clock the part holds under
load, which differs between boards and with power. Two samples of the
per-CU cycle counters on the stream, one before and one after the timed
launches, give every CU's mean core clock over them:
``100 MHz * d(memtime) / d(realtime)``. The counters of different CUs are not
aligned, so records are matched by (XCD, CU) between the two samples.
"""

from __future__ import annotations

import ctypes
import statistics
from typing import Any

from . import _ext

REALTIME_MHZ = 100.0  # s_memrealtime's constant rate on MI300-class parts
FIELDS = 4  # xcc id, HW_REG_HW_ID, memtime, memrealtime per record


def records() -> int:
    """Workgroups (records) of one sample launch."""
    return _ext.H3A_CLOCK_RECORDS


def sample(torch: Any, device: Any) -> Any:
    """Enqueue one clock sample on the current stream; returns the (records,
    4) int64 device tensor it fills (read it after synchronising)."""

    out = torch.zeros((records(), FIELDS), dtype=torch.int64, device=device)
    lib = _ext.load_library()
    stream = torch.cuda.current_stream(device).cuda_stream
    rc = lib.h3a_clock_sample(ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(stream))
    if rc != _ext.H3A_OK:
        raise RuntimeError(_ext.last_error(lib))
    return out


def _first_by_cu(rows) -> dict[tuple[int, int], tuple[int, int]]:
    """(xcc, CU field of HW_ID) -> (memtime, realtime) of the earliest record
    of that CU."""

    seen: dict[tuple[int, int], tuple[int, int]] = {}
    for xcc, hw, cycles, ticks in rows:
        key = (int(xcc), (int(hw) >> 8) & 0xFF)
        if key not in seen or ticks < seen[key][1]:
            seen[key] = (int(cycles), int(ticks))
    return seen


def mean_clock(before, after) -> dict[str, Any]:
    """Per-CU clocks between two samples (lists of 4-tuples or (N, 4)
    arrays): the mean, median, min and max over CUs in MHz, the mean of
    each XCD, the CUs matched and the realtime span in microseconds."""

    a = _first_by_cu(before.tolist() if hasattr(before, "tolist") else before)
    b = _first_by_cu(after.tolist() if hasattr(after, "tolist") else after)
    per_cu: dict[tuple[int, int], float] = {}
    spans = []
    for key, (c0, t0) in a.items():
        if key not in b:
            continue
        c1, t1 = b[key]
        if t1 <= t0 or c1 < c0:
            continue
        per_cu[key] = REALTIME_MHZ * (c1 - c0) / (t1 - t0)
        spans.append((t1 - t0) / REALTIME_MHZ)
    if not per_cu:
        return {"sclk_mhz": None, "cus": 0}
    vals = list(per_cu.values())
    by_xcd: dict[int, list[float]] = {}
    for (xcc, _), f in per_cu.items():
        by_xcd.setdefault(xcc, []).append(f)
    return {
        "sclk_mhz": statistics.fmean(vals),
        "sclk_median_mhz": statistics.median(vals),
        "sclk_min_mhz": min(vals),
        "sclk_max_mhz": max(vals),
        "sclk_by_xcd_mhz": {str(x): statistics.fmean(v) for x, v in sorted(by_xcd.items())},
        "cus": len(vals),
        "span_us": statistics.median(spans),
    }
