"""CPU tests of the clock arithmetic that turns two ``h3a_clock_sample``
records into per-CU core clocks (``h3_flash_amd.devclock.mean_clock``).

Records are (XCD, HW_REG_HW_ID, memtime, realtime). The cycle counters of
different CUs are not aligned, so a record must be compared with the record
of the same (XCD, CU) in the other sample, whatever the workgroup order; the
cases below give CUs offsets far apart, so matching by position or pooling
counters over an XCD gives wrong clocks.
"""

from __future__ import annotations

import pytest

from h3_flash_amd.devclock import mean_clock


def hw_id(cu: int, simd: int = 0, wave: int = 0) -> int:
    return (cu << 8) | (simd << 4) | wave


def test_same_cu_matched_across_orders():
    # XCD 0: CUs 3 and 5 at 1500 and 1600 MHz; XCD 1: CU 3 at 1400 MHz.
    # Realtime is 100 MHz: 10,000 ticks = 100 us, and f MHz over them is
    # f * 100 cycles.
    before = [
        (0, hw_id(3), 10_000_000, 500),
        (1, hw_id(3), 999_000_000, 505),
        (0, hw_id(5), 7_000, 502),
    ]
    after = [
        (0, hw_id(5), 7_000 + 1600 * 100, 10_502),
        (0, hw_id(3), 10_000_000 + 1500 * 100, 10_500),
        (1, hw_id(3), 999_000_000 + 1400 * 100, 10_505),
    ]
    r = mean_clock(before, after)
    assert r["cus"] == 3
    assert r["sclk_mhz"] == pytest.approx((1500 + 1600 + 1400) / 3)
    assert r["sclk_min_mhz"] == pytest.approx(1400)
    assert r["sclk_max_mhz"] == pytest.approx(1600)
    assert r["sclk_by_xcd_mhz"] == {"0": pytest.approx(1550), "1": pytest.approx(1400)}
    assert r["span_us"] == pytest.approx(100.0)


def test_earliest_record_of_a_cu_is_used_and_waves_share_the_cu():
    # Two waves on one CU (different SIMD / wave fields); the counter is the
    # CU's, so either record serves; the earliest one is taken.
    before = [(2, hw_id(7, 1, 2), 1_000_300, 103), (2, hw_id(7, 0, 0), 1_000_000, 100)]
    after = [(2, hw_id(7, 3, 1), 1_000_000 + 20 * 50, 150), (2, hw_id(7, 2, 0), 1_000_000 + 20 * 60, 160)]
    r = mean_clock(before, after)
    assert r["cus"] == 1
    assert r["sclk_mhz"] == pytest.approx(2000.0)


def test_unmatched_and_inconsistent_records_are_dropped():
    before = [(0, hw_id(1), 100, 10), (0, hw_id(2), 500, 10), (3, hw_id(1), 50, 10)]
    after = [(0, hw_id(1), 100 + 15 * 10, 20), (0, hw_id(2), 400, 20), (4, hw_id(1), 9_999, 20)]
    r = mean_clock(before, after)
    assert r["cus"] == 1  # CU 2 went backwards, XCD 3 / 4 never met
    assert r["sclk_mhz"] == pytest.approx(1500.0)
    assert mean_clock([], after) == {"sclk_mhz": None, "cus": 0}


def test_pooling_an_xcd_would_be_wrong():
    # The two CUs' counters differ by 10^9 cycles: any estimate that mixes
    # them (first record of the XCD before, another CU's after) is far off.
    before = [(0, hw_id(0), 0, 0), (0, hw_id(1), 1_000_000_000, 0)]
    after = [(0, hw_id(1), 1_000_000_000 + 15 * 1000, 1000), (0, hw_id(0), 15 * 1000, 1000)]
    assert mean_clock(before, after)["sclk_mhz"] == pytest.approx(1500.0)
