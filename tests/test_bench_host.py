"""Host-side logic of bench.py (no GPU): leg context caps, step statistics and clock parsing."""
import pathlib

import pytest

import bench


@pytest.mark.parametrize("ctx,steps,warmup", [(512, 20, 5),       # the driver's command: --steps 20 --warmup 5
                                              (512, 256, 16),     # the defaults
                                              (512, 1, 0), (4096, 8, 64), (2048, 300, 2), (16, 5, 5)])
def test_leg_caps_cover_every_prepare(ctx, steps, warmup):
    """Every cap a later prepare() asks for lies within the model's max_ctx, and each decode leg's cap covers the
    positions it visits: ctx .. ctx + max(steps, warmup) (warm-up and timed steps both start at ctx)."""
    caps = bench.leg_caps(ctx, steps, warmup)
    for leg in ("decode", "decode_long", "prefill"):
        assert caps[leg] <= caps["max_ctx"], leg
    assert caps["decode"] >= ctx + max(steps, warmup)
    assert caps["decode_long"] >= bench.CTX_LONG + max(bench.CTX_LONG_STEPS, bench.CTX_LONG_WARMUP)
    assert caps["prefill"] >= bench.PREFILL_TOKENS


def test_step_stats_median_and_iqr():
    st = bench.step_stats([0.001 * v for v in (5, 1, 4, 2, 3)])
    assert st["n"] == 5 and st["median_ms"] == 3.0
    assert st["q1_ms"] == 2.0 and st["q3_ms"] == 4.0 and st["iqr_ms"] == 2.0


def test_read_clocks_parses_starred_levels(tmp_path: pathlib.Path):
    (tmp_path / "pp_dpm_sclk").write_text("0: 500Mhz\n1: 2400Mhz *\n")
    (tmp_path / "pp_dpm_mclk").write_text("0: 900Mhz \n1: 1900Mhz *\n")
    hw = tmp_path / "hwmon" / "hwmon3"
    hw.mkdir(parents=True)
    (hw / "temp1_input").write_text("61000\n")
    assert bench.read_clocks(tmp_path) == {"sclk_mhz": 2400, "mclk_mhz": 1900, "temp_c": 61.0}
    assert bench.read_clocks(tmp_path / "absent") == {}


def test_token_quartiles():
    q = bench.token_quartiles([float(v) for v in range(1, 10)])          # 1..9: quartiles 3 and 7 (inclusive method)
    assert q == {"q1_us": 3.0, "q3_us": 7.0, "iqr_us": 4.0}
    assert bench.token_quartiles([5.0]) == {}
