"""The library's host-side Swin tables (ien_position_bias, ien_bias_tables)
against the oracle, bit for bit, and the window geometry checks (no GPU)."""

import numpy as np
import pytest


@pytest.mark.parametrize("window", [7, 8, 12])
def test_position_bias_matches_oracle(oracle, window):
    import ien

    rng = np.random.default_rng(window)
    side, heads = 2 * window - 1, 3
    t = rng.standard_normal((heads, side, side)).astype(np.float32)
    assert np.array_equal(ien.position_bias(t, heads, window, ien.POS_SCUNET),
                          oracle.position_bias(t, heads, window, oracle.POS_SCUNET))
    ts = rng.standard_normal((side * side, heads)).astype(np.float32)
    assert np.array_equal(ien.position_bias(ts, heads, window, ien.POS_SWIN),
                          oracle.position_bias(ts, heads, window, oracle.POS_SWIN))


@pytest.mark.parametrize("window,shift,masked", [(8, 4, -np.inf), (8, 0, -np.inf), (7, 3, -100.0), (12, 6, -100.0)])
def test_bias_tables_match_oracle(oracle, window, shift, masked):
    import ien

    p = np.random.default_rng(2).standard_normal((2, window * window, window * window)).astype(np.float32)
    assert np.array_equal(ien.bias_tables(p, window, shift, masked), oracle.bias_tables(p, window, shift, masked))


def test_window_geometry():
    import ien

    assert ien.window_count(ien.windows(8, 4, 16, 24)) == 6
    assert ien.window_count(ien.windows(7, 3, 10, 10)) == 4     # padded to 14 x 14
    assert ien.window_count(ien.windows(12, 6, 256, 256)) == 484  # 22 x 22, padded to 264
    for bad in [(8, 8, 16, 16), (17, 0, 32, 32), (8, -1, 16, 16), (8, 0, 0, 16)]:
        with pytest.raises(ien.IenError):
            ien.window_count(ien.windows(*bad))
