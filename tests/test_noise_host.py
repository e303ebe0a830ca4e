"""The host restatement of the library's random streams (tests/philox_np.py), which the GPU test of
the default noise path checks the kernels against: Philox4x32-10 words against the Random123
known-answer vectors (the same vectors the device Philox is checked with), and the float mappings
against what they must satisfy."""
import numpy as np

import philox_np as P


def test_philox_known_answers_host():
    ctr = np.array([[0, 0, 0, 0], [0xffffffff] * 4, [0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344]], np.uint32)
    keys = [(0, 0), (0xffffffff, 0xffffffff), (0xa4093822, 0x299f31d0)]
    want = [[0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8], [0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd],
            [0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1]]
    for c, (k0, k1), w in zip(ctr, keys, want):
        assert list(P.philox4x32_10(c, k0, k1)) == w


def test_uniform_mapping_edges():
    """u01 of the smallest and largest words, and 2 u - 1 in float32: the extremes of the reset
    noise's range."""
    u = P.u01(np.array([0, 0xff, 0x100, 0x7fffffff, 0xffffffff], np.uint32))
    assert u[0] == np.float32(2.0 ** -25) and u[1] == u[0] and u[2] == np.float32(1.5 * 2.0 ** -24)
    assert u[4] == np.float32(1.0) and 0 < u.min()
    pm = u * np.float32(2) - np.float32(1)
    assert pm[0] == np.float32(-1 + 2.0 ** -24) and pm[4] == 1.0


def test_streams_distinct_and_keyed_by_both_seed_words():
    """Different streams, steps, worlds and either seed word give different words."""
    w = np.arange(64)
    base = P.uniform_pm1(0x1_0000_0001, w, 3, P.STREAM_RESET)
    for other in (P.uniform_pm1(0x1_0000_0001, w, 3, P.STREAM_INIT), P.uniform_pm1(0x1_0000_0001, w, 4, P.STREAM_RESET),
                  P.uniform_pm1(0x1_0000_0001, w + 64, 3, P.STREAM_RESET), P.uniform_pm1(0x1, w, 3, P.STREAM_RESET),
                  P.uniform_pm1(0x1_0000_0000, w, 3, P.STREAM_RESET)):
        assert (other != base).mean() > 0.99


def test_box_muller_pairs_are_standard_normal():
    """The action noise of 4096 worlds x 8 steps (950,272 draws): moments, Kolmogorov-Smirnov against
    N(0, 1), and no correlation within a Box-Muller pair (values or squares)."""
    from scipy import stats
    z = np.concatenate([P.action_noise(77, np.arange(4096), s) for s in range(8)])
    n = z.size
    assert abs(z.mean()) < 5 / np.sqrt(n) and abs(z.var() - 1) < 5 * np.sqrt(2 / n)
    assert stats.kstest(z.ravel(), "norm").statistic < 1.95 / np.sqrt(n)
    a, b = z[:, 0:28:2].ravel(), z[:, 1:29:2].ravel()
    assert abs(np.corrcoef(a, b)[0, 1]) < 5 / np.sqrt(a.size)
    assert abs(np.corrcoef(a * a, b * b)[0, 1]) < 5 / np.sqrt(a.size)
