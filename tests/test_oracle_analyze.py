"""Pins the oracle's exponent-window selection against hand-derived answers.

The expected windows below were derived by hand from
kernel_benchmark/utils.h:189-272 (CPU) and
kernel_benchmark/zipserv_decode_attention_ext.cu:35-135 (GPU); each case
exercises one branch (tie-break, zero counts, 127-n fill with duplicates,
longest-run fallback, the 255 edge and the GPU clamp) so that a plausible
slip in either restatement changes an answer.
"""
import numpy as np
import pytest

import oracle as zo


def counts_of(d):
    c = np.zeros(256, np.int64)
    for e, n in d.items():
        c[e] = n
    return c


def test_plain_weight_window():
    c = counts_of({116: 8, 117: 7, 118: 5, 119: 4, 120: 3, 121: 2, 122: 1, 110: 1})
    assert zo.select_cpu(c) == list(range(116, 123))
    assert zo.select_gpu(c) == list(range(116, 123))


def test_tie_break_prefers_lower_exponent():
    # eight equal counts: CPU takes 100..106 (strict '>' keeps the first seen)
    c = counts_of({e: 10 for e in range(100, 108)})
    assert zo.select_cpu(c) == list(range(100, 107))
    # GPU replace-min only replaces on strictly greater, so 100..106 stay too
    assert zo.select_gpu(c) == list(range(100, 107))


def test_single_exponent_cpu_fill_and_fallback():
    # only exponent 127: candidates 127 + fill 126..121 -> no all-present
    # window -> longest run 121..127
    c = counts_of({127: 4096})
    assert zo.select_cpu(c) == list(range(121, 128))


def test_single_exponent_gpu_takes_zero_counts():
    # GPU slots start at -1 so e=0..6 (count 0) fill them; 127 replaces slot 0;
    # candidates {1..6, 127}: longest run 1..6 -> window 1..7 (127 is an outlier)
    c = counts_of({127: 4096})
    assert zo.select_gpu(c) == list(range(1, 8))


def test_cpu_fill_with_duplicates():
    # found {120,121,122}; fill 124,123,122,121 -> sorted
    # [120,121,121,122,122,123,124]; runs: best is 122,123,124 (len 3, found
    # last) -> start 122
    c = counts_of({120: 50, 121: 40, 122: 30})
    assert zo.select_cpu(c) == list(range(122, 129))


def test_noncontiguous_longest_run():
    c = counts_of({100: 9, 101: 9, 102: 9, 110: 9, 111: 9, 120: 9, 130: 9})
    assert zo.select_cpu(c) == list(range(100, 107))
    assert zo.select_gpu(c) == list(range(100, 107))


def test_first_equal_run_wins():
    # runs {50,51} and {60,61} have equal length 2: the first one is kept
    c = counts_of({50: 5, 51: 5, 60: 5, 61: 5, 70: 5, 80: 5, 90: 5})
    assert zo.select_cpu(c) == list(range(50, 57))


def test_window_at_top_edge():
    c = counts_of({e: 3 for e in range(249, 256)})
    assert zo.select_cpu(c) == list(range(249, 256))
    assert zo.select_gpu(c) == list(range(249, 256))


def test_window_past_255_cpu_unclamped_gpu_clamped():
    c = counts_of({**{e: 3 for e in range(250, 256)}, 10: 1})
    assert zo.select_cpu(c) == list(range(250, 257))
    assert zo.select_gpu(c) == list(range(248, 255))


def test_contiguous_window_not_starting_at_max():
    # top-7 = 116..122 but the most frequent is 120: window still starts at 116
    c = counts_of({120: 100, 119: 90, 121: 80, 118: 70, 122: 60, 117: 50, 116: 40, 90: 30})
    assert zo.select_cpu(c) == list(range(116, 123))


def test_first_candidate_with_all_present_window():
    # candidates 100,101,...: 100..106 has a hole at 103 -> first valid start is 104
    d = {100: 9, 101: 9, 102: 9, 104: 9, 105: 9, 106: 9, 107: 9, 108: 1, 109: 1, 110: 1}
    c = counts_of(d)
    # top-7 by count: 100,101,102,104,105,106,107; start 104 needs 104..110 > 0: yes
    assert zo.select_cpu(c) == list(range(104, 111))


def test_histogram_matches_numpy():
    rng = np.random.default_rng(3)
    a = rng.integers(0, 65536, size=10000, dtype=np.uint16)
    h = zo.histogram(a)
    np.testing.assert_array_equal(h, np.bincount((a >> 7) & 0xFF, minlength=256))


@pytest.mark.parametrize("std", [0.02, 1.0])
def test_analyze_on_data(std):
    rng = np.random.default_rng(0)
    a = zo.f32_to_bf16(rng.standard_normal(1 << 16, dtype=np.float32) * np.float32(std))
    top = zo.analyze_cpu(a)
    assert top == list(range(top[0], top[0] + 7))
    # the 7 most frequent exponents of a normal sample are contiguous
    h = zo.histogram(a)
    assert set(np.argsort(-h, kind="stable")[:7]) == set(top)
