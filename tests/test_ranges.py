"""CPU checks of the library's offline key-range builder, ud_chunked_limited_ranges (MaskSpec.ranges
and chunkedLimitedRanges, FastConformer.swift:324-357, with forwardOffline's clip to the valid length,
:380-381): bit-exact against the oracle's restatement, and against visibility masks built element by
element (NeMo's chunked_limited rule, tests/refimpl.py; the inclusive window that the reference
documents for chunked_limited_with_rc, FastConformer.swift:327-328)."""
import numpy as np
import pytest

import refimpl


def _ranges_from_mask(visible):
    """[T, 2] ranges of a boolean visibility matrix whose rows are contiguous runs."""
    T = visible.shape[0]
    out = np.zeros((T, 2), np.int32)
    for i in range(T):
        js = np.flatnonzero(visible[i])
        if len(js):
            assert js[-1] - js[0] + 1 == len(js), "row %d is not one run" % i
            out[i] = [js[0], js[-1] + 1]
    return out


@pytest.mark.parametrize("T,left,right", [(300, 70, 1), (157, 70, 13), (64, 0, 0), (50, 64, 3), (1, 5, 2),
                                          (1500, 70, 6)])
def test_chunked_limited_matches_oracle(ud, orc, T, left, right):
    got = ud.chunked_limited_ranges(T, left, right)
    assert got.shape == (1, T, 2)
    np.testing.assert_array_equal(got[0], orc.chunked_limited_ranges(T, left, right))


@pytest.mark.parametrize("T,left,right", [(300, 70, 1), (157, 70, 13), (40, 8, 3)])
def test_chunked_limited_clipped_matches_nemo_mask(ud, T, left, right):
    valid = np.array([T, T - 1, T // 2, 1, 0], np.int32)
    got = ud.chunked_limited_ranges(T, left, right, valid=valid)
    for b, v in enumerate(valid):
        hidden = refimpl.chunked_limited_mask(T, left, right, int(v))
        ref = _ranges_from_mask(~hidden)
        for i in range(T):
            lo, hi = got[b, i]
            if ref[i, 1] > ref[i, 0]:
                assert (lo, hi) == tuple(ref[i]), (b, i)
            else:
                assert hi <= lo, (b, i)          # the reference's clip leaves an empty range


@pytest.mark.parametrize("T,left,chunk,right", [(100, 16, 8, 2), (37, 0, 5, 0), (64, 70, 4, 7), (9, 3, 20, 1)])
def test_chunked_limited_rc_matches_window(ud, T, left, chunk, right):
    valid = np.array([T, T - 3], np.int32)
    got = ud.chunked_limited_ranges(T, left, right, valid=valid, chunk=chunk)
    i = np.arange(T)[:, None]
    j = np.arange(T)[None, :]
    c = i // chunk
    for b, v in enumerate(valid):
        visible = (j >= c * chunk - left) & (j <= c * chunk + chunk - 1 + right) & (j < v)
        ref = _ranges_from_mask(visible)
        for q in range(T):
            lo, hi = got[b, q]
            if ref[q, 1] > ref[q, 0]:
                assert (lo, hi) == tuple(ref[q]), (b, q)
            else:
                assert hi <= lo, (b, q)


def test_ranges_errors(ud):
    with pytest.raises(ud.EngineError):
        ud.chunked_limited_ranges(0, 70, 1)
    with pytest.raises(ud.EngineError):
        ud.chunked_limited_ranges(10, 4, 1, chunk=0)
    with pytest.raises(ud.EngineError):
        ud.chunked_limited_ranges(10, -1, 1)
