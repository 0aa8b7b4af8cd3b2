"""Pins the oracle's mel frontend (orc_mel_tables / orc_mel_frames) and its NemoMelStream restatement:
the reference KAT NemoMelStream == features (Tests/DictatorEngineTests/StreamingEquivalenceTests.swift:9-20),
torch.stft in NeMo's FilterbankFeatures arrangement, numpy.fft.rfft, and short clips."""
import numpy as np
import pytest

import refimpl


@pytest.fixture(scope="module")
def orc():
    from oracle import oracle as o
    o.lib()
    return o


def _speechlike(n, seed):
    """Harmonics with a slow envelope over low-level noise: ~60 dB of spectral dynamic range."""
    rng = np.random.default_rng(seed)
    t = np.arange(n) / 16000.0
    f0 = 120 + 40 * np.sin(2 * np.pi * 0.7 * t)
    ph = 2 * np.pi * np.cumsum(f0) / 16000.0
    x = sum(np.sin(h * ph) / h for h in range(1, 12)) * (0.2 + 0.15 * np.sin(2 * np.pi * 1.3 * t))
    return (0.3 * x + 1e-3 * rng.standard_normal(n)).astype(np.float32)


def test_stream_equals_full_kat(orc):
    """StreamingEquivalenceTests.testNemoMelStreamEqualsFullUtterance: constant 0.01 filterbank,
    symmetric Hann window, 16123 LCG samples (seed 5) pushed in sizes 1, 37, 160, 999, 3000."""
    fe = orc.MelFrontend(np.full((128, 257), 0.01, np.float32), refimpl.hann_symmetric())
    audio = orc.lcg_floats(16000 + 123, 5)
    full = fe.features(audio)
    st = orc.MelStream(fe)
    got, i, sizes = [], 0, [1, 37, 160, 999, 3000]
    while i < audio.size:
        n = min(sizes[0], audio.size - i)
        sizes.append(sizes.pop(0))
        got.append(st.push(audio[i:i + n]))
        i += n
    got.append(st.finish())
    got = np.concatenate(got)
    assert got.shape == full.shape == (16123 // 160 + 1, 128)
    assert np.abs(got - full).max() < 1e-4
    assert np.array_equal(got, full)            # frame-wise computation: exactly equal here
    assert np.all(full[-1] == 0) and np.all(np.isfinite(full))


@pytest.mark.parametrize("signal", ["lcg", "speech"])
def test_features_match_torch_stft_and_rfft(orc, signal):
    fb = refimpl.slaney_mel_fb()
    win = refimpl.hann_symmetric()
    n = 16000 + 77
    audio = orc.lcg_floats(n, 11) * np.float32(0.5) if signal == "lcg" else _speechlike(n, 12)
    fe = orc.MelFrontend(fb, win)
    got = fe.features(audio)
    ref = refimpl.mel_nemo(audio, fb, win)
    ref2 = refimpl.mel_rfft(audio, fb, win)
    assert got.shape == ref.shape == ref2.shape
    # The oracle differs from an exact DFT only by its fp32 tables (entries rounded to float,
    # relative 6e-8): in log-mel units that stays far below 1e-4 wherever mel >> 2^-24.
    assert np.abs(got - ref).max() <= 1e-4, np.abs(got - ref).max()
    assert np.abs(got - ref2).max() <= 1e-4
    assert np.abs(ref - ref2).max() <= 1e-9       # the two library routines agree with each other
    assert np.all(got[-1] == 0)
    # a plausible slip shows: the window one sample late changes the features well beyond the bar
    shifted = refimpl.mel_rfft(np.concatenate([[0.0], audio[:-1]]).astype(np.float32), fb, win)
    assert np.abs(shifted - got).max() > 1e-2


@pytest.mark.parametrize("n", [1, 150, 160, 199, 200, 201, 359, 360, 361, 1601])
def test_short_clips(orc, n):
    fb = refimpl.slaney_mel_fb()
    win = refimpl.hann_symmetric()
    audio = orc.lcg_floats(n, 3 + n)
    fe = orc.MelFrontend(fb, win)
    got = fe.features(audio)
    ref = refimpl.mel_rfft(audio, fb, win)
    assert got.shape == (n // 160 + 1, 128)
    assert np.abs(got - ref).max() <= 1e-4
    st = orc.MelStream(fe)
    inc = np.concatenate([st.push(audio[:n // 2]), st.push(audio[n // 2:]), st.finish()])
    assert np.array_equal(inc, got)


def test_empty_clip(orc):
    fe = orc.MelFrontend(refimpl.slaney_mel_fb(), refimpl.hann_symmetric())
    got = fe.features(np.zeros(0, np.float32))
    assert got.shape == (1, 128) and np.all(got == 0)
