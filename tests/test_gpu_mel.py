"""GPU parity of the log-mel frontend (ud_mel_features) against the oracle's NemoMelFrontend
restatement: several clips per call (speech-like, uniform noise, short and empty clips), the
zeroed final frame, frame-wise determinism across batch compositions, and error paths."""
import numpy as np
import pytest

import harness
import refimpl

pytestmark = pytest.mark.gpu

# log-mel units.  The oracle accumulates the DFT in double over the same fp32 tables; the kernel
# accumulates in fp32 FMAs as the reference's sgemm does.  Frames are compared where the oracle's
# mel energy is above the log guard's scale (log value > -15); the bar then bounds the relative
# power error the fp32 DFT may make on a frame's weakest bands.
MEL_TOL = 2e-3


def _clips(orc):
    return [harness.speechlike(16000 + 77, 1), orc.lcg_floats(12345, 2) * np.float32(0.5),
            harness.speechlike(3210, 3, scale=0.05), orc.lcg_floats(199, 4), orc.lcg_floats(1, 5),
            np.zeros(0, np.float32), orc.lcg_floats(160 * 37, 6)]


def _close(got, ref, what):
    assert got.shape == ref.shape, what
    err = np.abs(got - ref)
    live = ref > -15.0
    assert float(err[live].max(initial=0.0)) <= MEL_TOL, "%s: %.3g" % (what, err[live].max(initial=0.0))
    assert float(err.max(initial=0.0)) <= 5e-2, what
    assert harness.cosine(got, ref) >= 0.999999 or got.size == 0 or not np.any(ref), what


def test_features_match_oracle(gpu, orc):
    ud = gpu
    fb, win = refimpl.slaney_mel_fb(), refimpl.hann_symmetric()
    fe = ud.MelFrontend(fb, win)
    ofe = orc.MelFrontend(fb, win)
    clips = _clips(orc)
    got = fe.features(clips)
    for b, c in enumerate(clips):
        ref = ofe.features(c)
        assert got[b].shape == (c.size // 160 + 1, 128)
        assert np.all(got[b][-1] == 0), b
        _close(got[b], ref, "clip %d (%d samples)" % (b, c.size))
    fe.close()


def test_frames_independent_of_batch(gpu, orc):
    """A frame's value does not depend on the clip's position in the batch or on the batch size."""
    ud = gpu
    fe = ud.MelFrontend(refimpl.slaney_mel_fb(), refimpl.hann_symmetric())
    clips = _clips(orc)
    together = fe.features(clips)
    for b in (0, 2, 6):
        alone = fe.features([clips[b]])[0]
        assert np.array_equal(alone.view(np.uint32), together[b].view(np.uint32))
    swapped = fe.features(clips[::-1])
    for b in range(len(clips)):
        assert np.array_equal(swapped[len(clips) - 1 - b], together[b])


def test_frames_independent_of_workgroup_size(gpu, orc):
    """A large call runs 8 frames per workgroup, a small one 4 (below 1024 workgroups of 8); a
    clip's frames are bit-identical either way, and match the oracle in the large call."""
    ud = gpu
    fb, win = refimpl.slaney_mel_fb(), refimpl.hann_symmetric()
    fe = ud.MelFrontend(fb, win)
    ofe = orc.MelFrontend(fb, win)
    clips = [harness.speechlike(16000 + 37 * b, 100 + b) for b in range(80)]   # 80 x 13 groups of 8
    big = fe.features(clips)
    for b in (0, 41, 79):
        alone = fe.features([clips[b]])[0]
        assert np.array_equal(alone.view(np.uint32), big[b].view(np.uint32)), b
        _close(big[b], ofe.features(clips[b]), "clip %d of the large call" % b)
    fe.close()


def test_constant_filterbank_kat(gpu, orc):
    """The reference KAT's frontend (StreamingEquivalenceTests.swift:10-11): constant 0.01
    filterbank, symmetric Hann, 16123 LCG samples of seed 5."""
    ud = gpu
    fb, win = np.full((128, 257), 0.01, np.float32), refimpl.hann_symmetric()
    audio = orc.lcg_floats(16123, 5)
    got = ud.MelFrontend(fb, win).features([audio])[0]
    _close(got, orc.MelFrontend(fb, win).features(audio), "kat")


def test_sparse_filterbank_bands(gpu, orc):
    """Each band sums only its first..last nonzero bins: one-bin bands at every bin position (0 and
    256 included), a band with weights at the two end bins only, and an all-zero band."""
    ud = gpu
    fb = np.zeros((130, 257), np.float32)
    for m in range(128):
        fb[m, 2 * m + (m & 1)] = 0.5
    fb[128, 0] = fb[128, 256] = 1.0
    fb = np.concatenate([fb, np.zeros((1, 257), np.float32)])[:130]    # band 129: all zero
    fb[127, 256] = 0.25
    win = refimpl.hann_symmetric()
    audio = harness.speechlike(8000 + 11, 7)
    got = ud.MelFrontend(fb, win).features([audio])[0]
    ref = orc.MelFrontend(fb, win).features(audio)
    _close(got, ref, "sparse filterbank")
    z = got[:-1, 129]
    assert np.all(z == z[0]) and abs(float(z[0]) - np.log(2.0 ** -24)) < 1e-6


def test_mel_error_paths(gpu):
    ud = gpu
    with pytest.raises(ud.EngineError) as e:
        ud.MelFrontend(np.zeros((300, 257), np.float32), refimpl.hann_symmetric())
    assert e.value.status == -2
    fe = ud.MelFrontend(refimpl.slaney_mel_fb(), refimpl.hann_symmetric())
    a = ud.DeviceBuffer(2 * 1000 * 4)
    o = ud.DeviceBuffer(2 * 7 * 128 * 4)
    with pytest.raises(ud.EngineError) as e:
        fe.features_device(2, a, 1000, [1000, 1001], o, 7)        # clip longer than the stride
    assert e.value.status == -2
    with pytest.raises(ud.EngineError) as e:
        fe.features_device(2, a, 1000, [1000, 960], o, 6)         # 7 frames do not fit 6 rows
    assert e.value.status == -2
    assert list(fe.features_device(2, a, 1000, [1000, 960], o, 7)) == [7, 7]
    fe.close()
