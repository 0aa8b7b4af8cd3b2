"""Pins the oracle's NemotronStreamer restatement (oracle.Streamer): the schedule constants
(NemotronSchedule.swift:7-17; docs/specs/nemotron.md:292: 9 pre-encode frames, drop 2), the
reference property live == buffered (StreamingEquivalenceTests.swift:22-40), and chunk geometry
(every full chunk yields lookahead + 1 kept frames)."""
import numpy as np
import pytest

import harness
import refimpl
from conftest import load_pkg


@pytest.fixture(scope="module")
def orc():
    from oracle import oracle as o
    o.lib()
    return o


def _model(orc, ud, la, seed):
    cfg = ud.EncoderConfig(layers=1, max_chunk=la + 1, max_streams=1, dtype="f32")
    lw = [ud.synthetic_layer_weights(cfg, seed, 0)]
    model = orc.Model(lw, cfg.d_model, cfg.heads, cfg.ff_dim, cfg.conv_kernel)
    model.prepare(-(cfg.max_chunk - 1), cfg.left_context + cfg.max_chunk - 1)
    return model


def test_schedule_constants(orc):
    for la, first, chunk, ms in ((0, 1, 8, 80), (1, 9, 16, 160), (6, 49, 56, 560), (13, 105, 112, 1120)):
        s = orc.Schedule(la)
        assert (s.first_chunk, s.chunk, s.out_frames_per_chunk, 80 * (la + 1)) == (first, chunk, la + 1, ms)
        assert (s.pre_encode_cache, s.drop_extra, s.left_context) == (9, 2, 70)
        # both chunk kinds subsample to lookahead + 1 frames
        t = lambda n: orc.sub_next_len(orc.sub_next_len(orc.sub_next_len(n)))
        assert t(first) == la + 1 and t(9 + chunk) - 2 == la + 1


@pytest.mark.parametrize("la", [1, 2])
def test_live_equals_buffered(orc, la):
    ud = load_pkg()
    model = _model(orc, ud, la, 400 + la)
    sw = ud.synthetic_subsampling_weights(401)
    rw = ud.synthetic_rnnt_weights(402, blank_bias=0.6)
    fe = orc.MelFrontend(refimpl.slaney_mel_fb(), refimpl.hann_symmetric())
    audio = harness.speechlike(16000 + 555, 403)
    frames = audio.size // 160 + 1
    a = orc.Streamer(model, sw, rw, la, fe=fe)
    a.run_buffered(fe.features(audio), frames, frames)
    b = orc.Streamer(model, sw, rw, la, fe=fe)
    b.end_padding = False
    for i in range(0, audio.size, 1600):
        b.push(audio[i:i + 1600])
    b.flush()
    assert len(a.enc_rows) == len(b.enc_rows)
    for x, y in zip(a.enc_rows, b.enc_rows):
        assert np.array_equal(x, y)
    assert a.tokens == b.tokens
    # every chunk but the last keeps lookahead + 1 frames
    assert all(r.shape[0] == la + 1 for r in a.enc_rows[:-1])


def test_end_padding_runs_short_tail(orc):
    """A final chunk of 2 frames is dropped without end padding and run (zero-extended to 8
    frames, its 2 real rows valid) with it."""
    ud = load_pkg()
    model = _model(orc, ud, 1, 410)
    sw = ud.synthetic_subsampling_weights(411)
    rw = ud.synthetic_rnnt_weights(412)
    fe = orc.MelFrontend(refimpl.slaney_mel_fb(), refimpl.hann_symmetric())
    audio = harness.speechlike(14400, 413)       # 91 frames: 9 + 5 x 16 + 2
    runs = []
    for pad in (False, True):
        s = orc.Streamer(model, sw, rw, 1, fe=fe)
        s.end_padding = pad
        s.push(audio)
        s.flush()
        runs.append(s)
    assert len(runs[0].enc_rows) == 6 and len(runs[1].enc_rows) == 7
    for x, y in zip(runs[0].enc_rows, runs[1].enc_rows):
        assert np.array_equal(x, y)
    assert runs[1].enc_rows[-1].shape[0] == 1    # (9 + 2 valid rows of 17) -> 1 kept frame
