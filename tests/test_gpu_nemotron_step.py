"""GPU parity of ud_nemotron_step -- NemotronEncoder.step(mel:nRows:validRows:keepAll:) -> (proj,
frames) (Sources/DictatorCore/Nemotron/NemotronStreamer.swift:6-12; the GPU body
Sources/DictatorEngine/Models/Nemotron.swift:74-91) -- for several streams per call, against the
oracle's restatement of that step (oracle.Streamer.encoder_step), stream by stream:
  - the steps == 0 drop rule: a stream's first call drops no subsampled frame, later calls drop
    NemotronSchedule.dropExtra, and one call may mix first and later steps (two groups);
  - the keep rule: min(valid_T, outFramesPerChunk), or valid_T when keepAll (a final chunk);
  - partial valid rows (masked tail), and a chunk whose valid rows leave no kept frame."""
import numpy as np
import pytest

import harness

pytestmark = pytest.mark.gpu

LA = 1          # lookahead: 160 ms chunks


def _setup(ud, orc, S, seed=400):
    cfg = ud.EncoderConfig(layers=2, max_chunk=4, max_streams=S, dtype="f32")
    enc, model, _ = harness.make_encoder(ud, orc, cfg, seed=seed)
    sw = ud.synthetic_subsampling_weights(seed + 1)
    enc.set_subsampling_weights(sw)
    rw = ud.synthetic_rnnt_weights(seed + 2, blank_bias=0.6)
    dec = ud.Rnnt(max_streams=S)
    dec.set_weights(rw)
    return enc, model, sw, rw, dec


def test_nemotron_step_matches_oracle(gpu, orc):
    ud = gpu
    S = 3
    enc, model, sw, rw, dec = _setup(ud, orc, S)
    sched = orc.Schedule(LA)
    rng = np.random.default_rng(401)
    streams = [enc.new_stream() for _ in range(S)]
    oracles = [orc.Streamer(model, sw, rw, LA) for _ in range(S)]
    rest_rows = sched.pre_encode_cache + sched.chunk          # 25 mel rows: 2 frames after the drop
    # (active streams, mel rows, valid rows per stream, keep_all per stream)
    calls = [
        ([0, 1], sched.first_chunk, {0: sched.first_chunk, 1: 6}, {}),       # first steps, one partial
        ([0, 1], rest_rows, {0: rest_rows, 1: rest_rows}, {}),               # later steps
        ([0, 1, 2], rest_rows, {0: 20, 1: rest_rows, 2: rest_rows}, {0: True, 2: True}),  # mixed groups
        ([1, 2], rest_rows, {1: 3, 2: rest_rows}, {}),                       # stream 1: no kept frame
    ]
    P = dec.H
    checked = 0
    for active, rows, valid, keep_all in calls:
        n = len(active)
        mel = rng.standard_normal((n, rows, 128), dtype=np.float32)
        dmel = ud.DeviceBuffer.from_numpy(mel)
        proj_rows = 4
        dproj = ud.DeviceBuffer.zeros(n * proj_rows * P * 4)
        frames = dec.nemotron_step(enc, [streams[k] for k in active], dmel, rows,
                                   [valid[k] for k in active], [keep_all.get(k, False) for k in active],
                                   sched.drop_extra, sched.out_frames_per_chunk, dproj, proj_rows)
        got = dproj.download((n, proj_rows, P))
        for b, k in enumerate(active):
            ref, _ = oracles[k].encoder_step(mel[b], rows, valid[k], keep_all.get(k, False))
            assert frames[b] == ref.shape[0], (k, frames[b], ref.shape)
            if ref.shape[0]:
                assert harness.rel_err(got[b, :frames[b]], ref) <= 1e-4, k
                checked += 1
        # the streams' step counters advanced as the reference's do
        for k in active:
            assert streams[k].step == oracles[k].steps
    assert checked >= 6
    dec.close()
    enc.close()


def test_nemotron_step_refusals(gpu, orc):
    """A shape the call refuses before launching anything (projection rows too few for a group's
    frames), then the same call with enough rows: first steps keep min(4, 2) frames, or all 4
    with keep_all."""
    ud = gpu
    enc, model, sw, rw, dec = _setup(ud, orc, 2, seed=410)
    s = [enc.new_stream(), enc.new_stream()]
    sched = orc.Schedule(LA)
    mel = ud.DeviceBuffer.zeros(2 * 25 * 128 * 4)
    proj = ud.DeviceBuffer.zeros(2 * 4 * dec.H * 4)
    # a first step over 25 rows gives 4 frames: 3 projection rows per stream are too few
    with pytest.raises(ud.EngineError):
        dec.nemotron_step(enc, s, mel, 25, [25, 25], [False, False], sched.drop_extra, 2, proj, 3)
    assert s[0].step == 0                 # nothing ran
    frames = dec.nemotron_step(enc, s, mel, 25, [25, 25], [False, True], sched.drop_extra, 2, proj, 4)
    assert frames == [2, 4]
    dec.close()
    enc.close()
