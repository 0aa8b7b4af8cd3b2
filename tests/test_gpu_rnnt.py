"""GPU parity of the RNN-T joint and greedy decoder (ud_rnnt_*) against the oracle's RNNTDecoder:
the joint.enc projection, token-exact greedy decoding of several streams with state carried across
calls (blank frames, runs of 10 symbols, a token then blank), and the mel -> tokens chain through
the fp32 encoder step."""
import numpy as np
import pytest

import harness

pytestmark = pytest.mark.gpu


def _dec(ud, orc, seed, blank_bias, S):
    w = ud.synthetic_rnnt_weights(seed, blank_bias=blank_bias)
    r = ud.Rnnt(max_streams=S)
    r.set_weights(w)
    return r, orc.Rnnt(w), w


def test_joint_enc_projection(gpu, orc):
    ud = gpu
    r, _, w = _dec(ud, orc, 1, 0.0, 2)
    rng = np.random.default_rng(2)
    x = rng.standard_normal((37, 1024)).astype(np.float32)
    xb = ud.DeviceBuffer.from_numpy(x)
    ob = ud.DeviceBuffer(37 * 640 * 4)
    r.project(37, xb, ob)
    got = ob.download((37, 640))
    ref = x.astype(np.float64) @ w["joint.enc.weight"].astype(np.float64).T + w["joint.enc.bias"]
    assert harness.rel_err(got, ref) <= 1e-5
    r.close()


@pytest.mark.parametrize("blank_bias", [2.1, -50.0, 50.0])
def test_greedy_matches_oracle_across_calls(gpu, orc, blank_bias):
    ud = gpu
    S = 5
    r, ro, _ = _dec(ud, orc, 4, blank_bias, 8)
    slots = [6, 0, 3, 1, 7]
    rng = np.random.default_rng(5)
    ost = [ro.state() for _ in range(S)]
    rows = 6
    for call, frames in enumerate(([6, 4, 6, 0, 5], [3, 6, 1, 6, 2], [6, 6, 6, 6, 6])):
        f = rng.standard_normal((S, rows, 640)).astype(np.float32)
        fb = ud.DeviceBuffer.from_numpy(f)
        got, cnt = r.greedy(slots, fb, rows, frames, cap=40)
        for b in range(S):
            ref = ro.greedy(f[b, :frames[b]], ost[b])
            assert cnt[b] == len(ref), (call, b)
            assert got[b] == ref[:40], (call, b)
        if blank_bias < 0:
            assert all(cnt[b] == 10 * frames[b] for b in range(S))
        if blank_bias > 10:
            assert all(c == 0 for c in cnt)
    # a reset slot starts over from the initial state
    r.reset(3)
    ost[2] = ro.state()
    f = rng.standard_normal((1, rows, 640)).astype(np.float32)
    got, _ = r.greedy([3], ud.DeviceBuffer.from_numpy(f), rows, [rows], cap=80)
    assert got[0] == ro.greedy(f[0], ost[2])
    r.close()


@pytest.mark.parametrize("blank_bias", [1.2, -50.0])
def test_greedy_many_streams(gpu, orc, blank_bias):
    """72 streams x 5 frames: the decoder GEMMs take several 64-row blocks (the joint's 360 rows,
    the prediction's 72) and the iterations after the first a few rows (the 16- to 48-row tiles).
    Tokens equal the oracle's over two calls, the joint.enc projection of 360 rows is within 1e-5.  (Blank bias 1.2 on these rows: about 950 tokens in the first call, 0 to 40 per
    stream, so the iterations shrink from 72 streams to a few.)"""
    ud = gpu
    S, rows = 72, 5
    r, ro, w = _dec(ud, orc, 13, blank_bias, S)
    rng = np.random.default_rng(21)
    ost = [ro.state() for _ in range(S)]
    slots = list(range(S))[::-1]
    for call in range(2):
        enc = rng.standard_normal((S * rows, 1024)).astype(np.float32)
        eb = ud.DeviceBuffer.from_numpy(enc)
        pb = ud.DeviceBuffer(S * rows * 640 * 4)
        r.project(S * rows, eb, pb)
        proj = pb.download((S * rows, 640))
        ref = enc.astype(np.float64) @ w["joint.enc.weight"].astype(np.float64).T + w["joint.enc.bias"]
        assert harness.rel_err(proj, ref) <= 1e-5, call
        frames = [rows - (b % 3 == 1) for b in range(S)] if call else [rows] * S
        got, cnt = r.greedy(slots, pb, rows, frames, cap=64)
        proj = proj.reshape(S, rows, 640)
        n_tok = 0
        for b in range(S):
            want = ro.greedy(proj[b, :frames[b]], ost[b])
            assert cnt[b] == len(want) and got[b] == want[:64], (call, b)
            n_tok += len(want)
        if blank_bias > 0:
            assert 0 < n_tok < 10 * sum(frames), n_tok      # a mix of blank and emitting frames
    r.close()


def test_calls_on_alternating_hip_streams(gpu, orc):
    """joint.enc projections and greedy calls issued on two HIP streams in turn, with no
    synchronisation by the caller: each call waits for the previous one's work (the shared split-K
    workspace), so the projections and tokens equal those of the same calls on one stream."""
    ud = gpu
    S, rows = 4, 6
    r, ro, w = _dec(ud, orc, 11, 2.1, S)
    rng = np.random.default_rng(9)
    hs = [ud.HipStream(), ud.HipStream()]
    slots = [2, 0, 3, 1]
    ost = [ro.state() for _ in range(S)]
    for call in range(6):
        enc = rng.standard_normal((S * rows, 1024)).astype(np.float32)
        eb = ud.DeviceBuffer.from_numpy(enc)
        pb = ud.DeviceBuffer(S * rows * 640 * 4)
        r.project(S * rows, eb, pb, hip_stream=hs[call % 2])
        frames = [rows, rows - 1, 3, rows] if call % 3 else [rows] * S
        got, cnt = r.greedy(slots, pb, rows, frames, cap=64, hip_stream=hs[(call + 1) % 2])
        proj = pb.download((S * rows, 640))
        ref = enc.astype(np.float64) @ w["joint.enc.weight"].astype(np.float64).T + w["joint.enc.bias"]
        assert harness.rel_err(proj, ref) <= 1e-5, call
        proj = proj.reshape(S, rows, 640)
        for b in range(S):
            assert got[b] == ro.greedy(proj[b, :frames[b]], ost[b])[:64], (call, b)
    r.close()


def test_mel_to_tokens_chain(gpu, orc):
    """Subsampling + 2-layer fp32 encoder step + joint.enc + greedy for 3 streams over 3 chunks
    (first chunk 9 mel rows, then 16 + 9 pre-encode rows with 2 frames dropped), against the
    oracle's composition of the same steps."""
    ud = gpu
    cfg = ud.EncoderConfig(layers=2, max_chunk=2, max_streams=3, dtype="f32")
    enc, model, _ = harness.make_encoder(ud, orc, cfg, seed=91)
    sw = ud.synthetic_subsampling_weights(92)
    enc.set_subsampling_weights(sw)
    r, ro, w = _dec(ud, orc, 93, 0.95, 3)   # a mix of blank frames, short runs and 10-token frames
    S = 3
    streams = [enc.new_stream() for _ in range(S)]
    st = harness.OracleState(S, cfg)
    ost = [ro.state() for _ in range(S)]
    rng = np.random.default_rng(94)
    mel = rng.standard_normal((S, 9 + 16 * 2, 128)).astype(np.float32)
    xb, ob = ud.DeviceBuffer(S * 2 * 1024 * 4), ud.DeviceBuffer(S * 2 * 1024 * 4)
    pb = ud.DeviceBuffer(S * 2 * 640 * 4)
    idx, all_got, all_ref = 0, [[] for _ in range(S)], [[] for _ in range(S)]
    for step in range(3):
        first = step == 0
        size = 9 if first else 16
        start = idx if first else idx - 9
        chunk = np.ascontiguousarray(mel[:, start:idx + size])
        drop = 0 if first else 2
        T, vt = enc.subsample(S, ud.DeviceBuffer.from_numpy(chunk), xb, drop=drop)
        enc.encode_stream_step(streams, xb, ob, valid=vt, T=T)
        r.project(S * T, ob, pb)
        got, _ = r.greedy([0, 1, 2], pb, T, [T] * S, cap=64)
        x_ref = np.stack([orc.subsample(chunk[s], chunk.shape[1], sw)[drop:] for s in range(S)])
        y_ref = orc.stream_step(model, x_ref, vt, st.k, st.v, st.c, st.len)
        p_ref = y_ref.astype(np.float64) @ w["joint.enc.weight"].astype(np.float64).T + w["joint.enc.bias"]
        assert harness.rel_err(pb.download((S, T, 640)), p_ref) <= 1e-4
        for s in range(S):
            all_got[s] += got[s]
            all_ref[s] += ro.greedy(p_ref[s].astype(np.float32), ost[s])
        idx += size
    assert all_got == all_ref
    assert sum(len(t) for t in all_ref) > 0
    r.close()
    enc.close()


def test_rnnt_error_paths(gpu):
    ud = gpu
    r = ud.Rnnt(max_streams=2)
    pb = ud.DeviceBuffer(2 * 640 * 4)
    with pytest.raises(ud.EngineError) as e:
        r.greedy([0], pb, 1, [1])
    assert e.value.status == -5                      # weights not set
    w = ud.synthetic_rnnt_weights(1)
    with pytest.raises(ud.EngineError) as e:
        r.set_weights({"joint.pred.weight": np.zeros(3, np.float32)})
    assert e.value.status == -6
    with pytest.raises(ud.EngineError) as e:
        r.set_weights({"decoder.prediction.dec_rnn.lstm.weight_ih_l2": np.zeros(4 * 640 * 640, np.float32)})
    assert e.value.status == -6                      # layer 2 of 2
    r.set_weights(w)
    with pytest.raises(ud.EngineError) as e:
        r.greedy([0, 0], pb, 1, [1, 1])
    assert e.value.status == -1                      # repeated slot
    with pytest.raises(ud.EngineError) as e:
        r.greedy([2], pb, 1, [1])
    assert e.value.status == -1                      # slot outside the pool
    with pytest.raises(ud.EngineError) as e:
        r.reset(5)
    assert e.value.status == -2
    r.close()
    with pytest.raises(ud.EngineError) as e:
        ud.Rnnt(max_streams=2, hidden=96)            # hidden not a multiple of 64 (the GEMM tiles)
    assert e.value.status == -2
