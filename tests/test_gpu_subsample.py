"""GPU parity of the subsampling front-end (ud_encoder_subsample) against the oracle's
encodeSubsampling, and of the mel-in streaming step (front-end + ud_encoder_step) against the
oracle's subsample + stream_step over NeMo's pre-encode-cache chunk schedule."""
import numpy as np
import pytest

import harness

pytestmark = pytest.mark.gpu

def _sub_weights(ud, seed, half):
    """(encoder weights, oracle weights): the oracle follows the reference's f16 policy -- conv.*
    fp32, out.weight f16 (harness.oracle_sub_weights) -- so the library's half conv.3 / conv.6 and
    its half activations both count in the measured error."""
    w = ud.synthetic_subsampling_weights(seed)
    return w, harness.oracle_sub_weights(w, half)


def _check(got, ref, bf16, what):
    if bf16:
        harness.assert_bf16_close(got, ref, what)
    else:
        assert harness.rel_err(got, ref) <= 1e-4, what


def _check_front(got, ref, half, what):
    """Front-end output alone.  fp32: <= 1e-4 relative.  Half operands (activations rounded to
    11-bit mantissas, fp32 accumulation): max abs error <= 2e-3 x max(1, max |ref|), cosine >= 0.99999."""
    if not half:
        assert harness.rel_err(got, ref) <= 1e-4, what
        return
    err = float(np.abs(got - ref).max())
    cos = harness.cosine(got, ref)
    harness.MARGINS.append((harness._test_id(), what, "bf16", err, cos))
    assert err <= 2e-3 * max(1.0, float(np.abs(ref).max())) and cos >= 0.99999, "%s: err %.3g cos %.7f" % (what, err, cos)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("rows,drop", [(25, 2), (9, 0), (121, 2), (17, 1)])
def test_subsample_matches_oracle(gpu, orc, dtype, rows, drop):
    ud = gpu
    bf16 = dtype == "bf16"
    cfg = ud.EncoderConfig(layers=1, max_chunk=14, max_streams=6, dtype=dtype)
    enc = ud.Encoder(cfg)
    w, ow = _sub_weights(ud, 11, bf16)
    enc.set_subsampling_weights(w)
    n = 6
    rng = np.random.default_rng(rows * 10 + drop)
    mel = rng.standard_normal((n, rows, 128)).astype(np.float32)
    valid = np.array([rows, rows - 1, rows // 2, 1, 0, rows - 8], np.int32)
    T3 = orc.sub_next_len(orc.sub_next_len(orc.sub_next_len(rows)))
    T = T3 - drop
    mbuf = ud.DeviceBuffer(mel.nbytes)
    mbuf.upload(mel)
    obuf = ud.DeviceBuffer(n * T * 1024 * 4)
    gotT, vt = enc.subsample(n, mbuf, obuf, valid_mel=valid, drop=drop)
    assert gotT == T
    got = obuf.download((n, T, 1024))
    for s in range(n):
        ref = orc.subsample(mel[s], int(valid[s]), ow)[drop:]
        _check_front(got[s], ref, bf16, "stream %d (valid %d)" % (s, valid[s]))
        v3 = orc.sub_next_len(orc.sub_next_len(orc.sub_next_len(max(int(valid[s]), 0))))
        assert vt[s] == min(max(v3 - drop, 0), T)
    enc.close()


def test_subsample_64_streams_chunk2_shape(gpu, orc):
    """The 64-stream front-end: 64 streams x 25 mel rows (16 new + 9 pre-encode cache) -> 2 frames; the
    conv.3 GEMM has 64 x 7 x 33 = 14,784 rows (LDS-staged kernel)."""
    ud = gpu
    cfg = ud.EncoderConfig(layers=1, max_chunk=2, max_streams=64, dtype="bf16")
    enc = ud.Encoder(cfg)
    w, ow = _sub_weights(ud, 12, True)
    enc.set_subsampling_weights(w)
    n, rows = 64, 25
    rng = np.random.default_rng(9)
    mel = rng.standard_normal((n, rows, 128)).astype(np.float32)
    valid = np.where(np.arange(n) % 7 == 3, 19, rows).astype(np.int32)
    mbuf = ud.DeviceBuffer(mel.nbytes)
    mbuf.upload(mel)
    obuf = ud.DeviceBuffer(n * 2 * 1024 * 4)
    T, _ = enc.subsample(n, mbuf, obuf, valid_mel=valid, drop=2)
    assert T == 2
    got = obuf.download((n, 2, 1024))
    ref = np.stack([orc.subsample(mel[s], int(valid[s]), ow)[2:] for s in range(n)])
    _check_front(got, ref, True, "64 streams")
    enc.close()


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_mel_in_streaming_steps(gpu, orc, dtype):
    """Front-end + 2-layer step over NeMo's chunk schedule with lookahead 1 (first chunk 9 mel rows,
    then 16 new rows + 9 pre-encode cache rows with 2 frames dropped), 4 streams, 3 steps; the last
    step has a short final chunk on two streams."""
    ud = gpu
    bf16 = dtype == "bf16"
    cfg = ud.EncoderConfig(layers=2, max_chunk=2, max_streams=4, dtype=dtype)
    enc, model, _ = harness.make_encoder(ud, orc, cfg, seed=81)
    w, ow = _sub_weights(ud, 13, bf16)
    enc.set_subsampling_weights(w)
    S = 4
    streams = [enc.new_stream() for _ in range(S)]
    st = harness.OracleState(S, cfg)
    rng = np.random.default_rng(17)
    total = 9 + 16 * 2
    mel = rng.standard_normal((S, total, 128)).astype(np.float32)
    xbuf = ud.DeviceBuffer(S * 2 * 1024 * 4)
    obuf = ud.DeviceBuffer(S * 2 * 1024 * 4)
    idx = 0
    for step in range(3):
        first = step == 0
        size = 9 if first else 16
        start = idx if first else idx - 9
        rows = size + (idx - start)
        chunk = np.ascontiguousarray(mel[:, start:start + rows])
        valid = np.full(S, rows, np.int32)
        if step == 2:
            valid[1], valid[3] = rows - 5, rows - 12
        mbuf = ud.DeviceBuffer(chunk.nbytes)
        mbuf.upload(chunk)
        drop = 0 if first else 2
        T, vt = enc.subsample(S, mbuf, xbuf, valid_mel=valid, drop=drop)
        assert T == 2
        enc.encode_stream_step(streams, xbuf, obuf, valid=vt, T=T)
        got = obuf.download((S, T, 1024))
        x_ref = np.stack([orc.subsample(chunk[s], int(valid[s]), ow)[drop:] for s in range(S)])
        v_ref = np.array([min(max(orc.sub_next_len(orc.sub_next_len(orc.sub_next_len(int(valid[s])))) - drop, 0), T)
                          for s in range(S)], np.int32)
        np.testing.assert_array_equal(vt, v_ref)
        ref = orc.stream_step(model, x_ref, v_ref, st.k, st.v, st.c, st.len)
        _check(got, ref, bf16, "step %d" % step)
        idx += size
    enc.close()


def test_subsample_error_paths(gpu):
    ud = gpu
    cfg = ud.EncoderConfig(layers=1, max_chunk=2, max_streams=2, dtype="bf16")
    enc = ud.Encoder(cfg)
    mbuf = ud.DeviceBuffer(2 * 25 * 128 * 4)
    obuf = ud.DeviceBuffer(2 * 2 * 1024 * 4)
    with pytest.raises(ud.EngineError) as e:
        enc.subsample(2, mbuf, obuf, drop=2, mel_rows=25)
    assert e.value.status == -5                      # weights not set
    enc.set_subsampling_weights(ud.synthetic_subsampling_weights(1))
    with pytest.raises(ud.EngineError) as e:
        enc.set_weight("encoder.pre_encode.out.weight", np.zeros(7, np.float32))
    assert e.value.status == -6
    with pytest.raises(ud.EngineError) as e:
        enc.subsample(2, mbuf, obuf, drop=0, mel_rows=25)  # 4 frames > max_chunk 2
    assert e.value.status == -2
    with pytest.raises(ud.EngineError) as e:
        enc.subsample(3, mbuf, obuf, drop=2, mel_rows=25)  # n > max_streams
    assert e.value.status == -2
    with pytest.raises(ud.EngineError) as e:
        # 33 rows with drop 3 leave 2 frames, but the stages would need 9 conv rows where the
        # workspace holds 8 * max_chunk + 9 = 25 mel rows' worth: refused before any launch
        enc.subsample(2, mbuf, obuf, drop=3, mel_rows=33)
    assert e.value.status == -2 and "workspace" in str(e.value)
    T, vt = enc.subsample(2, mbuf, obuf, drop=2, mel_rows=25)
    assert T == 2 and list(vt) == [2, 2]
    ud.synchronize()
    enc.close()


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_subsample_nonfinite_masked_rows(gpu, dtype):
    """NaN and Inf in mel rows past a chunk's valid length never reach the output: every frame
    equals (bit for bit) the frame computed with those rows zeroed, and all frames are finite."""
    ud = gpu
    cfg = ud.EncoderConfig(layers=1, max_chunk=14, max_streams=3, dtype=dtype)
    enc = ud.Encoder(cfg)
    enc.set_subsampling_weights(ud.synthetic_subsampling_weights(14))
    n, rows, drop = 3, 121, 2
    valid = np.array([rows - 7, 60, 33], np.int32)
    rng = np.random.default_rng(5)
    clean = rng.standard_normal((n, rows, 128)).astype(np.float32)
    for s in range(n):
        clean[s, valid[s]:] = 0.0
    dirty = clean.copy()
    for s in range(n):
        dirty[s, valid[s]:] = np.where(rng.random((rows - valid[s], 128)) < 0.5, np.nan, np.inf)
    outs = []
    for mel in (clean, dirty):
        mbuf = ud.DeviceBuffer.from_numpy(mel)
        obuf = ud.DeviceBuffer(n * 14 * 1024 * 4)
        T, _ = enc.subsample(n, mbuf, obuf, valid_mel=valid, drop=drop)
        outs.append(obuf.download((n, T, 1024)))
    assert np.isfinite(outs[1]).all()
    np.testing.assert_array_equal(outs[1], outs[0])
    enc.close()
