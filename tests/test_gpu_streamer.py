"""GPU parity of the batched streaming driver (ud_streamer) against the oracle's NemotronStreamer
restatement (one stream at a time, every chunk at its own unpadded size), and the reference's
live-equals-buffered property (Tests/DictatorEngineTests/StreamingEquivalenceTests.swift:22-40):
  - live input pushed in uneven pieces by several streams that start at different times, so one
    batched step mixes first chunks and later chunks; final chunks shorter than 8 frames (padded
    or dropped), between 8 frames and a full chunk, and utterances shorter than the first chunk;
  - token-exact decoding, encoder rows and joint.enc rows to the fp32 bar;
  - run_buffered over full-utterance features == live push + flush, bit for bit."""
import numpy as np
import pytest

import harness
import refimpl

pytestmark = pytest.mark.gpu

# samples per stream: 91 mel frames (final chunk of 2 frames after 9 + 5 x 16), 57 frames (exact
# chunks), 7 frames (shorter than the first chunk), 70 frames (final chunk of 13)
LENGTHS = [14400, 9000, 1000, 11111]


def _setup(ud, orc, la, S, dtype="f32", seed=300):
    cfg = ud.EncoderConfig(layers=2, max_chunk=la + 1, max_streams=S, dtype=dtype)
    enc, model, _ = harness.make_encoder(ud, orc, cfg, seed=seed)
    sw = ud.synthetic_subsampling_weights(seed + 1)
    enc.set_subsampling_weights(sw)
    rw = ud.synthetic_rnnt_weights(seed + 2, blank_bias=0.6)
    dec = ud.Rnnt(max_streams=S)
    dec.set_weights(rw)
    fb, win = refimpl.slaney_mel_fb(), refimpl.hann_symmetric()
    fe = ud.MelFrontend(fb, win)
    return enc, model, sw, rw, dec, fe, orc.MelFrontend(fb, win)


def _audio(orc, n, k):
    return harness.speechlike(n, 40 + k, scale=0.3) + orc.lcg_floats(n, 50 + k) * np.float32(0.01)


def _oracle_live(orc, model, sw, rw, ofe, la, audio, pieces, end_padding):
    o = orc.Streamer(model, sw, rw, la, fe=ofe)
    o.end_padding = end_padding
    i = 0
    while i < audio.size:
        n = min(pieces, audio.size - i)
        o.push(audio[i:i + n])
        i += n
    o.flush()
    return o


@pytest.mark.parametrize("la,end_padding", [(1, True), (1, False), (2, True)])
def test_live_streams_match_oracle(gpu, orc, la, end_padding):
    ud = gpu
    S = len(LENGTHS)
    enc, model, sw, rw, dec, fe, ofe = _setup(ud, orc, la, S)
    st = ud.Streamer(enc, dec, fe, lookahead=la, max_streams=S)
    st.end_padding = end_padding
    st.record = True
    audio = [_audio(orc, n, k) for k, n in enumerate(LENGTHS)]
    pieces = [1000, 3333, 160, 1601]
    ids = [st.open() for _ in range(S)]
    pos = [0] * S
    # stream k starts after k rounds, so early batches mix first and later chunks
    rnd = 0
    while any(pos[k] < audio[k].size for k in range(S)):
        chunk = {}
        for k in range(S):
            if rnd >= k and pos[k] < audio[k].size:
                n = min(pieces[k], audio[k].size - pos[k])
                chunk[ids[k]] = audio[k][pos[k]:pos[k] + n]
                pos[k] += n
        st.push(chunk)
        rnd += 1
    st.flush(ids)
    batches, chunks = st.stats()
    assert batches < chunks                      # streams shared steps
    total = 0
    for k in range(S):
        o = _oracle_live(orc, model, sw, rw, ofe, la, audio[k], pieces[k], end_padding)
        got_enc, got_proj = st.recorded(ids[k], "enc"), st.recorded(ids[k], "proj")
        ref_enc = np.concatenate(o.enc_rows) if o.enc_rows else np.zeros((0, 1024), np.float32)
        ref_proj = np.concatenate(o.proj_rows) if o.proj_rows else np.zeros((0, 640), np.float32)
        assert got_enc.shape == ref_enc.shape, (k, got_enc.shape, ref_enc.shape)
        if ref_enc.size:
            assert harness.rel_err(got_enc, ref_enc) <= 1e-4, k
            assert harness.rel_err(got_proj, ref_proj) <= 1e-4, k
        assert st.tokens(ids[k]) == o.tokens, k
        total += len(o.tokens)
    assert total > 0
    st.close()
    dec.close()
    enc.close()


@pytest.mark.parametrize("la", [1, 6])
def test_live_equals_buffered(gpu, orc, la):
    """testNemotronLiveEqualsBuffered: runBuffered over features(audio) vs push of 1600-sample
    pieces + flush with end padding off; here also the kept encoder rows, bit for bit."""
    ud = gpu
    enc, model, sw, rw, dec, fe, ofe = _setup(ud, orc, la, 2, seed=310)
    audio = _audio(orc, 16000 * 2 + 777, 7)
    frames = audio.size // 160 + 1
    mel = fe.features([audio])[0]
    a = ud.Streamer(enc, dec, fe, lookahead=la, max_streams=2)
    a.record = True
    sa = a.open()
    a.run_buffered({sa: (mel, frames, frames)})
    b = ud.Streamer(enc, dec, fe, lookahead=la, max_streams=2)
    b.record = True
    b.end_padding = False
    sb = b.open()
    i = 0
    after_push = []                  # (tokens so far, samples pushed so far) after each push
    while i < audio.size:
        n = min(1600, audio.size - i)
        b.push({sb: audio[i:i + n]})
        i += n
        after_push.append((len(b.tokens(sb)), i))
    b.flush([sb])
    assert a.tokens(sa) == b.tokens(sb)
    assert len(a.tokens(sa)) > 0
    # NemotronStreamer's emissions: one per token of the live stream, in order, with the samples
    # pushed when its chunk ran (flush pushes none) and that step's wall seconds; wallTimes: one
    # per chunk, for live and buffered input; buffered input records no emissions
    em = b.emissions(sb)
    assert [e[0] for e in em] == b.tokens(sb)
    k = 0
    for cnt, pushed in after_push:
        while k < cnt:
            assert em[k][1] == pushed, k
            k += 1
    assert all(e[1] == audio.size for e in em[k:]) and all(e[2] > 0 for e in em)
    assert len(b.step_times(sb)) == b.stats()[1] and min(b.step_times(sb)) > 0
    assert a.emissions(sa) == [] and len(a.step_times(sa)) == a.stats()[1] > 1
    ea, eb = a.recorded(sa, "enc"), b.recorded(sb, "enc")
    assert ea.shape == eb.shape and np.array_equal(ea.view(np.uint32), eb.view(np.uint32))
    # and the buffered run equals the oracle's runBuffered over the same features
    o = orc.Streamer(model, sw, rw, la)
    o.run_buffered(mel, frames, frames)
    assert a.tokens(sa) == o.tokens
    assert harness.rel_err(ea, np.concatenate(o.enc_rows)) <= 1e-4
    # NemotronStreamer.text: the transcript through a SentencePiece vocabulary (a synthetic one for
    # the 1,025-id decoder: ordinary, byte-fallback and special pieces) equals the oracle's decode
    pieces = _synthetic_vocab(1025)
    tok = ud.Tokenizer.from_bytes("".join("%s\t%d\n" % (pc, -k) for k, pc in enumerate(pieces)).encode("utf-8"))
    assert a.text(sa, tok) == orc.sp_decode(pieces, a.tokens(sa)) == b.text(sb, tok)
    tok.close()
    a.close()
    b.close()
    dec.close()
    enc.close()


def _synthetic_vocab(n):
    """n SentencePiece-style pieces: specials, the 256 byte-fallback pieces, then word pieces."""
    rng = np.random.default_rng(5)
    words = ["".join(rng.choice(list("abcdefghé日▁"), size=int(rng.integers(1, 6)))) for _ in range(n)]
    pieces = ["<unk>", "<s>", "</s>"] + ["<0x%02X>" % b for b in range(256)] + words
    return pieces[:n]


def test_buffered_valid_frames_and_batching(gpu, orc):
    """run_buffered for 3 fresh streams at once with valid_frames below frames (NeMo's processed
    length): the masked tail rows of non-final chunks, against the oracle stream by stream."""
    ud = gpu
    enc, model, sw, rw, dec, fe, ofe = _setup(ud, orc, 1, 3, seed=320)
    rng = np.random.default_rng(321)
    runs, refs = {}, []
    st = ud.Streamer(enc, dec, None, lookahead=1, max_streams=3)
    st.record = True
    for k, (frames, valid) in enumerate(((75, 75), (60, 41), (30, 9))):
        mel = (rng.standard_normal((frames, 128)) * 2 - 6).astype(np.float32)
        sid = st.open()
        runs[sid] = (mel, frames, valid)
        o = orc.Streamer(model, sw, rw, 1)
        o.run_buffered(mel, frames, valid)
        refs.append((sid, o))
    st.run_buffered(runs)
    for sid, o in refs:
        got = st.recorded(sid, "enc")
        ref = np.concatenate(o.enc_rows)
        assert got.shape == ref.shape
        assert harness.rel_err(got, ref) <= 1e-4
        assert st.tokens(sid) == o.tokens
    st.close()
    dec.close()
    enc.close()


def test_bf16_live_stream(gpu, orc):
    """A bf16 encoder behind the streamer (front-end GEMMs in f16): kept encoder rows to the bf16
    bar against the oracle with the reference's f16 front-end policy (conv.* fp32, out f16)."""
    ud = gpu
    la = 1
    cfg = ud.EncoderConfig(layers=2, max_chunk=la + 1, max_streams=2, dtype="bf16")
    enc, model, _ = harness.make_encoder(ud, orc, cfg, seed=330)
    sw = ud.synthetic_subsampling_weights(331)
    enc.set_subsampling_weights(sw)
    osw = harness.oracle_sub_weights(sw, True)
    rw = ud.synthetic_rnnt_weights(332, blank_bias=0.6)
    dec = ud.Rnnt(max_streams=2)
    dec.set_weights(rw)
    fb, win = refimpl.slaney_mel_fb(), refimpl.hann_symmetric()
    st = ud.Streamer(enc, dec, ud.MelFrontend(fb, win), lookahead=la, max_streams=2)
    st.record = True
    sid = st.open()
    audio = _audio(orc, 8000 + 555, 9)
    for i in range(0, audio.size, 2560):
        st.push({sid: audio[i:i + 2560]})
    st.flush([sid])
    o = _oracle_live(orc, model, osw, rw, orc.MelFrontend(fb, win), la, audio, 2560, True)
    harness.assert_bf16_close(st.recorded(sid, "enc"), np.concatenate(o.enc_rows), "bf16 stream")
    st.close()
    dec.close()
    enc.close()


def test_streamer_error_paths(gpu, orc):
    ud = gpu
    enc, model, sw, rw, dec, fe, ofe = _setup(ud, orc, 1, 2, seed=340)
    with pytest.raises(ud.EngineError) as e:
        ud.Streamer(enc, dec, fe, lookahead=2, max_streams=2)       # needs max_chunk >= 3
    assert e.value.status == -2
    with pytest.raises(ud.EngineError) as e:
        ud.Streamer(enc, dec, fe, lookahead=1, max_streams=3)       # more than the encoder's pool
    assert e.value.status == -2
    st = ud.Streamer(enc, dec, fe, lookahead=1, max_streams=2)
    with pytest.raises(ud.EngineError) as e:
        st.push({0: np.zeros(10, np.float32)})                       # not open
    assert e.value.status == -1
    a, b = st.open(), st.open()
    with pytest.raises(ud.EngineError) as e:
        st.open()
    assert e.value.status == -7
    st.push({a: np.zeros(5000, np.float32)})
    with pytest.raises(ud.EngineError) as e:
        st.run_buffered({a: (np.zeros((20, 128), np.float32), 20, 20)})   # not fresh
    assert e.value.status == -5
    st.flush([a])
    with pytest.raises(ud.EngineError) as e:
        st.push({a: np.zeros(10, np.float32)})                       # flushed
    assert e.value.status == -5
    st.close_stream(a)
    assert st.open() == a
    st.close()                                                       # frees its encoder streams
    nomel = ud.Streamer(enc, dec, None, lookahead=1, max_streams=1)
    c = nomel.open()
    with pytest.raises(ud.EngineError) as e:
        nomel.push({c: np.zeros(10, np.float32)})                    # buffered-only streamer
    assert e.value.status == -5
    nomel.close()
    dec.close()
    enc.close()
