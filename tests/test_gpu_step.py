"""GPU parity of the whole cache-aware encoder step (ud_encoder_step) against the oracle's
encodeStreamStep, over several consecutive steps: fresh and full caches, valid < T, fp32 and bf16,
the 64-stream chunk-2 shape and the chunk-14 shape, graph replay vs eager launches, error paths."""
import os

import numpy as np
import pytest

import harness

pytestmark = pytest.mark.gpu


def _run_steps(ud, orc, cfg, S, T, n_steps, seed, seed_caches, valid_plan=None, enc_model=None, make_x=None,
               T_plan=None, store_limit=0.0, cache_blocks=None):
    """n_steps steps of S streams (T frames each, or T_plan(step) frames) through the encoder and
    the oracle; returns (encoder, streams, oracle state, [(got, ref) per step])."""
    enc, model, _ = enc_model or harness.make_encoder(ud, orc, cfg, seed=seed)
    rng = np.random.default_rng(seed + 1)
    streams = [enc.new_stream() for _ in range(S)]
    st = harness.OracleState(S, cfg)
    if seed_caches:
        st.seed_random(rng, cfg.left_context, blocks=cache_blocks)
        st.import_into(streams, ud, harness.is16(cfg))
    D = cfg.d_model
    T0 = T
    xbuf = ud.DeviceBuffer(S * cfg.max_chunk * D * 4)
    obuf = ud.DeviceBuffer(S * cfg.max_chunk * D * 4)
    results = []
    for step in range(n_steps):
        T = T_plan(step) if T_plan else T0
        x = (make_x or (lambda r, shape: r.standard_normal(shape)))(rng, (S, T, D)).astype(np.float32)
        valid = np.full(S, T, np.int32) if valid_plan is None else np.asarray(valid_plan(step, S, T), np.int32)
        xbuf.upload(x)
        enc.encode_stream_step(streams, xbuf, obuf, valid=valid, T=T)
        got = obuf.download((S, T, D))
        with orc.store_limit(store_limit):
            ref = orc.stream_step(model, x, valid, st.k, st.v, st.c, st.len)
        results.append((got, ref))
        for s, stream in enumerate(streams):
            assert stream.cache_len == st.len[s]
    return enc, streams, st, results


def test_step_fp32_two_layers_fresh_streams(gpu, orc):
    cfg = gpu.EncoderConfig(layers=2, max_chunk=2, max_streams=4, dtype="f32")
    plan = lambda step, S, T: [T, 1 if step == 2 else T, 0 if step == 3 else T]
    enc, streams, st, res = _run_steps(gpu, orc, cfg, S=3, T=2, n_steps=5, seed=21, seed_caches=False,
                                       valid_plan=plan)
    for i, (got, ref) in enumerate(res):
        assert harness.rel_err(got, ref) <= 1e-4, i
    # the caches after the steps match the oracle's (computed values, fp32 tolerance)
    for s, stream in enumerate(streams):
        for l in range(cfg.layers):
            k, v, c, n = stream.export_cache(l)
            assert n == st.len[s]
            assert harness.rel_err(k, st.k[s, l]) <= 1e-4
            assert harness.rel_err(v, st.v[s, l]) <= 1e-4
            assert harness.rel_err(c, st.c[s, l]) <= 1e-4
    enc.close()


def test_step_fp32_full_cache_chunk5(gpu, orc):
    cfg = gpu.EncoderConfig(layers=2, max_chunk=5, max_streams=2, dtype="f32")
    enc, _, _, res = _run_steps(gpu, orc, cfg, S=2, T=5, n_steps=3, seed=31, seed_caches=True)
    for i, (got, ref) in enumerate(res):
        assert harness.rel_err(got, ref) <= 1e-4, i
    enc.close()


def test_step_bf16_64_streams_chunk2(gpu, orc):
    """64 streams x 2 frames (L=70, seeded full caches) over 4 layers."""
    cfg = gpu.EncoderConfig(layers=4, max_chunk=2, max_streams=64, dtype="bf16")
    plan = lambda step, S, T: [T - (s % 3 == 1 and step == 1) for s in range(S)]
    enc, _, _, res = _run_steps(gpu, orc, cfg, S=64, T=2, n_steps=3, seed=41, seed_caches=True, valid_plan=plan)
    for i, (got, ref) in enumerate(res):
        harness.assert_bf16_close(got, ref, "step %d" % i)
    enc.close()


def test_step_bf16_24_layers(gpu, orc):
    """Full depth: bf16 error accumulated over 24 layers stays within 2e-2 abs / cosine 0.9995."""
    cfg = gpu.EncoderConfig(layers=24, max_chunk=2, max_streams=4, dtype="bf16")
    enc, _, _, res = _run_steps(gpu, orc, cfg, S=4, T=2, n_steps=2, seed=51, seed_caches=True)
    for i, (got, ref) in enumerate(res):
        harness.assert_bf16_close(got, ref, "step %d" % i)
    enc.close()


def test_step_bf16_64_streams_2_frames_full(gpu, orc):
    """64 streams x 2 frames exactly, 24 layers, seeded full caches, two steps (the second
    with a short final chunk on some streams), against the oracle's fp32 step."""
    cfg = gpu.EncoderConfig(layers=24, max_chunk=2, max_streams=64, dtype="bf16")
    plan = lambda step, S, T: [T - (s % 5 == 2 and step == 1) for s in range(S)]
    enc, _, _, res = _run_steps(gpu, orc, cfg, S=64, T=2, n_steps=2, seed=43, seed_caches=True, valid_plan=plan)
    for i, (got, ref) in enumerate(res):
        harness.assert_bf16_close(got, ref, "step %d" % i)
    enc.close()


def test_step_bf16_offset_rows(gpu, orc):
    """Rows far from zero mean (offsets 20-60, scales 0.5-4 per row): the residual stream keeps the
    offsets, so every LayerNorm of the step normalises rows whose mean is large against their
    spread (the two-pass variance).  5 streams x 2 frames = 10 rows: the 16-row tiles of the
    projections have padding rows too."""
    cfg = gpu.EncoderConfig(layers=2, max_chunk=2, max_streams=5, dtype="bf16")

    def make_x(r, shape):
        off = r.uniform(20.0, 60.0, shape[:2] + (1,))
        scale = r.uniform(0.5, 4.0, shape[:2] + (1,))
        return off + scale * r.standard_normal(shape)
    enc, _, _, res = _run_steps(gpu, orc, cfg, S=5, T=2, n_steps=2, seed=53, seed_caches=True, make_x=make_x)
    for i, (got, ref) in enumerate(res):
        harness.assert_bf16_close(got, ref, "step %d" % i)
    enc.close()


def test_step_bf16_mid_rows(gpu, orc):
    """48 streams x 6 frames = 288 rows: between the 128-row tiles of the streaming shapes and the
    2,048 rows where the LDS-staged projection kernel starts (128-row register tiles, split-K 4)."""
    cfg = gpu.EncoderConfig(layers=2, max_chunk=6, max_streams=48, dtype="bf16")
    plan = lambda step, S, T: [(T, 4, 0, T)[s % 4] if step == 1 else T for s in range(S)]
    enc, _, _, res = _run_steps(gpu, orc, cfg, S=48, T=6, n_steps=2, seed=47, seed_caches=True, valid_plan=plan)
    for i, (got, ref) in enumerate(res):
        harness.assert_bf16_close(got, ref, "step %d" % i)
    enc.close()


def test_step_bf16_chunk14(gpu, orc):
    """The 14-frame chunk (84 keys) on a few streams."""
    cfg = gpu.EncoderConfig(layers=2, max_chunk=14, max_streams=8, dtype="bf16")
    plan = lambda step, S, T: [T, 9, T, 0, T, T, 3, T][:S]
    enc, _, _, res = _run_steps(gpu, orc, cfg, S=8, T=14, n_steps=3, seed=61, seed_caches=True, valid_plan=plan)
    for i, (got, ref) in enumerate(res):
        harness.assert_bf16_close(got, ref, "step %d" % i)
    enc.close()


def test_step_bf16_chunk14_many_rows(gpu, orc):
    """250 streams x 14 frames = 3500 rows: the LDS-staged projection kernel at every tile it picks
    for the 14-frame chunk's shapes (224 x 256, 224 x 192, 224 x 128 with 2 K splits, 128 x 128),
    with a partial last 224-row tile (3500 = 15 x 224 + 140)."""
    cfg = gpu.EncoderConfig(layers=2, max_chunk=14, max_streams=250, dtype="bf16")
    plan = lambda step, S, T: [(T, 9, 0, 3, T)[s % 5] if step == 1 else T for s in range(S)]
    enc, _, _, res = _run_steps(gpu, orc, cfg, S=250, T=14, n_steps=2, seed=63, seed_caches=True, valid_plan=plan)
    for i, (got, ref) in enumerate(res):
        harness.assert_bf16_close(got, ref, "step %d" % i)
    enc.close()


def test_step_bf16_chunk14_24_layers(gpu, orc):
    """The 14-frame chunk at full depth: 32 streams x 14 frames x 24 layers from seeded full caches,
    two steps (ragged valid counts on the second), against the oracle's fp32 step -- the bf16
    error accumulated over 24 layers at 84 keys."""
    cfg = gpu.EncoderConfig(layers=24, max_chunk=14, max_streams=32, dtype="bf16")
    plan = lambda step, S, T: [(T, 11, T, 2)[s % 4] if step == 1 else T for s in range(S)]
    enc, _, _, res = _run_steps(gpu, orc, cfg, S=32, T=14, n_steps=2, seed=65, seed_caches=True, valid_plan=plan)
    for i, (got, ref) in enumerate(res):
        harness.assert_bf16_close(got, ref, "step %d" % i)
    enc.close()


def test_step_bf16_chunk14_24_layers_lds_tiles(gpu, orc):
    """24 layers at 148 streams x 14 frames = 2,072 rows: the LDS-staged projection kernel (the
    256-stream x 14-frame GEMM path) at full depth, two steps from fresh streams."""
    cfg = gpu.EncoderConfig(layers=24, max_chunk=14, max_streams=148, dtype="bf16")
    enc, _, _, res = _run_steps(gpu, orc, cfg, S=148, T=14, n_steps=2, seed=67, seed_caches=False)
    for i, (got, ref) in enumerate(res):
        harness.assert_bf16_close(got, ref, "step %d" % i)
    enc.close()


def test_step_bf16_256_streams_14_frames_full(gpu, orc):
    """256 streams x 14 frames (84 keys) exactly, 24 layers, seeded full caches, two steps
    (ragged valid counts on the second), against the oracle's fp32 step -- the workload the
    benchmark's chunk-14 line times.  (The 24 x 256 cached K/V windows are dealt from 96 distinct
    N(0,1) draws to keep the host-side set-up short.)"""
    cfg = gpu.EncoderConfig(layers=24, max_chunk=14, max_streams=256, dtype="bf16")
    plan = lambda step, S, T: [(T, 11, T, 0, 6, T, 1)[s % 7] if step == 1 else T for s in range(S)]
    enc, _, _, res = _run_steps(gpu, orc, cfg, S=256, T=14, n_steps=2, seed=69, seed_caches=True, valid_plan=plan,
                                cache_blocks=96)
    for i, (got, ref) in enumerate(res):
        harness.assert_bf16_close(got, ref, "step %d" % i)
    enc.close()


def test_step_bf16_1024_streams_chunk2(gpu, orc):
    """The streaming chunk (2 frames, 72 keys) at 1,024 streams = 2,048 rows: the projections move
    to the LDS-staged kernel, whose q/k/v epilogue then writes the K/V ring rows of 2-frame chunks
    (the 14-frame tests cover its other ring shape), and the wave attention kernel runs 8,192
    workgroups.  Two layers, seeded full caches, two steps with ragged valid counts on the second."""
    cfg = gpu.EncoderConfig(layers=2, max_chunk=2, max_streams=1024, dtype="bf16")
    plan = lambda step, S, T: [(T, 1, 0, T, T)[s % 5] if step == 1 else T for s in range(S)]
    enc, _, _, res = _run_steps(gpu, orc, cfg, S=1024, T=2, n_steps=2, seed=71, seed_caches=True, valid_plan=plan,
                                cache_blocks=64)
    for i, (got, ref) in enumerate(res):
        harness.assert_bf16_close(got, ref, "step %d" % i)
    enc.close()


def test_step_bf16_ring_longer_than_window(gpu, orc):
    """An encoder sized for 14-frame chunks stepping shorter chunks: the K/V rings hold
    L + max_chunk = 84 rows while a 5- or 7-frame step's window is 75 or 77 keys, so the chunk
    attention kernel reads ring rows outside the window and must mask them (and its key-band
    index clamps).  Eight steps of 5 and 7 frames wrap the 84-row rings several times; some
    streams have valid < T."""
    cfg = gpu.EncoderConfig(layers=2, max_chunk=14, max_streams=6, dtype="bf16")
    Ts = (5, 7, 7, 5, 7, 5, 5, 7)
    plan = lambda step, S, T: [(T, T - 2, 0, T, 1, T)[s] if step % 3 == 1 else T for s in range(S)]
    enc, _, _, res = _run_steps(gpu, orc, cfg, S=6, T=7, n_steps=len(Ts), seed=73, seed_caches=True,
                                valid_plan=plan, T_plan=lambda step: Ts[step])
    for i, (got, ref) in enumerate(res):
        harness.assert_bf16_close(got, ref, "step %d (T = %d)" % (i, Ts[i]))
    enc.close()


@pytest.mark.parametrize("S,T,layers", [(64, 2, 24), (32, 14, 24)])
def test_step_f16_weights(gpu, orc, S, T, layers):
    """The f16-weight encoder (UD_F16): linear weights rounded fp32 -> half directly, as
    WeightConverter.convert(.f16) writes the reference's f16 checkpoint (Core/Convert.swift:76-112),
    against the oracle given the same f16-rounded weights, at 64 streams x 2 frames and at the 14-frame chunk,
    24 layers, seeded full caches, two steps."""
    cfg = gpu.EncoderConfig(layers=layers, max_chunk=T, max_streams=S, dtype="f16")
    plan = lambda step, S_, T_: [(T_, T_ - 1, T_, 0)[s % 4] if step == 1 else T_ for s in range(S_)]
    enc, _, _, res = _run_steps(gpu, orc, cfg, S=S, T=T, n_steps=2, seed=75 + T, seed_caches=True, valid_plan=plan)
    for i, (got, ref) in enumerate(res):
        harness.assert_bf16_close(got, ref, "step %d" % i)
    enc.close()


def test_step_f16_weights_differ_from_bf16(gpu, orc):
    """The two 16-bit modes hold different weights: the same seeded model stepped by a UD_F16 and a
    UD_BF16 encoder gives different outputs, each within the bar of the oracle given its own
    rounding and, on average, closer to its own oracle than to the other's (f16 rounding keeps 3
    more bits)."""
    outs = {}
    for dt in ("f16", "bf16"):
        cfg = gpu.EncoderConfig(layers=2, max_chunk=2, max_streams=4, dtype=dt)
        enc, _, _, res = _run_steps(gpu, orc, cfg, S=4, T=2, n_steps=1, seed=77, seed_caches=True)
        got, ref = res[0]
        outs[dt] = (got, ref)
        harness.assert_bf16_close(got, ref, dt)
        enc.close()
    (g16, r16), (gbf, rbf) = outs["f16"], outs["bf16"]
    assert np.abs(g16 - gbf).max() > 0                  # different weights
    assert np.abs(g16 - r16).mean() < np.abs(g16 - rbf).mean()


def test_step_half_range_saturates(gpu, orc):
    """A 16-bit encoder's activations beyond half's range: feed_forward1.linear1 of layer 0 scaled by
    2e5 puts about a third of the FF hidden past 65504.  The library's 16-bit stores saturate at
    +-65504 (NaN kept), so the output stays finite and matches the oracle run with the same
    storage-range model (oracle.store_limit(65504)); the unclamped fp32 oracle differs from it by
    far more than the bar, so the clamp is what the comparison checks."""
    ud = gpu
    cfg = ud.EncoderConfig(layers=2, max_chunk=2, max_streams=4, dtype="bf16")
    scale = np.float32(2e5)

    def edit(l, w):
        if l == 0:
            w["feed_forward1.linear1.weight"] = w["feed_forward1.linear1.weight"] * scale
    enc_model = harness.make_encoder(ud, orc, cfg, seed=79, edit=edit)
    # the same state through the unclamped oracle, for the sensitivity check
    _, model, _ = enc_model
    rng = np.random.default_rng(5)
    x = rng.standard_normal((4, 2, 1024)).astype(np.float32)
    st = harness.OracleState(4, cfg)
    st.seed_random(np.random.default_rng(80), cfg.left_context)
    h = orc.layer_norm(x.reshape(8, 1024), model.layers[0][0], model.layers[0][1])
    pre = orc.gemm_nt(h, model.layers[0][2])
    assert (np.abs(pre) > 65504).mean() > 0.2           # the hidden does leave half's range
    enc, _, _, res = _run_steps(ud, orc, cfg, S=4, T=2, n_steps=2, seed=79, seed_caches=True, enc_model=enc_model,
                                store_limit=65504.0)
    for i, (got, ref) in enumerate(res):
        assert np.isfinite(got).all(), "step %d: non-finite output" % i
        harness.assert_bf16_close(got, ref, "step %d" % i)
    free = orc.stream_step(model, x, np.full(4, 2, np.int32), st.k, st.v, st.c, st.len)
    with orc.store_limit(65504.0):
        st2 = harness.OracleState(4, cfg)
        st2.seed_random(np.random.default_rng(80), cfg.left_context)
        clamped = orc.stream_step(model, x, np.full(4, 2, np.int32), st2.k, st2.v, st2.c, st2.len)
    assert np.abs(free - clamped).max() > 0.1
    enc.close()


def test_alternating_hip_streams_and_graph_eviction(gpu, orc):
    """Nine distinct (n, T) steps issued back to back, without host waits, on two HIP streams in
    turn: more step shapes than the encoder's graph cache holds (8), so the ninth evicts a graph
    whose last launch was on the other stream and may still be running.  The encoder orders its
    calls across streams and waits for its own work before destroying a graph; the outputs are
    bit-identical to the same steps launched eagerly and synchronously."""
    ud = gpu
    shapes = [(12, 2), (8, 3), (4, 6), (12, 1), (6, 5), (10, 4), (3, 6), (12, 6), (5, 2)]
    rng = np.random.default_rng(17)
    xs = [rng.standard_normal((n, T, 1024)).astype(np.float32) for n, T in shapes]
    outs = []
    for graphs in ("1", "0"):
        os.environ["UD_GRAPHS"] = graphs
        try:
            cfg = ud.EncoderConfig(layers=2, max_chunk=6, max_streams=12, dtype="bf16")
            enc, _, _ = harness.make_encoder(ud, orc, cfg, seed=81)
        finally:
            os.environ.pop("UD_GRAPHS", None)
        streams = [enc.new_stream() for _ in range(12)]
        xb = [ud.DeviceBuffer.from_numpy(x) for x in xs]
        ob = [ud.DeviceBuffer(x.nbytes) for x in xs]
        hs = [ud.HipStream(), ud.HipStream()]
        for i, (n, T) in enumerate(shapes):
            enc.encode_stream_step(streams[:n], xb[i], ob[i], T=T, hip_stream=hs[i % 2] if graphs == "1" else None)
            if graphs == "0":
                ud.synchronize()
        for h in hs:
            h.synchronize()
        outs.append([o.download(x.shape) for o, x in zip(ob, xs)])
        enc.close()
    for i, (a, b) in enumerate(zip(*outs)):
        np.testing.assert_array_equal(a, b, err_msg="step %d %s" % (i, shapes[i]))


def test_graph_replay_matches_eager(gpu, orc):
    """The captured hipGraph replay gives bit-identical results to eager launches (the step is
    deterministic: split-K partials are reduced in a fixed order)."""
    outs = []
    for graphs in ("1", "0"):
        os.environ["UD_GRAPHS"] = graphs
        try:
            cfg = gpu.EncoderConfig(layers=2, max_chunk=2, max_streams=8, dtype="bf16")
            enc, _, _, res = _run_steps(gpu, orc, cfg, S=8, T=2, n_steps=3, seed=71, seed_caches=True)
            outs.append([g for g, _ in res])
            enc.close()
        finally:
            os.environ.pop("UD_GRAPHS", None)
    for a, b in zip(*outs):
        np.testing.assert_array_equal(a, b)


def test_error_paths(gpu, orc):
    ud = gpu
    with pytest.raises(ud.EngineError) as e:         # step rows past the 32-bit indexing bound
        ud.Encoder(ud.EncoderConfig(layers=1, max_chunk=16, max_streams=65537, dtype="bf16"))
    assert e.value.status == -2
    cfg = ud.EncoderConfig(layers=1, max_chunk=2, max_streams=2, dtype="bf16")
    enc = ud.Encoder(cfg)
    s0 = enc.new_stream()
    x = ud.DeviceBuffer(2 * 1024 * 4)
    o = ud.DeviceBuffer(2 * 1024 * 4)
    with pytest.raises(ud.EngineError) as e:
        enc.encode_stream_step([s0], x, o, T=2)
    assert e.value.status == -5                      # not finalized
    with pytest.raises(ud.EngineError) as e:
        enc.set_weight("encoder.layers.0.no_such.weight", np.zeros(4, np.float32))
    assert e.value.status == -6
    with pytest.raises(ud.EngineError) as e:
        enc.set_weight("encoder.layers.0.norm_out.weight", np.zeros(5, np.float32))
    assert e.value.status == -6
    with pytest.raises(ud.EngineError) as e:
        enc.finalize()                               # weights missing
    assert e.value.status == -5
    for l, w in enumerate([ud.synthetic_layer_weights(cfg, 1, 0)]):
        enc.set_layer_weights(l, w)
    enc.finalize()
    s1 = enc.new_stream()
    with pytest.raises(ud.EngineError) as e:
        enc.new_stream()
    assert e.value.status == -7                      # pool exhausted
    with pytest.raises(ud.EngineError) as e:
        enc.encode_stream_step([s0, s0], x, o, T=1)
    assert e.value.status == -1                      # duplicate stream
    with pytest.raises(ud.EngineError) as e:
        enc.encode_stream_step([s0], x, o, T=3)
    assert e.value.status == -2                      # T > max_chunk
    with pytest.raises(ud.EngineError) as e:
        enc.encode_stream_step([s0], x, x, T=1)
    assert e.value.status == -1                      # aliasing
    enc.encode_stream_step([s0, s1], x, o, T=1)
    ud.synchronize()
    assert s0.cache_len == 1 and s0.step == 1
    s0.reset()
    assert s0.cache_len == 0 and s0.step == 0
    enc.close()


def test_recycled_slot_starts_clean_after_async_step(gpu, orc):
    """A stream destroyed while its step still runs on a non-blocking HIP stream, and a new stream
    created at once in the freed slot: the new stream's K/V and conv caches are all zero (creation
    waits for the device before clearing the slot)."""
    ud = gpu
    cfg = ud.EncoderConfig(layers=4, max_chunk=14, max_streams=4, dtype="bf16")
    enc, _, _ = harness.make_encoder(ud, orc, cfg, seed=91)
    streams = [enc.new_stream() for _ in range(4)]
    rng = np.random.default_rng(3)
    x = ud.DeviceBuffer.from_numpy(rng.standard_normal((4, 14, 1024)).astype(np.float32))
    o = ud.DeviceBuffer(4 * 14 * 1024 * 4)
    hs = ud.HipStream()
    for _ in range(3):
        enc.encode_stream_step(streams, x, o, T=14, hip_stream=hs)
    victim = streams[2]
    victim.close()                   # the queued steps may still be writing its rings
    fresh = enc.new_stream()
    hs.synchronize()
    assert fresh.cache_len == 0
    for l in range(cfg.layers):
        k, v, c, _ = fresh.export_cache(l)
        assert not np.any(k) and not np.any(v) and not np.any(c), "layer %d" % l
    enc.close()

