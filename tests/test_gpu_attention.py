"""GPU parity of the fused rel-pos attention kernel through the C ABI: the reference KAT, one
72-key window (fp32, 2 queries over 72 keys, 8 x 128) and bf16, multi-block keys, the ring-cache form with its
bit-exact cache update."""
import numpy as np
import pytest

import harness
from test_oracle import _kat_attention_inputs, kat_attention_reference

pytestmark = pytest.mark.gpu


def _dev(ud, a):
    return ud.DeviceBuffer.from_numpy(np.ascontiguousarray(a))


def _bf16_dev(ud, a):
    bits = ud.round_bf16(a).view(np.uint32) >> 16
    return ud.DeviceBuffer.from_numpy(bits.astype(np.uint16))


def _run_op(ud, d, dtype="f32"):
    Tq, Tk, H, dk = d["Tq"], d["Tk"], d["H"], d["dk"]
    put = _dev if dtype == "f32" else _bf16_dev
    q, k, v, p = (put(ud, d[n]) for n in ("q", "k", "v", "table"))
    u, vb = _dev(ud, d["u"].astype(np.float32)), _dev(ud, d["vb"].astype(np.float32))
    rr = _dev(ud, d["ranges"].astype(np.int32))
    out = ud.DeviceBuffer(Tq * H * dk * (4 if dtype == "f32" else 2))
    ud.rel_pos_attention(q, k, v, p, d["offset"], u, vb, rr, out, H, Tq, Tk, dk, d["table"].shape[0], dtype=dtype)
    if dtype == "f32":
        return out.download((Tq, H * dk))
    bits = out.download((Tq, H * dk), np.uint16).astype(np.uint32) << 16
    return bits.view(np.float32)


def test_relpos_kat_fp32(gpu, orc):
    """ConformerOpTests.swift:81-142 on the HIP kernel: literal NeMo rel_shift, tol 1e-5."""
    d = _kat_attention_inputs(orc)
    got = _run_op(gpu, d)
    assert np.abs(got - kat_attention_reference(d)).max() < 1e-5


def _window_inputs(orc, seed=7, Tk=72, Tq=2, H=8, dk=128):
    rng = np.random.default_rng(seed)
    D = H * dk
    L = Tk - Tq
    x = rng.standard_normal((Tk, D)).astype(np.float32)
    z = orc.layer_norm(x, np.ones(D, np.float32), np.zeros(D, np.float32))
    b = np.float32(np.sqrt(6.0 / (2 * D)))
    W = [((rng.random((D, D), dtype=np.float32) * 2 - 1) * b) for _ in range(4)]
    q = orc.gemm_nt(z[L:], W[0])
    k = orc.gemm_nt(z, W[1])
    v = orc.gemm_nt(z, W[2])
    table = orc.pos_table(W[3], -(Tk - 1), Tk - 1)     # NeMo's 2*Tk-1 rows, rel -71..71
    u = (rng.standard_normal((H, dk)) * 0.02).astype(np.float32)
    vb = (rng.standard_normal((H, dk)) * 0.02).astype(np.float32)
    ranges = np.array([[0, Tk]] * Tq, np.int32)
    return dict(Tq=Tq, Tk=Tk, H=H, dk=dk, q=q, k=k, v=v, u=u, vb=vb, table=table, offset=Tk - 1, ranges=ranges)


def test_relpos_window_fp32(gpu, orc):
    d = _window_inputs(orc)
    ref = orc.relpos_attention(d["q"], d["k"], d["v"], d["table"], d["u"], d["vb"], d["ranges"], d["offset"], d["H"])
    got = _run_op(gpu, d)
    assert harness.rel_err(got, ref) <= 1e-4


def test_relpos_window_bf16(gpu, orc):
    d = _window_inputs(orc)
    r = {n: gpu.round_bf16(d[n]) for n in ("q", "k", "v", "table")}
    ref = orc.relpos_attention(r["q"], r["k"], r["v"], r["table"], d["u"], d["vb"], d["ranges"], d["offset"], d["H"])
    got = _run_op(gpu, d, "bf16")
    harness.assert_bf16_close(got, ref, "72-key window bf16")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_relpos_multiblock_and_ragged_ranges(gpu, orc, dtype):
    """Tk = 300 spans several key blocks (online softmax); per-query ranges include empty ones."""
    rng = np.random.default_rng(11)
    Tq, Tk, H, dk = 9, 300, 2, 64
    HD = H * dk
    d = dict(Tq=Tq, Tk=Tk, H=H, dk=dk)
    for n, shape in (("q", (Tq, HD)), ("k", (Tk, HD)), ("v", (Tk, HD))):
        d[n] = rng.standard_normal(shape).astype(np.float32)
    d["table"] = rng.standard_normal((2 * Tk - 1, HD)).astype(np.float32) * 0.5
    d["u"] = rng.standard_normal((H, dk)).astype(np.float32) * 0.1
    d["vb"] = rng.standard_normal((H, dk)).astype(np.float32) * 0.1
    d["offset"] = Tk - 1
    d["ranges"] = np.array([[0, 300], [10, 290], [150, 151], [299, 300], [40, 40], [200, 100], [-5, 3],
                            [250, 400], [0, 129]], np.int32)
    if dtype == "bf16":
        for n in ("q", "k", "v", "table"):
            d[n] = gpu.round_bf16(d[n])
    ref = orc.relpos_attention(d["q"], d["k"], d["v"], d["table"], d["u"], d["vb"], d["ranges"], d["offset"], H)
    got = _run_op(gpu, d, dtype)
    assert not np.any(got[4]) and not np.any(got[5])
    if dtype == "f32":
        assert harness.rel_err(got, ref) <= 1e-4
    else:
        harness.assert_bf16_close(got, ref, "multiblock bf16")


@pytest.mark.parametrize("dtype,T,L", [("f32", 2, 70), ("bf16", 2, 70), ("bf16", 14, 70), ("f32", 5, 70),
                                       ("bf16", 1, 70), ("bf16", 3, 70), ("bf16", 4, 70), ("bf16", 2, 63),
                                       ("bf16", 2, 17)])
def test_ring_attention_and_cache_update(gpu, orc, dtype, T, L):
    """The step's fused attention over ring caches (ud_layer_attention): output against the oracle
    on [cache ; new] keys with range [L - cache_len, L + valid), and the ring update bit-exact:
    afterwards the exported window is exactly the last L rows of [old window ; new rows].  The
    fourth stream has an empty range (no cache, no valid frame): its output is 0.  L = 63 puts
    ring rows and new rows in the same 16-key pass; L = 17 leaves most passes past the window."""
    _ring_case(gpu, orc, dtype, T, L, 1.0)


@pytest.mark.parametrize("T", [2, 14])
def test_ring_attention_large_scores(gpu, orc, T):
    """q scaled by 8: scores with a spread of about +-25 before the softmax (a nearly one-hot
    softmax), through the wave kernel (T = 2) and the MFMA kernel's full-window path (T = 14, the
    first stream's cache full and every frame valid)."""
    _ring_case(gpu, orc, "bf16", T, 70, 8.0)


def _ring_case(gpu, orc, dtype, T, L, q_scale):
    ud = gpu
    cfg = ud.EncoderConfig(layers=2, left_context=L, max_chunk=max(T, 2), max_streams=4, dtype=dtype)
    enc, model, _ = harness.make_encoder(ud, orc, cfg, seed=5)
    D, H = cfg.d_model, cfg.heads
    rng = np.random.default_rng(3)
    S = 4
    streams = [enc.new_stream() for _ in range(S)]
    st = harness.OracleState(S, cfg)
    st.seed_random(rng, 0)
    st.len[:] = [L, min(33, L), 0, 0]
    st.import_into(streams, ud, dtype == "bf16")
    valid = np.array([T, max(T - 1, 0), T, 0], np.int32)
    layer = 1
    qkv = rng.standard_normal((S, T, 3 * D)).astype(np.float32)
    qkv[:, :, :D] *= q_scale
    if dtype == "bf16":
        # a 16-bit encoder's activations (qkv in, att out) are IEEE half
        qkv = ud.round_f16(qkv)
        qbuf = _dev(ud, ud.f16_bits(qkv))
        att = ud.DeviceBuffer(S * T * D * 2)
    else:
        qbuf = _dev(ud, qkv)
        att = ud.DeviceBuffer(S * T * D * 4)
    enc.layer_attention(streams, T, layer, qbuf, att, valid=valid)
    ud.synchronize()
    if dtype == "bf16":
        got = ud.from_f16_bits(att.download((S, T, D), np.uint16))
    else:
        got = att.download((S, T, D))
    P = model.P[layer]
    if dtype == "bf16":
        P = ud.round_f16(P)
    for s in range(S):
        keys = np.concatenate([st.k[s, layer], qkv[s, :, D:2 * D]])
        vals = np.concatenate([st.v[s, layer], qkv[s, :, 2 * D:]])
        rr = np.array([[L - st.len[s], L + valid[s]]] * T, np.int32)
        u = model.layers[layer][11]
        vb = model.layers[layer][12]
        ref = orc.relpos_attention(qkv[s, :, :D], keys, vals, P, u, vb, rr, model.rel_offset, H)
        if valid[s] == 0 and st.len[s] == 0:
            assert not np.any(ref) and not np.any(got[s]), s
            continue
        if dtype == "f32":
            assert harness.rel_err(got[s], ref) <= 1e-4, s
        else:
            harness.assert_bf16_close(got[s], ref, "ring stream %d" % s)
    # commit and check the ring update bit-exactly
    enc.advance(streams, T)
    for s, stream in enumerate(streams):
        k, v, c, n = stream.export_cache(layer)
        assert n == min(int(st.len[s]) + T, L)
        want_k = np.concatenate([st.k[s, layer], qkv[s, :, D:2 * D]])[-L:]
        want_v = np.concatenate([st.v[s, layer], qkv[s, :, 2 * D:]])[-L:]
        np.testing.assert_array_equal(k, want_k)
        np.testing.assert_array_equal(v, want_v)
    enc.close()
