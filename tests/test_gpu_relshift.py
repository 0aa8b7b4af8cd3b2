"""Bit-exact rel_shift indexing through every attention kernel, on the GPU through the C ABI.

The positional term alone decides the softmax: q = 0, K = 0, pos_bias_u = 0 and pos_bias_v = e_0
in each head, so score(i, j) = P[t(i, j)][head column 0] / sqrt(dk), where t(i, j) is the table row
that rel_shift assigns to query i and key j.  Each head's table column 0 peaks at one row t*: in the
single-op and offline kernels P is given directly (one nonzero row per head); in the streaming ring
kernels P is the encoder's own table PE . W_pos^T, with W_pos's head row set to c PE[t*] so that
P[t] = c PE[t] . PE[t*] (a sum of cos(w_k (t - t*)), largest at t = t*).  The peak's score beats
every other score by more than 120, so exp() of every other score underflows to exactly 0,
the softmax is exactly one-hot and the output row equals the V row of the key with
(Tk - Tq + i) - j + rel_offset = t* (20_conformer.metal:183, 189; NeMo's pad/view rel_shift),
bit for bit.  A wrong index (off by one, a transposed i/j, a wrong band origin or ring slot) selects
another V row and fails.  Every table row is the peak of some head in some call, so the whole band
is covered; queries whose peak key falls outside their range are not checked."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

H, DK = 8, 128
D = H * DK
# Scale of the positional peak in the ring tests: the peak is C_PEAK * 512 (< 65504, the IEEE-half
# maximum of a 16-bit encoder's tables) and beats every other row by >= 2.6 % of it, i.e. its score
# beats every other score by more than MARGIN; exp(-MARGIN) underflows to 0 in fp32 (below 2^-150
# from a margin of 104 on).
C_PEAK = 125.0
MARGIN = 120.0


def _bf16_bits(a):
    a = np.ascontiguousarray(a, np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    return (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF).astype(np.uint16)


def _from_bits(b):
    return (b.astype(np.uint32) << 16).view(np.float32)


def _sinusoid(pos):
    """NeMo RelPositionalEncoding row (FastConformer.swift:147-158): fp32 angle, double sin/cos."""
    k = np.float32(-(np.float32(np.log(10000.0)) / np.float32(D)))
    div = np.exp((np.arange(0, D, 2, dtype=np.float32) * k).astype(np.float64)).astype(np.float32)
    ang = (np.float32(pos) * div).astype(np.float32).astype(np.float64)
    out = np.empty(D, np.float32)
    out[0::2] = np.sin(ang)
    out[1::2] = np.cos(ang)
    return out


def _peak_rows(n_rel, calls):
    """Table row of each (call, head): every row is some head's peak."""
    rows = np.arange(calls * H) % n_rel
    return rows.reshape(calls, H)


def _direct_table(n_rel, peaks, dtype):
    """P [n_rel, D] with column h*128 nonzero (= 5000) only at row peaks[h]."""
    P = np.zeros((n_rel, D), np.float32)
    for h in range(H):
        P[peaks[h], h * DK] = 5000.0
    return P


def _biases():
    u = np.zeros((H, DK), np.float32)
    vb = np.zeros((H, DK), np.float32)
    vb[:, 0] = 1.0
    return u, vb


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_relshift_exact_op_kernel(gpu, dtype):
    """relpos_op_kernel (ud_relpos_attention): Tq 5 queries over Tk 40 keys, 8 heads."""
    ud = gpu
    Tq, Tk = 5, 40
    n_rel, rel_offset = Tq + Tk - 1, Tq - 1
    rng = np.random.default_rng(1)
    v = rng.standard_normal((Tk, D)).astype(np.float32)
    if dtype == "bf16":
        v = _from_bits(_bf16_bits(v))
    enc = (lambda a: _bf16_bits(a)) if dtype == "bf16" else (lambda a: np.ascontiguousarray(a, np.float32))
    dev = ud.DeviceBuffer.from_numpy
    zeros_q, zeros_k = dev(enc(np.zeros((Tq, D)))), dev(enc(np.zeros((Tk, D))))
    u, vb = _biases()
    ranges = dev(np.tile(np.array([0, Tk], np.int32), (Tq, 1)))
    checked = 0
    for peaks in _peak_rows(n_rel, (n_rel + H - 1) // H):
        P = _direct_table(n_rel, peaks, dtype)
        out = ud.DeviceBuffer(Tq * D * (2 if dtype == "bf16" else 4))
        ud.rel_pos_attention(zeros_q, zeros_k, dev(enc(v)), dev(enc(P)), rel_offset, dev(u), dev(vb), ranges, out, H,
                             Tq, Tk, DK, n_rel, dtype=dtype)
        ud.synchronize()
        got = _from_bits(out.download((Tq, D), np.uint16)) if dtype == "bf16" else out.download((Tq, D))
        for h in range(H):
            rel = int(peaks[h]) - rel_offset
            for i in range(Tq):
                j = (Tk - Tq + i) - rel
                if 0 <= j < Tk:
                    np.testing.assert_array_equal(got[i, h * DK:(h + 1) * DK], v[j, h * DK:(h + 1) * DK],
                                                  err_msg="head %d query %d table row %d" % (h, i, peaks[h]))
                    checked += 1
    assert checked >= Tq * Tk // 2


def test_relshift_exact_offline_dense_kernel(gpu):
    """relpos_dense_kernel (ud_relpos_attention_batched): 2 utterances x 200 frames (query tiles of
    128 and key tiles of 64 with the 3-chunk band ring), full-context ranges."""
    ud = gpu
    B, T = 2, 200
    n_rel, rel_offset = 2 * T - 1, T - 1
    rng = np.random.default_rng(2)
    v = _from_bits(_bf16_bits(rng.standard_normal((B, T, D))))
    dev = ud.DeviceBuffer.from_numpy
    zq = dev(np.zeros((B, T, D), np.uint16))
    vdev = dev(_bf16_bits(v))
    u, vb = _biases()
    ranges = dev(np.tile(np.array([0, T], np.int32), (B, T, 1)))
    # every table row would take 50 launches; rows within 70 of the diagonal (the ones the streaming
    # masks use), both ends of the table and tile-edge offsets are covered instead
    rows = np.unique(np.concatenate([np.arange(rel_offset - 72, rel_offset + 73), [0, 1, n_rel - 2, n_rel - 1],
                                     rel_offset + np.array([-191, -128, -127, -64, -63, 63, 64, 127, 128, 191])]))
    rows = np.concatenate([rows, rows[:(-len(rows)) % H]])
    for peaks in rows.reshape(-1, H):
        P = _direct_table(n_rel, peaks, "bf16")
        out = ud.DeviceBuffer(B * T * D * 2)
        ud.rel_pos_attention_batched(zq, zq, vdev, dev(_bf16_bits(P)), rel_offset, dev(u), dev(vb), ranges, out, B,
                                     T, H, n_rel)
        ud.synchronize()
        got = _from_bits(out.download((B, T, D), np.uint16))
        for h in range(H):
            rel = int(peaks[h]) - rel_offset
            i = np.arange(T)
            j = i - rel
            ok = (j >= 0) & (j < T)
            for b in range(B):
                np.testing.assert_array_equal(got[b, i[ok], h * DK:(h + 1) * DK], v[b, j[ok], h * DK:(h + 1) * DK],
                                              err_msg="utterance %d head %d table row %d" % (b, h, peaks[h]))


@pytest.mark.parametrize("dtype,T", [("bf16", 2), ("bf16", 4), ("bf16", 14), ("bf16", 5), ("f32", 2)])
def test_relshift_exact_ring_kernels(gpu, dtype, T):
    """The streaming kernels over the ring caches (ud_layer_attention): bf16 T 2 and 4 (small
    kernel, both query-tile widths), bf16 T 5 and 14 (MFMA kernel), fp32 T 2 (general ring kernel).
    Tables come from the encoder's own finalize (a 16-bit encoder's tables, caches and activations
    are IEEE half); the ring origin is moved off slot 0 so the ring wrap is part of the index."""
    ud = gpu
    L = 70
    n_rel, rel_offset = L + 2 * T - 1, T - 1
    layers = (n_rel + H - 1) // H
    cfg = ud.EncoderConfig(layers=layers, max_chunk=T, max_streams=2, dtype=dtype)
    enc = ud.Encoder(cfg)
    rels = np.arange(n_rel) - rel_offset
    PE = np.stack([_sinusoid(r) for r in rels])
    peaks = _peak_rows(n_rel, layers)
    for l in range(layers):
        w = ud.synthetic_layer_weights(cfg, 5, l)
        wpos = np.zeros((D, D), np.float32)
        for h in range(H):
            wpos[h * DK] = C_PEAK * PE[peaks[l, h]]
        w["self_attn.linear_pos.weight"] = wpos
        u, vb = _biases()
        w["self_attn.pos_bias_u"], w["self_attn.pos_bias_v"] = u, vb
        enc.set_layer_weights(l, w)
    enc.finalize()
    # the margin the test relies on, from the same table computed on the host
    for l in range(layers):
        for h in range(H):
            wrow = PE[peaks[l, h]] * C_PEAK
            if dtype == "bf16":
                wrow = _from_bits(_bf16_bits(wrow))
            col = np.sort(PE.astype(np.float64) @ wrow.astype(np.float64))[::-1]
            assert (col[0] - col[1]) / np.sqrt(DK) > MARGIN
            assert np.abs(col).max() < 65504.0          # the table fits IEEE half (16-bit encoders)
    rng = np.random.default_rng(3)
    S = 2
    streams = [enc.new_stream() for _ in range(S)]
    kc = np.zeros((L, D), np.float32)
    conv = np.zeros((8, D), np.float32)
    # a 16-bit encoder's caches and activations are IEEE half: values exact in half
    vcache = rng.standard_normal((S, layers, L, D)).astype(np.float32)
    if dtype == "bf16":
        vcache = ud.round_f16(vcache)
    for s, st in enumerate(streams):
        for l in range(layers):
            st.import_cache(l, kc, vcache[s, l], conv, L)
    enc.advance(streams, 17)               # ring origin 17: cached key j sits in slot (17 + j) % 70
    for s, st in enumerate(streams):
        for l in range(layers):
            st.import_cache(l, kc, vcache[s, l], conv, L)
    vnew = rng.standard_normal((S, T, D)).astype(np.float32)
    if dtype == "bf16":
        vnew = ud.round_f16(vnew)
    qkv = np.zeros((S, T, 3 * D), np.float32)
    qkv[:, :, 2 * D:] = vnew
    esz = 2 if dtype == "bf16" else 4
    qkv_dev = ud.DeviceBuffer.from_numpy(ud.f16_bits(qkv) if dtype == "bf16" else qkv)
    checked = 0
    for l in range(layers):
        att = ud.DeviceBuffer(S * T * D * esz)
        enc.layer_attention(streams, T, l, qkv_dev, att)
        ud.synchronize()
        got = ud.from_f16_bits(att.download((S, T, D), np.uint16)) if dtype == "bf16" else att.download((S, T, D))
        for s in range(S):
            window = np.concatenate([vcache[s, l], vnew[s]])       # [L cached ; T new], logical order
            for h in range(H):
                rel = int(peaks[l, h]) - rel_offset
                for i in range(T):
                    j = (L + i) - rel
                    if 0 <= j < L + T:
                        np.testing.assert_array_equal(
                            got[s, i, h * DK:(h + 1) * DK], window[j, h * DK:(h + 1) * DK],
                            err_msg="layer %d stream %d head %d query %d table row %d" % (l, s, h, i, peaks[l, h]))
                        checked += 1
    assert checked >= S * T * n_rel // 2
    enc.close()
