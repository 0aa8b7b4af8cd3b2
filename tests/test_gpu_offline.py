"""GPU parity of the offline (whole-utterance) rel-pos attention, ud_relpos_attention_batched, against
the oracle's relpos_attention on the same bf16 inputs: key padding, chunked_limited masks clipped to
the valid length (forwardOffline, FastConformer.swift:361-398), tile-ragged lengths and the
8 x 1500-frame batch (sampled query rows)."""
import numpy as np
import pytest

import harness

pytestmark = pytest.mark.gpu

H, DK = 8, 128


def _bits(ud, a):
    return (ud.round_bf16(a).view(np.uint32) >> 16).astype(np.uint16)


def _inputs(ud, rng, B, T):
    D = H * DK
    q, k, v = (ud.round_bf16(rng.standard_normal((B, T, D)).astype(np.float32)) for _ in range(3))
    P = ud.round_bf16((rng.standard_normal((2 * T - 1, D)) * 0.5).astype(np.float32))
    u = (rng.standard_normal((H, DK)) * 0.02).astype(np.float32)
    vb = (rng.standard_normal((H, DK)) * 0.02).astype(np.float32)
    return q, k, v, P, u, vb


def _run(ud, q, k, v, P, u, vb, ranges):
    B, T, D = q.shape
    dev = ud.DeviceBuffer.from_numpy
    out = ud.DeviceBuffer(B * T * D * 2)
    ud.rel_pos_attention_batched(dev(_bits(ud, q)), dev(_bits(ud, k)), dev(_bits(ud, v)), dev(_bits(ud, P)), T - 1,
                                 dev(u), dev(vb), dev(np.ascontiguousarray(ranges, np.int32)), out, B, T, H,
                                 P.shape[0])
    ud.synchronize()
    return (out.download((B, T, D), np.uint16).astype(np.uint32) << 16).view(np.float32)


def _oracle(orc, q, k, v, P, u, vb, ranges):
    return np.stack([orc.relpos_attention(q[b], k[b], v[b], P, u, vb, ranges[b], q.shape[1] - 1, H)
                     for b in range(q.shape[0])])


def test_offline_key_padding(gpu, orc):
    """Two utterances of 200 frames (two query tiles, four 64-key tiles), valid 200 and 137."""
    ud = gpu
    rng = np.random.default_rng(31)
    B, T = 2, 200
    q, k, v, P, u, vb = _inputs(ud, rng, B, T)
    lens = [200, 137]
    ranges = np.zeros((B, T, 2), np.int32)
    for b, n in enumerate(lens):
        ranges[b, :, 1] = n
    got = _run(ud, q, k, v, P, u, vb, ranges)
    harness.assert_bf16_close(got, _oracle(orc, q, k, v, P, u, vb, ranges), "offline key padding")


def test_offline_chunked_limited_mask(gpu, orc):
    """chunked_limited [70, 1] over 300 frames clipped to 250 valid (the offline streaming mask);
    plus one query row with an empty range."""
    ud = gpu
    rng = np.random.default_rng(32)
    B, T = 1, 300
    q, k, v, P, u, vb = _inputs(ud, rng, B, T)
    # the product's range builder: chunked_limited [70, 1] with the clip to 250 valid frames
    ranges = ud.chunked_limited_ranges(T, 70, 1, valid=[250])
    ranges[0, 17] = [40, 40]
    got = _run(ud, q, k, v, P, u, vb, ranges)
    assert not np.any(got[0, 17])
    harness.assert_bf16_close(got, _oracle(orc, q, k, v, P, u, vb, ranges), "offline chunked mask")


def test_offline_batch_1500_sampled(gpu, orc):
    """8 utterances x 1500 frames, valid lengths uniform in 900..1500 (key padding); 48 query rows
    per utterance (first, last, tile edges, random) are checked against the oracle."""
    ud = gpu
    rng = np.random.default_rng(33)
    B, T = 8, 1500
    q, k, v, P, u, vb = _inputs(ud, rng, B, T)
    lens = rng.integers(900, 1501, B)
    ranges = np.zeros((B, T, 2), np.int32)
    ranges[:, :, 1] = lens[:, None]
    got = _run(ud, q, k, v, P, u, vb, ranges)
    for b in range(B):
        rows = np.unique(np.concatenate([[0, 63, 64, 127, 128, 1407, 1408, T - 1, lens[b] - 1],
                                         rng.integers(0, T, 39)]))
        sel = np.zeros((T, 2), np.int32)
        sel[rows] = ranges[b, rows]
        ref = orc.relpos_attention(q[b], k[b], v[b], P, u, vb, sel, T - 1, H)
        harness.assert_bf16_close(got[b, rows], ref[rows], "utterance %d" % b)


@pytest.mark.parametrize("order", ["growing", "shrinking"])
def test_offline_running_max(gpu, orc, order):
    """Scores that grow (or shrink) along the keys: with q and k aligned and k scaled by its key index,
    every 64-key tile raises (or never raises) each query's running maximum, so the accumulator is
    rescaled on every tile (or only on the first); scores reach about +-25 before the scale."""
    ud = gpu
    rng = np.random.default_rng(34)
    B, T = 1, 320
    q, k, v, P, u, vb = _inputs(ud, rng, B, T)
    ramp = np.linspace(0.0, 1.0, T, dtype=np.float32)
    if order == "shrinking":
        ramp = ramp[::-1].copy()
    q = ud.round_bf16((np.abs(q) * 0.5 + 0.5).astype(np.float32))
    k = ud.round_bf16((0.25 * rng.standard_normal((B, T, H * DK)) + 2.0 * ramp[None, :, None]).astype(np.float32))
    ranges = np.zeros((B, T, 2), np.int32)
    ranges[:, :, 1] = T
    got = _run(ud, q, k, v, P, u, vb, ranges)
    harness.assert_bf16_close(got, _oracle(orc, q, k, v, P, u, vb, ranges), "offline running max " + order)


@pytest.mark.parametrize("B,Hh,T", [(3, 3, 150), (2, 8, 130), (66, 4, 24), (65, 1, 20)])
def test_offline_grid_orders(gpu, orc, B, Hh, T):
    """Every grid order of the kernel: (utterance, head) pairs that do not divide among the 8 XCDs
    (3 x 3), that do (2 x 8), and more than 64 utterances (taken in order, with and without the
    XCD grouping), each with ragged valid lengths so the longest-first order is not the identity."""
    ud = gpu
    rng = np.random.default_rng(35 + B + Hh)
    D = Hh * DK
    q, k, v = (ud.round_bf16(rng.standard_normal((B, T, D)).astype(np.float32)) for _ in range(3))
    P = ud.round_bf16((rng.standard_normal((2 * T - 1, D)) * 0.5).astype(np.float32))
    u = (rng.standard_normal((Hh, DK)) * 0.02).astype(np.float32)
    vb = (rng.standard_normal((Hh, DK)) * 0.02).astype(np.float32)
    lens = rng.integers(1, T + 1, B)
    ranges = np.zeros((B, T, 2), np.int32)
    ranges[:, :, 1] = lens[:, None]
    dev = ud.DeviceBuffer.from_numpy
    out = ud.DeviceBuffer(B * T * D * 2)
    ud.rel_pos_attention_batched(dev(_bits(ud, q)), dev(_bits(ud, k)), dev(_bits(ud, v)), dev(_bits(ud, P)), T - 1,
                                 dev(u), dev(vb), dev(ranges), out, B, T, Hh, P.shape[0])
    ud.synchronize()
    got = (out.download((B, T, D), np.uint16).astype(np.uint32) << 16).view(np.float32)
    ref = np.stack([orc.relpos_attention(q[b], k[b], v[b], P, u, vb, ranges[b], T - 1, Hh) for b in range(B)])
    harness.assert_bf16_close(got, ref, "offline grid order B=%d H=%d" % (B, Hh))


def test_offline_error_paths(gpu):
    ud = gpu
    b = ud.DeviceBuffer(1 << 12)
    with pytest.raises(ud.EngineError):
        ud._check(ud.lib().ud_relpos_attention_batched(0, b.ptr, b.ptr, b.ptr, b.ptr, b.ptr, b.ptr, b.ptr, b.ptr,
                                                       1, 4, 8, 128, 3, 7, None))
    with pytest.raises(ud.EngineError):
        ud.rel_pos_attention_batched(b, b, b, b, 3, b, b, b, b, 1, 4, 8, 7, head_dim=64)
