"""Pins the oracle's decoder attention (orc_gqa_attention) and RoPE (orc_rope_rotate_half) against
the reference's known-answer tests (Tests/DictatorEngineTests/VoxtralOpTests.swift) and against
independent formulations: a float64 numpy softmax attention and a rotation by a complex
exponential."""
import numpy as np


def _f16(x):
    # the reference's roundTrip(_, .f16): IEEE half, round to nearest even
    return x.astype(np.float16).astype(np.float32)


def numpy_gqa(q, k, v, ranges, Hq, Hkv):
    """Textbook softmax attention in float64 (vectorised), query head h -> kv head h // (Hq/Hkv)."""
    Tq = q.shape[0]
    d = q.shape[1] // Hq
    out = np.zeros((Tq, Hq * d))
    for i in range(Tq):
        lo, hi = max(int(ranges[i, 0]), 0), min(int(ranges[i, 1]), k.shape[0])
        for h in range(Hq):
            if hi <= lo:
                continue
            kvh = h // (Hq // Hkv)
            qh = q[i, h * d:(h + 1) * d].astype(np.float64)
            kk = k[lo:hi, kvh * d:(kvh + 1) * d].astype(np.float64)
            vv = v[lo:hi, kvh * d:(kvh + 1) * d].astype(np.float64)
            s = kk @ qh / np.sqrt(d)
            p = np.exp(s - s.max())
            out[i, h * d:(h + 1) * d] = (p / p.sum()) @ vv
    return out


def test_gqa_attention_kat(orc):
    """VoxtralOpTests.swift:6-38: 3 queries over 1200 f16 keys (3 online-softmax blocks in the
    reference kernel), 8 query heads on 2 kv heads, head_dim 64; tolerance 2e-5."""
    Tq, Tk, Hq, Hkv, d = 3, 1200, 8, 2, 64
    q = orc.lcg_floats(Tq * Hq * d, 51).reshape(Tq, Hq * d)
    k = _f16(orc.lcg_floats(Tk * Hkv * d, 52)).reshape(Tk, Hkv * d)
    v = _f16(orc.lcg_floats(Tk * Hkv * d, 53)).reshape(Tk, Hkv * d)
    ranges = np.array([[0, 1200], [450, 1100], [700, 701]], np.int32)
    got = orc.gqa_attention(q, k, v, ranges, Hq, Hkv)
    assert np.abs(got - numpy_gqa(q, k, v, ranges, Hq, Hkv)).max() < 2e-5


def test_gqa_multi_query_kat(orc):
    """VoxtralOpTests.swift:42-59: 4 queries, 32 heads x 64, f16 caches of 700 keys, ranges
    [m, 697 + m): the oracle's several-query call equals one call per query (each query is
    computed on its own) and the float64 numpy attention."""
    Tq, Tk, H, d = 4, 700, 32, 64
    q = orc.lcg_floats(Tq * H * d, 55).reshape(Tq, H * d)
    k = _f16(orc.lcg_floats(Tk * H * d, 56)).reshape(Tk, H * d)
    v = _f16(orc.lcg_floats(Tk * H * d, 57)).reshape(Tk, H * d)
    ranges = np.array([[0, 697], [1, 698], [2, 699], [3, 700]], np.int32)
    got = orc.gqa_attention(q, k, v, ranges, H, H)
    per = np.concatenate([orc.gqa_attention(q[i:i + 1], k, v, ranges[i:i + 1], H, H) for i in range(Tq)])
    assert np.abs(got - per).max() <= 1e-5
    assert np.abs(got - numpy_gqa(q, k, v, ranges, H, H)).max() < 2e-5


def test_gqa_head_map_and_edges(orc):
    """Query head h reads kv head h // (Hq/Hkv): with V constant per kv head the output of head h
    is exactly that constant; a single key returns its V row; an empty range returns 0."""
    Tq, Tk, Hq, Hkv, d = 4, 40, 8, 2, 16
    rng = np.random.default_rng(3)
    q = rng.standard_normal((Tq, Hq * d)).astype(np.float32)
    k = rng.standard_normal((Tk, Hkv * d)).astype(np.float32)
    v = np.concatenate([np.full((Tk, d), 1.5 + c, np.float32) for c in range(Hkv)], axis=1)
    ranges = np.array([[0, 40], [5, 6], [30, 30], [-3, 100]], np.int32)
    got = orc.gqa_attention(q, k, v, ranges, Hq, Hkv)
    for h in range(Hq):
        want = 1.5 + h // (Hq // Hkv)
        assert np.all(got[[0, 1, 3], h * d:(h + 1) * d] == np.float32(want)), h
    assert not np.any(got[2])
    v2 = rng.standard_normal((Tk, Hkv * d)).astype(np.float32)
    got2 = orc.gqa_attention(q, k, v2, ranges, Hq, Hkv)
    for h in range(Hq):
        kvh = h // (Hq // Hkv)
        np.testing.assert_array_equal(got2[1, h * d:(h + 1) * d], v2[5, kvh * d:(kvh + 1) * d])


def rope_complex(x, H, d, inv_freq, pos):
    """Rotate-half RoPE as multiplication of x_i + i x_{i+d/2} by exp(i angle), angle the float32
    product pos * inv_freq (as the reference forms it)."""
    y = x.astype(np.float64).copy()
    half = d // 2
    for t in range(x.shape[0]):
        ang = (np.float32(pos[t]) * inv_freq).astype(np.float64)
        rot = np.exp(1j * ang)
        for h in range(H):
            z = (x[t, h * d:h * d + half] + 1j * x[t, h * d + half:(h + 1) * d].astype(np.float64)) * rot
            y[t, h * d:h * d + half] = z.real
            y[t, h * d + half:(h + 1) * d] = z.imag
    return y


def test_rope_kat(orc, ud):
    """VoxtralOpTests.swift:60-75: T=5 rows, 3 heads x 16, pos0 = 1234, theta 1e6; tolerance 1e-5."""
    T, H, d, pos0 = 5, 3, 16, 1234
    x = orc.lcg_floats(T * H * d, 61).reshape(T, H * d)
    inv = ud.rope_inv_freq(d, 1e6)
    np.testing.assert_array_equal(inv, np.array([np.float32(1.0 / 1e6 ** (2 * i / d)) for i in range(d // 2)]))
    got = orc.rope_rotate_half(x, H, d, inv, pos0=pos0)
    ref = rope_complex(x, H, d, inv, np.arange(pos0, pos0 + T))
    assert np.abs(got - ref).max() < 1e-5


def test_rope_positions_and_norm(orc, ud):
    """Per-row positions equal pos0 + t when given as such; the rotation preserves each pair's
    norm; position 0 is the identity."""
    T, H, d = 6, 4, 128
    rng = np.random.default_rng(8)
    x = rng.standard_normal((T, H * d + 8)).astype(np.float32)   # ld > H*d: the tail is untouched
    inv = ud.rope_inv_freq(d, 1e6)
    a = orc.rope_rotate_half(x, H, d, inv, pos0=100)
    b = orc.rope_rotate_half(x, H, d, inv, positions=np.arange(100, 100 + T))
    np.testing.assert_array_equal(a, b)
    np.testing.assert_array_equal(a[:, H * d:], x[:, H * d:])
    half = d // 2
    for h in range(H):
        n0 = x[:, h * d:h * d + half] ** 2 + x[:, h * d + half:(h + 1) * d] ** 2
        n1 = a[:, h * d:h * d + half] ** 2 + a[:, h * d + half:(h + 1) * d] ** 2
        assert np.abs(n1 - n0).max() < 1e-4
    z = orc.rope_rotate_half(x, H, d, inv, positions=np.zeros(T, np.int32))
    np.testing.assert_array_equal(z, x)
