"""Pins the CPU oracle (oracle/ud_oracle.c) against the reference's own known-answer tests and
against library routines / closed forms, so that a plausible slip in the oracle fails here."""
import json
import os

import numpy as np
import pytest

import refimpl


def _torch():
    # torch is a CPU-side reference here; it is imported lazily so that a GPU test process that only
    # collects this module never loads torch's bundled HIP runtime.
    import torch
    import torch.nn.functional as F
    return torch, F

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _lcg_py(n, seed):
    # Tests/DictatorEngineTests/GemmTests.swift:7-14 in Python big-int arithmetic.
    M = (1 << 64) - 1
    a, c = 6364136223846793005, 1442695040888963407
    s = (seed * a + c) & M
    out = []
    for _ in range(n):
        s = (s * a + c) & M
        out.append(float((s >> 11) % (1 << 24)) / float(1 << 23) - 1.0)
    return np.array(out, np.float32)


def test_lcg_matches_reference_generator(orc):
    for seed in (0, 1, 11, 41, 46, 12345678901):
        np.testing.assert_array_equal(orc.lcg_floats(257, seed), _lcg_py(257, seed))
    x = orc.lcg_floats(200000, 7)
    assert x.min() >= -1.0 and x.max() < 1.0 and abs(float(x.mean())) < 0.01


def test_lcg_golden_fixture(orc):
    with open(os.path.join(GOLDEN, "lcg.json")) as f:
        g = json.load(f)
    for seed, vals in g["values"].items():
        np.testing.assert_array_equal(orc.lcg_floats(len(vals), int(seed)), np.array(vals, np.float32))


def test_bf16_rounding_matches_torch(orc):
    torch, F = _torch()
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[~np.isnan(x)]
    edge = np.array([0.0, -0.0, 1.0, 1.00390625, 1.0078125, 1.01171875, 3.4e38, -3.4e38, np.inf, -np.inf,
                     1e-40, -1e-40, 65504.0], np.float32)
    x = np.concatenate([x, edge])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(orc.bf16_bits(x), want)
    nan = np.array([np.nan, -np.nan], np.float32)
    assert list(orc.bf16_bits(nan)) == [0x7FC0, 0x7FC0]
    # widening then rounding is the identity on bf16 values
    r = orc.round_bf16(x[np.isfinite(x)])
    np.testing.assert_array_equal(orc.round_bf16(r), r)


def test_layer_norm_kat(orc):
    torch, F = _torch()
    # ConformerOpTests.swift:6-25: T=5, D=1024, x*3+0.5, seeds 11-13, SiLU, tol 1e-5
    T, D = 5, 1024
    x = orc.lcg_floats(T * D, 11).reshape(T, D) * 3 + 0.5
    g, b = orc.lcg_floats(D, 12), orc.lcg_floats(D, 13)
    got = orc.layer_norm(x, g, b, act=orc.ACT_SILU)
    ref = F.silu(F.layer_norm(torch.from_numpy(x).double(), (D,), torch.from_numpy(g).double(),
                              torch.from_numpy(b).double(), eps=1e-5)).numpy()
    assert np.abs(got - ref).max() < 1e-5
    got = orc.layer_norm(x, g, b)
    ref = F.layer_norm(torch.from_numpy(x).double(), (D,), torch.from_numpy(g).double(),
                       torch.from_numpy(b).double(), eps=1e-5).numpy()
    assert np.abs(got - ref).max() < 1e-5


GEMM_SHAPES = [(1, 1, 1), (1, 1024, 1024), (7, 33, 65), (64, 64, 64), (100, 257, 130), (129, 640, 1024),
               (3, 4096, 1024)]


@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
def test_gemm_kat(orc, M, N, K):
    # GemmTests.swift:36-45: LCG seeds 1/2, tol 1e-4*sqrt(K)+1e-5 against an fp64-accumulated GEMM
    a = orc.lcg_floats(M * K, 1).reshape(M, K)
    b = orc.lcg_floats(N * K, 2).reshape(N, K)
    ref = a.astype(np.float64) @ b.astype(np.float64).T
    assert np.abs(orc.gemm_nt(a, b) - ref).max() < 1e-4 * np.sqrt(K) + 1e-5


def test_gemm_epilogue_kat(orc):
    torch, F = _torch()
    # GemmTests.swift:66-91: alpha .5, bias, act, outScale .25, residual x2
    M, N, K = 37, 70, 50
    a = orc.lcg_floats(M * K, 5).reshape(M, K)
    b = orc.lcg_floats(N * K, 6).reshape(N, K)
    bias, res = orc.lcg_floats(N, 7), orc.lcg_floats(M * N, 8).reshape(M, N)
    ab = torch.from_numpy(a).double() @ torch.from_numpy(b).double().T
    for act, fn in [(orc.ACT_NONE, lambda v: v), (orc.ACT_RELU, F.relu), (orc.ACT_SILU, F.silu),
                    (orc.ACT_GELU_ERF, lambda v: F.gelu(v))]:
        got = orc.gemm_nt(a, b, bias=bias, R=res, alpha=0.5, act=act, out_scale=0.25, res_scale=2.0)
        ref = (0.25 * fn(0.5 * ab + torch.from_numpy(bias).double()) + 2 * torch.from_numpy(res).double()).numpy()
        assert np.abs(got - ref).max() < 2e-5, act


def test_glu_and_dwconv_kat(orc):
    torch, F = _torch()
    # ConformerOpTests.swift:27-47: T=6, D=64, K=9, seeds 21-24
    T, D, K = 6, 64, 9
    x = orc.lcg_floats(T * 2 * D, 21).reshape(T, 2 * D)
    ref = F.glu(torch.from_numpy(x).double(), dim=-1).numpy()
    assert np.abs(orc.glu(x) - ref).max() < 1e-6
    xin = orc.lcg_floats((T + K - 1) * D, 22).reshape(T + K - 1, D)
    w, bias = orc.lcg_floats(D * K, 23).reshape(D, K), orc.lcg_floats(D, 24)
    ref2 = np.stack([np.correlate(xin[:, d].astype(np.float64), w[d].astype(np.float64), "valid") + bias[d]
                     for d in range(D)], axis=1)
    assert np.abs(orc.dwconv1d(xin, w, bias) - ref2).max() < 1e-5


def test_sinusoid_closed_form(orc):
    D = 1024
    # The reference rounds div and angle = pos*div to fp32 (FastConformer.swift:150-153): the angle
    # error is at most 2*|pos*div|*2^-24 <= |pos|*1.2e-7, plus the final rounding of sin/cos.
    for pos in (-1499, -71, -1, 0, 1, 2, 70, 71, 1499):
        pe = refimpl.nemo_pe(abs(pos) + 1, D)[0 if pos >= 0 else -1]
        np.testing.assert_allclose(orc.sinusoid(pos, D), pe, rtol=0, atol=abs(pos) * 1.2e-7 + 1e-7)
    rows = orc.pe_rows(-3, 5, 64)
    for r, pos in enumerate(range(-3, 6)):
        np.testing.assert_array_equal(rows[r], orc.sinusoid(pos, 64))


def _rel_shift_index(Tq, Tk, i, j):
    # the oracle's (and the kernels') folded index: table row for (i, j) with rel_offset = Tk-1
    return (Tk - Tq + i) - j + (Tk - 1)


@pytest.mark.parametrize("Tq,Tk", [(1, 1), (2, 72), (7, 12), (14, 84), (5, 5), (3, 40)])
def test_rel_shift_index_map_bit_exact(Tq, Tk):
    """NeMo's pad/view rel_shift applied to a matrix of column indices gives, for (i, j < Tk), the
    pe row n = (Tk-1) - rel with rel = (Tk-Tq+i) - j; the folded table index (rows ascending in
    rel, offset Tk-1) is row(rel) = rel + Tk-1.  Integer-exact for every (i, j)."""
    torch, F = _torch()
    npos = 2 * Tk - 1
    cols = torch.arange(npos, dtype=torch.float64).repeat(Tq, 1)
    shifted = refimpl.nemo_rel_shift(cols)[:, :Tk].numpy().astype(np.int64)
    for i in range(Tq):
        for j in range(Tk):
            n = shifted[i, j]
            rel_from_nemo = (Tk - 1) - n
            table_row = rel_from_nemo + (Tk - 1)
            assert table_row == _rel_shift_index(Tq, Tk, i, j)


def _kat_attention_inputs(orc):
    # ConformerOpTests.swift:81-100
    Tq, cache, H, dk = 7, 5, 2, 16
    Tk = cache + Tq
    HD = H * dk
    q = orc.lcg_floats(Tq * HD, 41).reshape(Tq, HD)
    k = orc.lcg_floats(Tk * HD, 42).reshape(Tk, HD)
    v = orc.lcg_floats(Tk * HD, 43).reshape(Tk, HD)
    u = orc.lcg_floats(HD, 44).reshape(H, dk)
    vb = orc.lcg_floats(HD, 45).reshape(H, dk)
    nPos = 2 * Tk - 1
    pe = orc.lcg_floats(nPos * HD, 46).reshape(nPos, HD)
    offset = Tk - 1
    table = np.zeros_like(pe)
    for rel in range(-(Tk - 1), Tk):
        table[rel + offset] = pe[(Tk - 1) - rel]
    ranges = np.array([[max(0, i - 3), min(Tk, cache + i + 2)] for i in range(Tq)], np.int32)
    return dict(Tq=Tq, Tk=Tk, H=H, dk=dk, q=q, k=k, v=v, u=u, vb=vb, pe=pe, table=table, offset=offset,
                ranges=ranges)


def kat_attention_reference(d):
    """ConformerOpTests.swift:111-140: matrix_bd then NeMo's pad/view rel_shift, float64 numpy."""
    Tq, Tk, H, dk = d["Tq"], d["Tk"], d["H"], d["dk"]
    f64 = lambda a, n: a.astype(np.float64).reshape(n, H, dk).transpose(1, 0, 2)
    q, k, v, pe = f64(d["q"], Tq), f64(d["k"], Tk), f64(d["v"], Tk), f64(d["pe"], 2 * Tk - 1)
    u = d["u"].astype(np.float64).reshape(H, 1, dk)
    vb = d["vb"].astype(np.float64).reshape(H, 1, dk)
    ac = (q + u) @ k.transpose(0, 2, 1)
    bd = refimpl.nemo_rel_shift(np.ascontiguousarray((q + vb) @ pe.transpose(0, 2, 1)))[:, :, :Tk]
    s = (ac + bd) / np.sqrt(dk)
    mask = np.ones((Tq, Tk), bool)
    for i, (lo, hi) in enumerate(d["ranges"]):
        mask[i, lo:hi] = False
    s = np.where(mask, -np.inf, s)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    return (p @ v).transpose(1, 0, 2).reshape(Tq, H * dk)


def test_relpos_attention_kat_matches_nemo_rel_shift(orc):
    d = _kat_attention_inputs(orc)
    got = orc.relpos_attention(d["q"], d["k"], d["v"], d["table"], d["u"], d["vb"], d["ranges"], d["offset"], d["H"])
    assert np.abs(got - kat_attention_reference(d)).max() < 1e-5


def test_relpos_attention_invariants(orc):
    d = _kat_attention_inputs(orc)
    # keys outside a query's range carry exactly zero weight: poisoning them changes nothing
    v2 = d["v"].copy()
    k2 = d["k"].copy()
    ranges = np.array([[3, 8]] * d["Tq"], np.int32)
    base = orc.relpos_attention(d["q"], d["k"], d["v"], d["table"], d["u"], d["vb"], ranges, d["offset"], d["H"])
    v2[:3] = 1e30
    v2[8:] = -1e30
    k2[:3] = 7.0
    got = orc.relpos_attention(d["q"], k2, v2, d["table"], d["u"], d["vb"], ranges, d["offset"], d["H"])
    np.testing.assert_array_equal(got, base)
    # a single-key range returns that value row exactly (probability 1)
    one = np.array([[4, 5]] * d["Tq"], np.int32)
    got = orc.relpos_attention(d["q"], d["k"], d["v"], d["table"], d["u"], d["vb"], one, d["offset"], d["H"])
    np.testing.assert_allclose(got, np.repeat(d["v"][4:5], d["Tq"], 0), rtol=1e-6)
    # empty ranges give 0 (20_conformer.metal:212)
    empty = np.array([[5, 5], [6, 2], [0, 0], [11, 11], [12, 40], [-4, 0], [3, 3]], np.int32)
    got = orc.relpos_attention(d["q"], d["k"], d["v"], d["table"], d["u"], d["vb"], empty, d["offset"], d["H"])
    assert not np.any(got)


def _small_model(ud, orc, layers=2, D=64, H=4, ff=128, seed=3):
    cfg = ud.EncoderConfig(layers=layers, d_model=D, heads=H, ff_dim=ff)
    lw = [ud.synthetic_layer_weights(cfg, seed, l, ln_jitter=0.2) for l in range(layers)]
    return cfg, lw


@pytest.mark.parametrize("valid", [20, 15])
def test_encoder_offline_matches_torch_nemo_layer(ud, orc, valid):
    """The oracle's layer composition (encodeLayer) against a torch restatement of NeMo's
    ConformerLayer with library conv1d/layer_norm/softmax and the literal rel_shift."""
    torch, F = _torch()
    T, L, R = 20, 6, 1
    cfg, lw = _small_model(ud, orc)
    D, H = cfg.d_model, cfg.heads
    model = orc.Model(lw, D, H, cfg.ff_dim, 9).prepare(-(T - 1), T - 1)
    x = np.random.default_rng(5).standard_normal((T, D)).astype(np.float32)
    ranges = orc.chunked_limited_ranges(T, L, R)
    ranges[:, 1] = np.minimum(ranges[:, 1], valid)
    got = orc.encoder_offline(model, x, ranges, valid)
    pe_in = refimpl.nemo_pe(T, D)
    mask = refimpl.chunked_limited_mask(T, L, R, valid)
    ref = torch.from_numpy(x).double()
    for l in range(cfg.layers):
        ref = refimpl.layer_nemo(ref, lw[l], pe_in, mask, valid, H)
    ref = ref.numpy()
    # rows >= valid are padding: NeMo hides padded queries entirely, the reference clips key ranges
    # only (FastConformer.swift:380-381); valid rows agree.
    err = np.abs(got[:valid] - ref[:valid]).max() / np.abs(ref[:valid]).max()
    assert err < 1e-5, err


def test_store_limit_matches_clamped_torch_layer(ud, orc):
    """The oracle's storage-range model (orc_set_store_limit) against the torch restatement of
    NeMo's layer with torch.clamp at the same points.  The limit (1.5) is below the typical LayerNorm
    output, FF hidden and q/k/v magnitudes here, so those clamp points engage: a missing or
    misplaced clamp there moves the result far beyond the tolerance (checked by removing the clamp
    on v).  The attention output is a convex combination of clamped V rows, so its clamp never
    engages.  Limit 0 restores the fp32 path."""
    torch, F = _torch()
    T, L, R, valid = 16, 6, 1, 16
    cfg, lw = _small_model(ud, orc, layers=1)
    D, H = cfg.d_model, cfg.heads
    lw[0]["feed_forward1.linear1.weight"] = lw[0]["feed_forward1.linear1.weight"] * 4
    model = orc.Model(lw, D, H, cfg.ff_dim, 9).prepare(-(T - 1), T - 1)
    x = np.random.default_rng(6).standard_normal((T, D)).astype(np.float32)
    ranges = orc.chunked_limited_ranges(T, L, R)
    pe_in = refimpl.nemo_pe(T, D)
    mask = refimpl.chunked_limited_mask(T, L, R, valid)
    xt = torch.from_numpy(x).double()
    ref_clip = refimpl.layer_nemo(xt, lw[0], pe_in, mask, valid, H, clip=1.5).numpy()
    ref_free = refimpl.layer_nemo(xt, lw[0], pe_in, mask, valid, H).numpy()
    with orc.store_limit(1.5):
        got = orc.encoder_offline(model, x, ranges, valid)
    free = orc.encoder_offline(model, x, ranges, valid)
    assert np.abs(ref_clip - ref_free).max() > 0.1           # the clamps change the result
    assert np.abs(got - ref_clip).max() / np.abs(ref_clip).max() < 1e-5
    assert np.abs(free - ref_free).max() / np.abs(ref_free).max() < 1e-5


def test_streaming_equals_offline_chunked(ud, orc):
    """Cache-aware streaming (L cached frames, chunks of T) equals the offline chunked_limited
    forward with [L, T-1] (docs/specs/nemotron.md:197-208), here exactly since there is no
    subsampling edge: pins the cache rule, cache_len masking and the conv cache."""
    torch, F = _torch()
    L, T, steps, S = 6, 2, 6, 2
    cfg, lw = _small_model(ud, orc)
    D, H = cfg.d_model, cfg.heads
    N = T * steps
    xs = np.random.default_rng(9).standard_normal((S, N, D)).astype(np.float32)
    smodel = orc.Model(lw, D, H, cfg.ff_dim, 9).prepare(-(T - 1), L + T - 1)
    kc = np.zeros((S, cfg.layers, L, D), np.float32)
    vc = np.zeros_like(kc)
    cc = np.zeros((S, cfg.layers, 8, D), np.float32)
    cl = np.zeros(S, np.int32)
    outs = []
    for st in range(steps):
        outs.append(orc.stream_step(smodel, xs[:, st * T:(st + 1) * T], np.full(S, T, np.int32), kc, vc, cc, cl))
        assert list(cl) == [min((st + 1) * T, L)] * S
    got = np.concatenate(outs, axis=1)
    pe_in = refimpl.nemo_pe(N, D)
    mask = refimpl.chunked_limited_mask(N, L, T - 1, N)
    for s in range(S):
        ref = torch.from_numpy(xs[s]).double()
        for l in range(cfg.layers):
            ref = refimpl.layer_nemo(ref, lw[l], pe_in, mask, N, H)
        err = np.abs(got[s] - ref.numpy()).max() / np.abs(ref.numpy()).max()
        assert err < 1e-5, err


def test_stream_cache_rule(ud, orc):
    """After a step the K cache equals the last L rows of [previous cache ; this chunk's K
    projection]: checked by re-deriving layer 0's new K rows from its input.  The conv cache is the
    last K-1 rows of [previous conv cache ; this chunk's GLU rows] with the rows at and past the
    valid count zeroed (maskRows, FastConformer.swift:302, 470-472): here the chunk's last row."""
    L, T, S = 6, 4, 1
    cfg, lw = _small_model(ud, orc, layers=1)
    D, H = cfg.d_model, cfg.heads
    smodel = orc.Model(lw, D, H, cfg.ff_dim, 9).prepare(-(T - 1), L + T - 1)
    rng = np.random.default_rng(2)
    kc = rng.standard_normal((S, 1, L, D)).astype(np.float32)
    vc = rng.standard_normal((S, 1, L, D)).astype(np.float32)
    cc = rng.standard_normal((S, 1, 8, D)).astype(np.float32)
    cl = np.array([1], np.int32)
    x = rng.standard_normal((S, T, D)).astype(np.float32)
    k0, c0 = kc.copy(), cc.copy()
    orc.stream_step(smodel, x, np.array([T - 1], np.int32), kc, vc, cc, cl)
    w = lw[0]
    r1 = x[0] + 0.5 * orc.gemm_nt(orc.gemm_nt(orc.layer_norm(x[0], w["norm_feed_forward1.weight"],
                                                             w["norm_feed_forward1.bias"]),
                                              w["feed_forward1.linear1.weight"], act=orc.ACT_SILU),
                                  w["feed_forward1.linear2.weight"])
    knew = orc.gemm_nt(orc.layer_norm(r1, w["norm_self_att.weight"], w["norm_self_att.bias"]),
                       w["self_attn.linear_k.weight"])
    np.testing.assert_array_equal(kc[0, 0, :L - T], k0[0, 0, T:])
    np.testing.assert_allclose(kc[0, 0, L - T:], knew, rtol=1e-5, atol=1e-5)
    assert cl[0] == 1 + T                   # advances by T, not by the valid count (FastConformer.swift:477)
    np.testing.assert_array_equal(cc[0, 0, :8 - T], c0[0, 0, T:])
    np.testing.assert_array_equal(cc[0, 0, 7], 0.0)                 # the masked GLU row
    assert np.all(np.abs(cc[0, 0, 8 - T:7]).max(axis=1) > 0)          # the valid GLU rows
