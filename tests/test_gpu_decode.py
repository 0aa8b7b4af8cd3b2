"""GPU parity of the decoder attention entry points (include/ud_decode.h) through the C ABI:
paged grouped-query attention against the oracle on the gathered contiguous K/V (the reference
KAT with f16 caches, random page tables, group sizes 1..8, head_dim 64/128, window starts, empty
ranges, the 64-sequence decode shape), the paged append bit-exact, RoPE against the oracle."""
import numpy as np
import pytest

from test_oracle_decode import _f16
import harness

pytestmark = pytest.mark.gpu

PAGE = 16


def _bits16(a, kv_dtype):
    if kv_dtype == "f16":
        return np.ascontiguousarray(a.astype(np.float16)).view(np.uint16)
    return (np.ascontiguousarray(a, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


def _from16(bits, kv_dtype):
    if kv_dtype == "f16":
        return bits.view(np.float16).astype(np.float32)
    return (bits.astype(np.uint32) << 16).view(np.float32)


def build_pages(seqs, Hkv, d, rng, spare=3):
    """Paged cache holding the given per-sequence K (or V) arrays [len_i, Hkv*d] (16-bit bits),
    pages shuffled, plus `spare` never-referenced pages filled with NaN bit patterns."""
    max_blocks = max((len(s) + PAGE - 1) // PAGE for s in seqs) + 1
    nblk = sum((len(s) + PAGE - 1) // PAGE for s in seqs) + spare
    perm = rng.permutation(nblk)
    pages = np.full((nblk, Hkv, PAGE, d), 0x7FFF, np.uint16)     # NaN in both bf16 and f16
    table = np.full((len(seqs), max_blocks), -1, np.int32)        # unused entries: invalid
    nxt = 0
    for i, s in enumerate(seqs):
        for b in range((len(s) + PAGE - 1) // PAGE):
            phys = int(perm[nxt]); nxt += 1
            table[i, b] = phys
            rows = s[b * PAGE:(b + 1) * PAGE].reshape(-1, Hkv, d)
            pages[phys, :, :len(rows), :] = rows.transpose(1, 0, 2)
    return pages, table, max_blocks


def run_paged(ud, q, kseqs, vseqs, ranges, Hq, Hkv, d, kv_dtype, rng):
    n = len(kseqs)
    kb = [_bits16(k, kv_dtype) for k in kseqs]
    vb = [_bits16(v, kv_dtype) for v in vseqs]
    state = np.random.default_rng(int(rng.integers(1 << 30)))
    kp, table, max_blocks = build_pages(kb, Hkv, d, state)
    vp = np.full_like(kp, 0x7FFF)        # V pages follow K's page assignment
    for i, s in enumerate(vb):
        for b in range((len(s) + PAGE - 1) // PAGE):
            rows = s[b * PAGE:(b + 1) * PAGE].reshape(-1, Hkv, d)
            vp[table[i, b], :, :len(rows), :] = rows.transpose(1, 0, 2)
    max_keys = int(max(1, ranges[:, 1].max()))
    dev = ud.DeviceBuffer.from_numpy
    ws = ud.DeviceBuffer.zeros(max(16, ud.gqa_workspace_bytes(n, Hq, d, max_keys)))
    out = ud.DeviceBuffer(n * Hq * d * 4)
    ud.gqa_attention_paged(dev(np.ascontiguousarray(q, np.float32)), dev(kp), dev(vp), dev(table), max_blocks,
                           dev(np.ascontiguousarray(ranges, np.int32)), out, n, Hq, Hkv, d, max_keys, ws,
                           kv_dtype=kv_dtype)
    ud.synchronize()
    return out.download((n, Hq * d))


def oracle_paged(orc, q, kseqs, vseqs, ranges, Hq, Hkv, kv_dtype):
    out = []
    for i in range(len(kseqs)):
        k = _from16(_bits16(kseqs[i], kv_dtype), kv_dtype)
        v = _from16(_bits16(vseqs[i], kv_dtype), kv_dtype)
        out.append(orc.gqa_attention(q[i:i + 1], k, v, ranges[i:i + 1], Hq, Hkv)[0])
    return np.stack(out)


def test_paged_gqa_reference_kat_f16(gpu, orc):
    """VoxtralOpTests.swift:6-38 through the page table: the three queries become three sequences
    that share one paged f16 cache; tolerance 2e-5 as in the reference."""
    ud = gpu
    Tq, Tk, Hq, Hkv, d = 3, 1200, 8, 2, 64
    q = orc.lcg_floats(Tq * Hq * d, 51).reshape(Tq, Hq * d)
    k = _f16(orc.lcg_floats(Tk * Hkv * d, 52)).reshape(Tk, Hkv * d)
    v = _f16(orc.lcg_floats(Tk * Hkv * d, 53)).reshape(Tk, Hkv * d)
    ranges = np.array([[0, 1200], [450, 1100], [700, 701]], np.int32)
    got = run_paged(ud, q, [k] * 3, [v] * 3, ranges, Hq, Hkv, d, "f16", np.random.default_rng(1))
    ref = orc.gqa_attention(q, k, v, ranges, Hq, Hkv)
    assert np.abs(got - ref).max() < 2e-5


@pytest.mark.parametrize("Hq,Hkv,d,kv_dtype", [(32, 8, 128, "bf16"), (8, 8, 64, "bf16"), (16, 8, 128, "f16"),
                                               (16, 2, 64, "bf16"), (8, 4, 128, "bf16"), (8, 8, 128, "bf16"),
                                               (64, 8, 128, "bf16")])
def test_paged_gqa_ragged(gpu, orc, Hq, Hkv, d, kv_dtype):
    """Ragged lengths across split and page boundaries (1, 15, 16, 17, 255, 256, 257, 700), a window
    start, an empty range; pages shuffled, unused pages full of NaN."""
    ud = gpu
    rng = np.random.default_rng(Hq * 1000 + d)
    lens = [1, 15, 16, 17, 255, 256, 257, 700, 300, 40]
    n = len(lens)
    kseqs = [rng.standard_normal((L, Hkv * d)).astype(np.float32) for L in lens]
    vseqs = [rng.standard_normal((L, Hkv * d)).astype(np.float32) for L in lens]
    ranges = np.array([[0, L] for L in lens], np.int32)
    ranges[8] = [137, 300]          # window start inside a page
    ranges[9] = [20, 20]            # empty
    q = rng.standard_normal((n, Hq * d)).astype(np.float32)
    got = run_paged(ud, q, kseqs, vseqs, ranges, Hq, Hkv, d, kv_dtype, rng)
    ref = oracle_paged(orc, q, kseqs, vseqs, ranges, Hq, Hkv, kv_dtype)
    assert not np.any(got[9])
    if kv_dtype == "f16":
        # f16 pages: fp32 arithmetic on the widened K/V, as the reference kernel
        assert np.abs(got - ref).max() < 1e-4
    else:
        # bf16 pages: packed bf16 dot products (q and the probabilities rounded to bf16)
        harness.assert_bf16_close(got, ref, "paged gqa %s" % kv_dtype)


@pytest.mark.parametrize("d,kv_dtype", [(64, "bf16"), (64, "f16"), (128, "bf16")])
def test_paged_gqa_long_context(gpu, orc, d, kv_dtype):
    """Contexts past 64 splits (the combine merges them 64 at a time; 128-key splits, 256-key on the
    MFMA path of bf16 pages at head_dim 128): 17,000 and 9,000 keys, a window [5,000, 13,100)
    whose first and last splits are partial, and a 300-key sequence in the same call."""
    ud = gpu
    rng = np.random.default_rng(61 + d)
    Hq, Hkv = 8, 2
    lens = [17000, 9000, 300, 13100]
    n = len(lens)
    kseqs = [rng.standard_normal((L, Hkv * d)).astype(np.float32) for L in lens]
    vseqs = [rng.standard_normal((L, Hkv * d)).astype(np.float32) for L in lens]
    ranges = np.array([[0, L] for L in lens], np.int32)
    ranges[3] = [5000, 13100]
    q = rng.standard_normal((n, Hq * d)).astype(np.float32)
    got = run_paged(ud, q, kseqs, vseqs, ranges, Hq, Hkv, d, kv_dtype, rng)
    ref = oracle_paged(orc, q, kseqs, vseqs, ranges, Hq, Hkv, kv_dtype)
    if kv_dtype == "f16":
        assert np.abs(got - ref).max() < 1e-4
    else:
        harness.assert_bf16_close(got, ref, "long context")


def test_paged_gqa_decode_shape(gpu, orc):
    """The 64-sequence decode step: 32 query heads on 8 kv heads x 128, context lengths uniform in
    512..4096, bf16 pages of 16."""
    ud = gpu
    rng = np.random.default_rng(55)
    n, Hq, Hkv, d = 64, 32, 8, 128
    lens = rng.integers(512, 4097, n)
    kseqs = [rng.standard_normal((int(L), Hkv * d)).astype(np.float32) for L in lens]
    vseqs = [rng.standard_normal((int(L), Hkv * d)).astype(np.float32) for L in lens]
    ranges = np.stack([np.zeros(n, np.int32), lens.astype(np.int32)], 1)
    q = rng.standard_normal((n, Hq * d)).astype(np.float32)
    got = run_paged(ud, q, kseqs, vseqs, ranges, Hq, Hkv, d, "bf16", rng)
    ref = oracle_paged(orc, q, kseqs, vseqs, ranges, Hq, Hkv, "bf16")
    harness.assert_bf16_close(got, ref, "decode shape")


def test_paged_append_bit_exact(gpu):
    ud = gpu
    rng = np.random.default_rng(9)
    n, Hkv, d, max_blocks, nblk = 5, 8, 128, 4, 24
    kp = rng.integers(0, 1 << 16, (nblk, Hkv, PAGE, d), dtype=np.uint16)
    vp = rng.integers(0, 1 << 16, (nblk, Hkv, PAGE, d), dtype=np.uint16)
    table = rng.permutation(nblk)[:n * max_blocks].reshape(n, max_blocks).astype(np.int32)
    pos = np.array([0, 15, 16, 33, 63], np.int32)
    kn = rng.integers(0, 1 << 16, (n, Hkv * d), dtype=np.uint16)
    vn = rng.integers(0, 1 << 16, (n, Hkv * d), dtype=np.uint16)
    dev = ud.DeviceBuffer.from_numpy
    kpd, vpd = dev(kp), dev(vp)
    ud.paged_kv_append(dev(kn), dev(vn), kpd, vpd, dev(table), max_blocks, dev(pos), n, Hkv, d)
    ud.synchronize()
    k2 = kpd.download(kp.shape, np.uint16)
    v2 = vpd.download(vp.shape, np.uint16)
    wk, wv = kp.copy(), vp.copy()
    for i in range(n):
        phys, row = table[i, pos[i] // PAGE], pos[i] % PAGE
        wk[phys, :, row, :] = kn[i].reshape(Hkv, d)
        wv[phys, :, row, :] = vn[i].reshape(Hkv, d)
    np.testing.assert_array_equal(k2, wk)
    np.testing.assert_array_equal(v2, wv)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_rope_matches_oracle(gpu, orc, dtype):
    ud = gpu
    rng = np.random.default_rng(21)
    T, H, d, ld = 7, 8, 128, 8 * 128 + 64
    x = rng.standard_normal((T, ld)).astype(np.float32)
    pos = rng.integers(0, 4096, T).astype(np.int32)
    inv = ud.rope_inv_freq(d, 1e6)
    if dtype == "bf16":
        x = ud.round_bf16(x)
        buf = ud.DeviceBuffer.from_numpy((x.view(np.uint32) >> 16).astype(np.uint16))
    else:
        buf = ud.DeviceBuffer.from_numpy(x)
    ud.rope_rotate_half(buf, T, H, d, ld, ud.DeviceBuffer.from_numpy(inv), positions=ud.DeviceBuffer.from_numpy(pos),
                        dtype=dtype)
    ud.synchronize()
    ref = orc.rope_rotate_half(x, H, d, inv, positions=pos)
    if dtype == "f32":
        got = buf.download((T, ld))
        assert np.abs(got - ref).max() < 1e-5
    else:
        got = (buf.download((T, ld), np.uint16).astype(np.uint32) << 16).view(np.float32)
        assert np.abs(got - ref).max() <= np.abs(ref).max() * 2.0 ** -8


def test_decode_error_paths(gpu):
    ud = gpu
    b = ud.DeviceBuffer(1 << 16)
    with pytest.raises(ud.EngineError):        # group 3 unsupported
        ud.gqa_attention_paged(b, b, b, b, 4, b, b, 1, 6, 2, 128, 64, b)
    with pytest.raises(ud.EngineError):        # head_dim 96 unsupported
        ud.gqa_attention_paged(b, b, b, b, 4, b, b, 1, 8, 2, 96, 64, b)
    small = ud.DeviceBuffer(16)
    with pytest.raises(ud.EngineError):        # workspace too small
        ud.gqa_attention_paged(b, b, b, b, 4, b, b, 1, 8, 2, 128, 64, small)
    with pytest.raises(ud.EngineError):        # max_keys beyond the page table
        ud.gqa_attention_paged(b, b, b, b, 4, b, b, 1, 8, 2, 128, 65, b)
    with pytest.raises(ud.EngineError):        # more than 65535 splits of 128 keys (grid y)
        ud.gqa_attention_paged(b, b, b, b, 1 << 20, b, b, 1, 8, 2, 128, 65535 * 128 + 1, b)
    with pytest.raises(ud.EngineError):        # more than 65535 sequences (grid z)
        ud.gqa_attention_paged(b, b, b, b, 4, b, b, 65536, 8, 2, 128, 64, b)
