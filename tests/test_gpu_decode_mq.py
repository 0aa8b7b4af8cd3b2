"""GPU parity of the multi-query decode attention (ud_gqa_attention_paged_mq): 1 .. 8 query rows
per sequence, each with its own key range, every K/V page read once for all of them (the
reference's attention_mq_split, Sources/DictatorEngine/Metal/30_voxtral.metal:240-338, dispatched
for 1 < Tq <= 8 by Core/Ops.swift:141-162).  Checked against the oracle (orc_gqa_attention takes
several queries with their own ranges) and against one call per query: the reference's own KAT
(Tests/DictatorEngineTests/VoxtralOpTests.swift:42-59, multi-query equals per-query), the paged
decode benchmark's heads and contexts at 4 queries per sequence, and every tile shape of the MFMA kernel (4 .. 64
query rows per kv head) and of the VALU kernel."""
import numpy as np
import pytest

import harness
from test_gpu_decode import PAGE, _bits16, _from16, build_pages
from test_oracle_decode import _f16

pytestmark = pytest.mark.gpu


def _pages(ud, kseqs, vseqs, Hkv, d, kv_dtype, rng):
    kb = [_bits16(k, kv_dtype) for k in kseqs]
    vb = [_bits16(v, kv_dtype) for v in vseqs]
    kp, table, max_blocks = build_pages(kb, Hkv, d, np.random.default_rng(int(rng.integers(1 << 30))))
    vp = np.full_like(kp, 0x7FFF)        # V pages follow K's page assignment; unused pages NaN
    for i, s in enumerate(vb):
        for b in range((len(s) + PAGE - 1) // PAGE):
            rows = s[b * PAGE:(b + 1) * PAGE].reshape(-1, Hkv, d)
            vp[table[i, b], :, :len(rows), :] = rows.transpose(1, 0, 2)
    dev = ud.DeviceBuffer.from_numpy
    return dev(kp), dev(vp), dev(table), max_blocks


def run_mq(ud, q, pages, ranges, Hq, Hkv, d, kv_dtype):
    """q [n, M, Hq*d], ranges [n, M, 2] -> out [n, M, Hq*d] from one multi-query call."""
    kp, vp, table, max_blocks = pages
    n, M = q.shape[:2]
    max_keys = int(max(1, ranges[..., 1].max()))
    dev = ud.DeviceBuffer.from_numpy
    ws = ud.DeviceBuffer.zeros(max(16, ud.gqa_workspace_bytes(n * M, Hq, d, max_keys)))
    out = ud.DeviceBuffer(n * M * Hq * d * 4)
    ud.gqa_attention_paged_mq(dev(np.ascontiguousarray(q, np.float32)), kp, vp, table, max_blocks,
                              dev(np.ascontiguousarray(ranges, np.int32)), out, n, M, Hq, Hkv, d, max_keys, ws,
                              kv_dtype=kv_dtype)
    ud.synchronize()
    return out.download((n, M, Hq * d))


def run_per_query(ud, q, pages, ranges, Hq, Hkv, d, kv_dtype):
    """The same queries one at a time (a one-query call per position m)."""
    return np.stack([run_mq(ud, q[:, m:m + 1], pages, ranges[:, m:m + 1], Hq, Hkv, d, kv_dtype)[:, 0]
                     for m in range(q.shape[1])], axis=1)


def oracle_mq(orc, q, kseqs, vseqs, ranges, Hq, Hkv, kv_dtype):
    out = []
    for i in range(len(kseqs)):
        k = _from16(_bits16(kseqs[i], kv_dtype), kv_dtype)
        v = _from16(_bits16(vseqs[i], kv_dtype), kv_dtype)
        out.append(orc.gqa_attention(q[i], k, v, ranges[i], Hq, Hkv))
    return np.stack(out)


def test_mq_reference_kat(gpu, orc):
    """VoxtralOpTests.swift:42-59: 4 queries, 32 heads x 64 (one kv head per query head), f16 caches
    of 700 keys, causal-window ranges [m, 697 + m); the multi-query result equals the per-query one
    within 1e-5 (here: exactly, the rows are independent in every product) and the oracle within
    the f16-page tolerance."""
    ud = gpu
    Tq, Tk, H, d = 4, 700, 32, 64
    q = orc.lcg_floats(Tq * H * d, 55).reshape(1, Tq, H * d)
    k = _f16(orc.lcg_floats(Tk * H * d, 56)).reshape(Tk, H * d)
    v = _f16(orc.lcg_floats(Tk * H * d, 57)).reshape(Tk, H * d)
    ranges = np.array([[[0, 697], [1, 698], [2, 699], [3, 700]]], np.int32)
    pages = _pages(ud, [k], [v], H, d, "f16", np.random.default_rng(1))
    got = run_mq(ud, q, pages, ranges, H, H, d, "f16")
    per = run_per_query(ud, q, pages, ranges, H, H, d, "f16")
    assert np.abs(got - per).max() <= 1e-5
    np.testing.assert_array_equal(got, per)
    ref = oracle_mq(orc, q, [k], [v], ranges, H, H, "f16")
    assert np.abs(got - ref).max() < 1e-4


def test_mq_decode_shape_four_queries(gpu, orc):
    """The paged decode benchmark's heads and contexts (64 sequences, 32 query / 8 kv heads x 128, contexts uniform
    in 512..4096, bf16 pages of 16) at 4 new positions per sequence: query m sees keys
    [0, ctx - 3 + m) (causal over the new tokens), a sliding-window start on every fifth sequence."""
    ud = gpu
    rng = np.random.default_rng(56)
    n, M, Hq, Hkv, d = 64, 4, 32, 8, 128
    lens = rng.integers(512, 4097, n)
    kseqs = [rng.standard_normal((int(L), Hkv * d)).astype(np.float32) for L in lens]
    vseqs = [rng.standard_normal((int(L), Hkv * d)).astype(np.float32) for L in lens]
    ranges = np.zeros((n, M, 2), np.int32)
    for i, L in enumerate(lens):
        for m in range(M):
            ranges[i, m] = [0 if i % 5 else 300 + 7 * m, L - (M - 1) + m]
    q = rng.standard_normal((n, M, Hq * d)).astype(np.float32)
    pages = _pages(ud, kseqs, vseqs, Hkv, d, "bf16", rng)
    got = run_mq(ud, q, pages, ranges, Hq, Hkv, d, "bf16")
    np.testing.assert_array_equal(got, run_per_query(ud, q, pages, ranges, Hq, Hkv, d, "bf16"))
    harness.assert_bf16_close(got, oracle_mq(orc, q, kseqs, vseqs, ranges, Hq, Hkv, "bf16"), "decode shape, 4 queries")


@pytest.mark.parametrize("Hq,Hkv,d,kv_dtype,M", [
    (64, 8, 128, "bf16", 8),    # 64 query rows per kv head: four 16-row MFMA tiles
    (64, 8, 128, "bf16", 5),    # 40 rows: three tiles, the last partly padding
    (32, 8, 128, "bf16", 3),    # 12 rows: one tile
    (32, 8, 128, "bf16", 6),    # 24 rows: two tiles
    (16, 8, 128, "bf16", 8),    # 16 rows, group 2
    (8, 8, 128, "bf16", 7),     # group 1
    (16, 8, 128, "f16", 3),     # f16 pages: the VALU kernel, K/V in registers across the queries
    (16, 2, 64, "bf16", 8),     # head_dim 64: the VALU kernel
])
def test_mq_tile_shapes(gpu, orc, Hq, Hkv, d, kv_dtype, M):
    """Ranges per query across split (256 / 128 keys) and page boundaries: full contexts, windows,
    an empty range (output 0), single keys, and a sequence whose queries' ranges leave a gap."""
    ud = gpu
    rng = np.random.default_rng(Hq * 100 + M * 10 + d)
    lens = [1, 17, 256, 257, 700, 1300, 40, 513]
    n = len(lens)
    kseqs = [rng.standard_normal((L, Hkv * d)).astype(np.float32) for L in lens]
    vseqs = [rng.standard_normal((L, Hkv * d)).astype(np.float32) for L in lens]
    ranges = np.zeros((n, M, 2), np.int32)
    for i, L in enumerate(lens):
        for m in range(M):
            ranges[i, m] = [0, max(1, L - (M - 1) + m)]
    ranges[4, :, 0] = 137                        # window start inside a page
    ranges[5, 0] = [600, 1290]
    ranges[5, M - 1] = [1299, 1300]              # a single key
    ranges[6, M // 2] = [20, 20]                 # empty
    ranges[7, 0] = [0, 100]                      # a gap: [100, 400) in no query's range
    ranges[7, 1:] = [400, 513]
    q = rng.standard_normal((n, M, Hq * d)).astype(np.float32)
    pages = _pages(ud, kseqs, vseqs, Hkv, d, kv_dtype, rng)
    got = run_mq(ud, q, pages, ranges, Hq, Hkv, d, kv_dtype)
    assert not np.any(got[6, M // 2])
    np.testing.assert_array_equal(got, run_per_query(ud, q, pages, ranges, Hq, Hkv, d, kv_dtype))
    ref = oracle_mq(orc, q, kseqs, vseqs, ranges, Hq, Hkv, kv_dtype)
    if kv_dtype == "f16":
        assert np.abs(got - ref).max() < 1e-4
    else:
        harness.assert_bf16_close(got, ref, "mq %d x %d/%d" % (M, Hq, Hkv))


def test_mq_error_paths(gpu):
    ud = gpu
    b = ud.DeviceBuffer(1 << 16)
    with pytest.raises(ud.EngineError) as e:      # 9 queries per sequence
        ud.gqa_attention_paged_mq(b, b, b, b, 4, b, b, 1, 9, 8, 2, 128, 64, b)
    assert e.value.status == -2
    with pytest.raises(ud.EngineError) as e:      # 0 queries
        ud.gqa_attention_paged_mq(b, b, b, b, 4, b, b, 1, 0, 8, 2, 128, 64, b)
    assert e.value.status == -2
    small = ud.DeviceBuffer(ud.gqa_workspace_bytes(2, 8, 128, 64))
    with pytest.raises(ud.EngineError) as e:      # workspace sized for n, not n x queries
        ud.gqa_attention_paged_mq(b, b, b, b, 4, b, b, 2, 4, 8, 2, 128, 64, small)
    assert e.value.status == -2
    with pytest.raises(ud.EngineError) as e:      # n x queries beyond the combine grid
        ud.gqa_attention_paged_mq(b, b, b, b, 4, b, b, 10000, 8, 8, 2, 128, 64, b)
    assert e.value.status == -2
