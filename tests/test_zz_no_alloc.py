"""The allocation-free decode entry point (ud_gqa_attention_paged_noalloc) against the workspace
entry point it varies (ud_gqa_attention_paged), through the C ABI: two calls in a row on the same
device, the second with a smaller input, each bit-identical to the workspace call on the same
inputs (the two share their kernels), plus the refusal of a call whose partials exceed the static
scratch."""
import numpy as np
import pytest

from test_gpu_decode import _bits16, build_pages

pytestmark = pytest.mark.gpu


def _case(ud, rng, n, Hq, Hkv, d, lo, hi, kv_dtype):
    lens = rng.integers(lo, hi + 1, size=n)
    kseqs = [rng.standard_normal((int(L), Hkv * d)).astype(np.float32) for L in lens]
    vseqs = [rng.standard_normal((int(L), Hkv * d)).astype(np.float32) for L in lens]
    kb = [_bits16(k, kv_dtype) for k in kseqs]
    vb = [_bits16(v, kv_dtype) for v in vseqs]
    kp, table, max_blocks = build_pages(kb, Hkv, d, np.random.default_rng(int(rng.integers(1 << 30))))
    vp = np.full_like(kp, 0x7FFF)
    for i, s in enumerate(vb):
        for b in range((len(s) + 15) // 16):
            rows = s[b * 16:(b + 1) * 16].reshape(-1, Hkv, d)
            vp[table[i, b], :, :len(rows), :] = rows.transpose(1, 0, 2)
    # ranges: a window start on some sequences, the full context on the rest
    starts = np.where(rng.random(n) < 0.3, rng.integers(0, np.maximum(lens // 2, 1)), 0)
    ranges = np.stack([starts, lens], axis=1).astype(np.int32)
    q = rng.standard_normal((n, Hq * d)).astype(np.float32)
    dev = ud.DeviceBuffer.from_numpy
    return dict(q=dev(q), kp=dev(kp), vp=dev(vp), table=dev(table), max_blocks=max_blocks,
                ranges=dev(ranges), n=n, Hq=Hq, Hkv=Hkv, d=d, max_keys=int(lens.max()), kv_dtype=kv_dtype)


def _run(ud, c, noalloc):
    out = ud.DeviceBuffer(c["n"] * c["Hq"] * c["d"] * 4)
    args = (c["q"], c["kp"], c["vp"], c["table"], c["max_blocks"], c["ranges"], out, c["n"], c["Hq"], c["Hkv"],
            c["d"], c["max_keys"])
    if noalloc:
        ud.gqa_attention_paged_noalloc(*args, kv_dtype=c["kv_dtype"])
    else:
        ws = ud.DeviceBuffer.zeros(max(16, ud.gqa_workspace_bytes(c["n"], c["Hq"], c["d"], c["max_keys"])))
        ud.gqa_attention_paged(*args, ws, kv_dtype=c["kv_dtype"])
    ud.synchronize()
    return out.download((c["n"], c["Hq"] * c["d"]))


def test_noalloc_matches_workspace_entry_twice(gpu):
    ud = gpu
    rng = np.random.default_rng(20261202)
    # call 1: the decode shape's heads (32 query / 8 kv, head_dim 128) with contexts up to 4096
    big = _case(ud, rng, 24, 32, 8, 128, 512, 4096, "bf16")
    need = ud.gqa_workspace_bytes(big["n"], big["Hq"], big["d"], big["max_keys"])
    assert need <= ud.GQA_NOALLOC_SCRATCH_BYTES
    print("noalloc call 1: n=24 Hq=32 Hkv=8 d=128 max_keys=%d, %d scratch bytes" % (big["max_keys"], need), flush=True)
    got1 = _run(ud, big, True)
    ref1 = _run(ud, big, False)
    assert np.isfinite(got1).all()
    np.testing.assert_array_equal(got1, ref1)
    # call 2, right after on the same device: fewer sequences, shorter contexts, f16 pages and
    # head_dim 64 -- the scratch still holds call 1's partials
    small = _case(ud, rng, 5, 8, 2, 64, 1, 700, "f16")
    print("noalloc call 2: n=5 Hq=8 Hkv=2 d=64 max_keys=%d" % small["max_keys"], flush=True)
    got2 = _run(ud, small, True)
    ref2 = _run(ud, small, False)
    assert np.isfinite(got2).all()
    np.testing.assert_array_equal(got2, ref2)
    # and the large call again after the small one
    np.testing.assert_array_equal(_run(ud, big, True), ref1)


def test_noalloc_allocates_nothing_and_replays_from_a_graph(gpu):
    """What the entry point is for: after one warm-up call on a stream, a second call there leaves
    the device's free memory unchanged (hipMemGetInfo before and after), and the call captured into
    a HIP graph replays to the eager result -- three replays, each after the output is overwritten
    and after a different eager call has reused the shared scratch."""
    ud = gpu
    rng = np.random.default_rng(20261203)
    c = _case(ud, rng, 16, 32, 8, 128, 512, 4096, "bf16")
    other = _case(ud, rng, 3, 8, 2, 64, 1, 500, "f16")
    ref = _run(ud, c, False)
    hs = ud.HipStream()
    out = ud.DeviceBuffer(c["n"] * c["Hq"] * c["d"] * 4)
    args = (c["q"], c["kp"], c["vp"], c["table"], c["max_blocks"], c["ranges"], out, c["n"], c["Hq"], c["Hkv"],
            c["d"], c["max_keys"])
    ud.gqa_attention_paged_noalloc(*args, kv_dtype="bf16", hip_stream=hs)       # warm-up on this stream
    hs.synchronize()
    free0, _ = ud.mem_get_info()
    ud.gqa_attention_paged_noalloc(*args, kv_dtype="bf16", hip_stream=hs)
    hs.synchronize()
    free1, _ = ud.mem_get_info()
    assert free1 == free0, "free device memory changed by %d bytes" % (free0 - free1)
    np.testing.assert_array_equal(out.download(ref.shape), ref)
    with ud.Graph.capture(hs) as g:
        ud.gqa_attention_paged_noalloc(*args, kv_dtype="bf16", hip_stream=hs)
    for r in range(3):
        ud.lib().ud_memset(out.ptr, 0xFF, out.nbytes)                           # NaN bit patterns
        _run(ud, other, True)                                                   # the scratch reused eagerly
        g.launch(hs)
        hs.synchronize()
        np.testing.assert_array_equal(out.download(ref.shape), ref, err_msg="replay %d" % r)


def test_noalloc_refuses_beyond_scratch(gpu):
    """A call whose partials would exceed the static scratch fails with UD_ERR_SHAPE before any
    launch (64 sequences x 32 heads x 8192 keys at head_dim 128 need 65 MiB)."""
    ud = gpu
    n, Hq, Hkv, d, max_keys = 64, 32, 8, 128, 8192
    assert ud.gqa_workspace_bytes(n, Hq, d, max_keys) > ud.GQA_NOALLOC_SCRATCH_BYTES
    q = ud.DeviceBuffer(n * Hq * d * 4)
    pages = ud.DeviceBuffer(16 * Hkv * 16 * d * 2)
    table = ud.DeviceBuffer.from_numpy(np.zeros((n, max_keys // 16), np.int32))
    ranges = ud.DeviceBuffer.from_numpy(np.zeros((n, 2), np.int32))
    out = ud.DeviceBuffer(n * Hq * d * 4)
    with pytest.raises(ud.EngineError) as ei:
        ud.gqa_attention_paged_noalloc(q, pages, pages, table, max_keys // 16, ranges, out, n, Hq, Hkv, d, max_keys)
    assert ei.value.status == -2
    assert "scratch" in str(ei.value)
