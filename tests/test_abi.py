"""CPU checks of the C ABI boundary and the host binding: the library loads, exports every
function the public headers declare, and the binding refuses to run without a HIP device (no
CPU fallback)."""
import ctypes
import glob
import os
import re

import numpy as np
import pytest

from conftest import ROOT


def _declared():
    names = []
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        src = open(h).read()
        names += re.findall(r"UD_API\s+[\w\s\*]+?\b(ud_\w+)\s*\(", src)
    return sorted(set(names))


def test_headers_declare_the_boundary():
    names = _declared()
    for must in ("ud_encoder_create", "ud_encoder_set_weight", "ud_encoder_finalize", "ud_stream_create",
                 "ud_encoder_step", "ud_stream_export_cache", "ud_stream_import_cache", "ud_relpos_attention",
                 "ud_last_error", "ud_malloc", "ud_event_elapsed_ms"):
        assert must in names


def test_library_exports_every_declared_symbol(ud):
    lib = ud.load_library()
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_library_is_gfx950_only():
    # the fat binary in the library carries a gfx950 code object and no other target
    data = open(os.path.join(ROOT, "universal-dictator_amd", "lib", "libud_encoder.so"), "rb").read()
    assert b"gfx950" in data
    for other in (b"gfx942", b"gfx90a", b"gfx1100", b"sm_"):
        assert other + b"\x00" not in data and b"amdgcn-amd-amdhsa--" + other not in data


def test_no_device_means_error_not_fallback(ud):
    lib = ud.load_library()
    n = ctypes.c_int32(0)
    lib.ud_device_count(ctypes.byref(n))
    if n.value > 0:
        pytest.skip("a HIP device is present")
    with pytest.raises(ud.EngineError):
        ud.lib()
    with pytest.raises(ud.EngineError):
        ud.Encoder(ud.EncoderConfig(layers=1))


def test_host_bf16_rounding_matches_oracle(ud, orc):
    rng = np.random.default_rng(4)
    x = (rng.standard_normal(100000) * 10.0 ** rng.integers(-30, 30, 100000)).astype(np.float32)
    x = np.concatenate([x, np.array([np.inf, -np.inf, 0.0, -0.0, 1.00390625, 3.4e38], np.float32)])
    np.testing.assert_array_equal(ud.round_bf16(x), orc.round_bf16(x))


def test_synthetic_weights_shapes(ud):
    cfg = ud.EncoderConfig(layers=1)
    w = ud.synthetic_layer_weights(cfg, 0, 0)
    assert set(w) == set(ud.LAYER_WEIGHT_SUFFIXES)
    assert w["feed_forward1.linear1.weight"].shape == (4096, 1024)
    assert w["conv.pointwise_conv1.weight"].shape == (2048, 1024)
    assert w["conv.depthwise_conv.weight"].shape == (1024, 9)
    assert w["self_attn.pos_bias_u"].shape == (8, 128)
    b = np.sqrt(6.0 / 5120)
    assert np.abs(w["feed_forward1.linear1.weight"]).max() <= b
    w2 = ud.synthetic_layer_weights(cfg, 0, 0)
    np.testing.assert_array_equal(w["self_attn.linear_q.weight"], w2["self_attn.linear_q.weight"])
