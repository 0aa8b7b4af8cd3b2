"""Pins the oracle's subsampling front-end (orc_conv2d_cl, orc_subsample) against library routines:
torch's conv2d on the reference conv2d KAT shapes, and a torch restatement of NeMo's causal
dw_striding ConvSubsampling (tests/refimpl.py) that flattens channel-major into the checkpoint's
out.weight, so a wrong pad side, stride-length rule, mask stage or flatten order fails here."""
import numpy as np
import pytest

import refimpl
from conftest import load_pkg


def _torch():
    import torch
    import torch.nn.functional as F
    return torch, F


@pytest.mark.parametrize("groups,pad", [(1, 2), (4, 1)])
def test_conv2d_reference_kat_against_torch(orc, groups, pad):
    """ConformerOpTests.swift:49-78: 9 x 13 x 4 -> 4 channels, stride 2, ReLU, last output row
    masked; LCG inputs (seeds 31, 32, 33)."""
    torch, F = _torch()
    Hin, Win, Cin, Cout, stride = 9, 13, 4, 4, 2
    Hout = (Hin + pad + 1 - 3) // stride + 1
    Wout = (Win + pad + 1 - 3) // stride + 1
    x = orc.lcg_floats(Hin * Win * Cin, 31).reshape(Hin, Win, Cin)
    w = orc.lcg_floats(Cout * (Cin // groups) * 9, 32).reshape(Cout, Cin // groups, 3, 3)
    b = orc.lcg_floats(Cout, 33)
    got = orc.conv2d_cl(x, w, b, stride, pad, pad, groups, act=orc.ACT_RELU, valid_h=Hout - 1)
    assert got.shape == (Hout, Wout, Cout)
    xt = torch.as_tensor(x, dtype=torch.float64).permute(2, 0, 1)[None]
    ref = F.conv2d(F.pad(xt, (pad, 1, pad, 1)), torch.as_tensor(w, dtype=torch.float64),
                   torch.as_tensor(b, dtype=torch.float64), stride=stride, groups=groups)
    ref = F.relu(ref)[0].permute(1, 2, 0).numpy()
    ref[Hout - 1:] = 0.0
    assert ref.shape == got.shape
    assert np.abs(got - ref).max() < 1e-5


@pytest.mark.parametrize("T0,valid", [(25, 25), (25, 18), (9, 9), (9, 4), (121, 121), (121, 83), (16, 0)])
def test_subsample_matches_nemo_restatement(orc, T0, valid):
    ud = load_pkg()
    sw = ud.synthetic_subsampling_weights(seed=5)
    rng = np.random.default_rng(T0 * 100 + valid)
    mel = rng.standard_normal((T0, 128)).astype(np.float32)
    got = orc.subsample(mel, valid, sw)
    ref = refimpl.subsampling_nemo(mel, valid, sw).numpy()
    assert got.shape == ref.shape == (orc.sub_next_len(orc.sub_next_len(orc.sub_next_len(T0))), 1024)
    scale = np.abs(ref).max()
    assert np.abs(got - ref).max() <= 1e-5 * max(scale, 1.0), (np.abs(got - ref).max(), scale)


def test_subsample_length_rule_and_receptive_field(orc):
    """Output length L -> L//2+1 three times; frame k depends only on mel rows 8k-14 .. 8k
    (docs/specs/nemotron.md:52-81): perturbing row r changes exactly frames ceil(r/8) .. (r+14)//8."""
    ud = load_pkg()
    sw = ud.synthetic_subsampling_weights(seed=6)
    rng = np.random.default_rng(3)
    mel = rng.standard_normal((41, 128)).astype(np.float32)
    base = orc.subsample(mel, 41, sw)
    assert base.shape[0] == 6
    for r in (0, 7, 8, 20, 40):
        m2 = mel.copy()
        m2[r] += 1.0
        diff = np.abs(orc.subsample(m2, 41, sw) - base).max(axis=1) > 0
        k = np.arange(6)
        expect = (8 * k - 14 <= r) & (r <= 8 * k)
        np.testing.assert_array_equal(diff, expect, err_msg="row %d" % r)


def test_streamed_chunks_equal_offline(orc):
    """NeMo's pre-encode cache schedule (NemotronSchedule.swift:1-17; NemotronStreamer.swift:70-97):
    first chunk 1 + 8*la rows, then chunks of 8 + 8*la rows prefixed by the previous 9 rows with the
    first 2 subsampled frames dropped, reproduce the offline subsampling exactly (bit for bit)."""
    ud = load_pkg()
    sw = ud.synthetic_subsampling_weights(seed=7)
    rng = np.random.default_rng(4)
    la = 1
    total = 1 + 8 * la + 4 * (8 + 8 * la)
    mel = rng.standard_normal((total, 128)).astype(np.float32)
    offline = orc.subsample(mel, total, sw)
    frames = []
    idx = 0
    while idx < total:
        first = idx == 0
        size = 1 + 8 * la if first else 8 + 8 * la
        start = idx if first else idx - 9
        chunk = mel[start:idx + size]
        out = orc.subsample(chunk, chunk.shape[0], sw)
        frames.append(out if first else out[2:])
        idx += size
    streamed = np.concatenate(frames)
    assert streamed.shape[0] == (la + 1) * 5
    np.testing.assert_array_equal(streamed, offline[:streamed.shape[0]])
