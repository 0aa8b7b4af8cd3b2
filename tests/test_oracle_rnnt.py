"""Pins the oracle's RNN-T decoder (orc_rnnt_predict / orc_rnnt_joint_argmax / orc_rnnt_greedy,
restating Sources/DictatorCore/Decoding/RNNT.swift) against torch: torch.nn.LSTMCell for the
prediction network and NeMo's greedy loop without the reference's prediction cache
(tests/refimpl.py), across chunk boundaries, at both emission extremes."""
import numpy as np
import pytest

import refimpl
from conftest import load_pkg


def _torch():
    import torch
    import torch.nn.functional as F
    return torch, F


def test_predict_matches_lstmcell(orc):
    torch, F = _torch()
    ud = load_pkg()
    w = ud.synthetic_rnnt_weights(3)
    r = orc.Rnnt(w)
    rng = np.random.default_rng(1)
    h = rng.standard_normal((2, 640)).astype(np.float32) * 0.5
    c = rng.standard_normal((2, 640)).astype(np.float32) * 0.5
    for tok in (0, 17, 1023, 1024):
        proj, ho, co = r.predict(tok, h, c)
        x = torch.zeros(640, dtype=torch.float64) if tok == 1024 else torch.as_tensor(w["decoder.prediction.embed.weight"][tok], dtype=torch.float64)
        for l in range(2):
            cell = torch.nn.LSTMCell(640, 640).double()
            with torch.no_grad():
                for n in ("weight_ih", "weight_hh", "bias_ih", "bias_hh"):
                    getattr(cell, n).copy_(torch.as_tensor(w["decoder.prediction.dec_rnn.lstm.%s_l%d" % (n, l)], dtype=torch.float64))
                hh, cc = cell(x[None], (torch.as_tensor(h[l], dtype=torch.float64)[None], torch.as_tensor(c[l], dtype=torch.float64)[None]))
            assert np.abs(ho[l] - hh[0].numpy()).max() < 1e-5
            assert np.abs(co[l] - cc[0].numpy()).max() < 1e-5
            x = hh[0]
        ref = F.linear(x, torch.as_tensor(w["joint.pred.weight"], dtype=torch.float64),
                       torch.as_tensor(w["joint.pred.bias"], dtype=torch.float64)).numpy()
        assert np.abs(proj - ref).max() < 1e-5


@pytest.mark.parametrize("blank_bias,chunks", [(2.1, (5, 7, 4)), (-50.0, (3, 2)), (50.0, (4,))])
def test_greedy_matches_nemo_loop_across_chunks(orc, blank_bias, chunks):
    """blank_bias 2.1: blank frames, frames with 10 tokens and a frame with one token then blank; -50: every frame emits max_symbols (10) tokens;
    +50: nothing is emitted.  The oracle's state (with its cached prediction) carries across chunks
    and must give NeMo's tokens exactly."""
    ud = load_pkg()
    w = ud.synthetic_rnnt_weights(4, blank_bias=blank_bias)
    r = orc.Rnnt(w)
    rng = np.random.default_rng(5)
    f = rng.standard_normal((sum(chunks), 640)).astype(np.float32)
    st = r.state()
    got = []
    t = 0
    for n in chunks:
        got += r.greedy(f[t:t + n], st)
        t += n
    ref, _ = refimpl.rnnt_greedy_nemo(f, w)
    assert got == ref
    if blank_bias < 0:
        assert len(got) == 10 * f.shape[0]
    if blank_bias > 10:
        assert got == []
    else:
        assert len(got) > 0
