"""Independent restatements used to pin the oracle (tests only).

These restate NeMo's modules with torch/numpy library routines in float64, in the structure NeMo
uses rather than the oracle's: rel_shift is the literal pad/view trick
(Tests/DictatorEngineTests/ConformerOpTests.swift:111-122; reference/nemo/check_spec.py:143-146),
the depthwise conv is torch conv1d with causal left padding, masks are boolean matrices filled
with -10000 before softmax and zeroed after (docs/specs/nemotron.md:83-135).
"""
import numpy as np


def nemo_rel_shift(x):
    """NeMo RelPositionMultiHeadAttention.rel_shift on x [..., Tq, nPos] (numpy or torch): pad one
    zero column on the left, view as [..., nPos+1, Tq], drop the first row, view back as
    [..., Tq, nPos]."""
    *lead, tq, npos = x.shape
    if isinstance(x, np.ndarray):
        pad = np.concatenate([np.zeros((*lead, tq, 1), x.dtype), x], axis=-1)
    else:
        import torch.nn.functional as F
        pad = F.pad(x, (1, 0))
    pad = pad.reshape(*lead, npos + 1, tq)
    return pad[..., 1:, :].reshape(*lead, tq, npos)


def nemo_pe(T, D):
    """NeMo RelPositionalEncoding rows for positions T-1 ... -(T-1) (row r = position T-1-r), in
    float64 closed form."""
    pos = np.arange(T - 1, -T, -1, dtype=np.float64)[:, None]
    div = np.exp(np.arange(0, D, 2, dtype=np.float64) * -(np.log(10000.0) / D))
    pe = np.zeros((2 * T - 1, D))
    pe[:, 0::2] = np.sin(pos * div)
    pe[:, 1::2] = np.cos(pos * div)
    return pe


def layer_nemo(x, w, pe, mask, valid, H, Kc=9, clip=None):
    """One NeMo ConformerLayer (conformer_modules.py:160-233 per docs/specs/nemotron.md:83-135) on a
    full utterance x [T, D] (float64 torch).  pe: projected-input table rows for positions
    T-1..-(T-1) [2T-1, D]; mask [T, T] bool, True = hidden; rows >= valid are padding.
    clip: if set, the activations a 16-bit encoder stores in 16 bits (the LayerNorm outputs feeding
    a projection, the FF hidden, q/k/v, the attention output, the conv LayerNorm + SiLU output) are
    clamped to [-clip, clip] (torch.clamp)."""
    import torch
    import torch.nn.functional as F
    T, D = x.shape
    dk = D // H
    c16 = (lambda y: torch.clamp(y, -clip, clip)) if clip else (lambda y: y)
    t = lambda k: torch.as_tensor(w[k], dtype=torch.float64)
    ln = lambda y, n: c16(F.layer_norm(y, (D,), t(n + ".weight"), t(n + ".bias"), eps=1e-5))
    r = x + 0.5 * F.linear(c16(F.silu(F.linear(ln(x, "norm_feed_forward1"), t("feed_forward1.linear1.weight")))),
                           t("feed_forward1.linear2.weight"))
    z = ln(r, "norm_self_att")
    q = c16(F.linear(z, t("self_attn.linear_q.weight"))).view(T, H, dk).transpose(0, 1)
    k = c16(F.linear(z, t("self_attn.linear_k.weight"))).view(T, H, dk).transpose(0, 1)
    v = c16(F.linear(z, t("self_attn.linear_v.weight"))).view(T, H, dk).transpose(0, 1)
    p = F.linear(torch.as_tensor(pe), t("self_attn.linear_pos.weight")).view(2 * T - 1, H, dk).transpose(0, 1)
    qu = q + t("self_attn.pos_bias_u").view(H, 1, dk)
    qv = q + t("self_attn.pos_bias_v").view(H, 1, dk)
    ac = qu @ k.transpose(1, 2)
    bd = nemo_rel_shift(qv @ p.transpose(1, 2))[:, :, :T]
    s = (ac + bd) / np.sqrt(dk)
    m = torch.as_tensor(mask)
    s = s.masked_fill(m, -10000.0)
    a = torch.softmax(s, dim=-1).masked_fill(m, 0.0)
    o = c16((a @ v).transpose(0, 1).reshape(T, D))
    r = r + F.linear(o, t("self_attn.linear_out.weight"))
    z = ln(r, "norm_conv")
    g = F.glu(F.linear(z, t("conv.pointwise_conv1.weight")), dim=-1)
    g[valid:] = 0.0
    dw = t("conv.depthwise_conv.weight").view(D, 1, Kc)
    c = F.conv1d(F.pad(g.T.unsqueeze(0), (Kc - 1, 0)), dw, groups=D)[0].T
    c = c16(F.silu(F.layer_norm(c, (D,), t("conv.batch_norm.weight"), t("conv.batch_norm.bias"), eps=1e-5)))
    r = r + F.linear(c, t("conv.pointwise_conv2.weight"))
    r = r + 0.5 * F.linear(c16(F.silu(F.linear(ln(r, "norm_feed_forward2"), t("feed_forward2.linear1.weight")))),
                           t("feed_forward2.linear2.weight"))
    return F.layer_norm(r, (D,), t("norm_out.weight"), t("norm_out.bias"), eps=1e-5)


def chunked_limited_mask(T, left, right, valid):
    """NeMo chunked_limited visibility (conformer_encoder.py:803-822 per docs/specs/nemotron.md:137-149):
    visible(i,j) = 0 <= i//chunk - j//chunk <= left//chunk; keys >= valid hidden.  True = hidden."""
    cs = right + 1
    i = np.arange(T)[:, None] // cs
    j = np.arange(T)[None, :] // cs
    vis = (i - j >= 0) & (i - j <= left // cs)
    vis &= np.arange(T)[None, :] < valid
    return ~vis


def subsampling_nemo(mel, valid, w):
    """NeMo ConvSubsampling, dw_striding causal 8x (subsampling.py:142-215, 425-431 per
    docs/specs/nemotron.md:52-81) on one utterance, float64 torch: the image is [1, 1, T, F] (time =
    height), CausalConv2D pads (left 2, right 1, top 2, bottom 1) and convolves with stride 2,
    MaskedConvSequential zeroes time rows >= the running length before every layer and after the
    last, the length after a stride-2 conv is (L + 2 + 1 - 3) // 2 + 1, and the flatten is
    [B, C, T, F] -> [B, T, C*F] (channel-major) into pre_encode.out.  w maps NeMo names to arrays."""
    import torch
    import torch.nn.functional as F
    t = lambda n: torch.as_tensor(np.asarray(w["encoder.pre_encode." + n]), dtype=torch.float64)
    x = torch.as_tensor(np.asarray(mel), dtype=torch.float64)[None, None]
    C = t("conv.0.weight").shape[0]
    length = int(valid)

    def mask(y):
        keep = (torch.arange(y.shape[2]) < length).to(y.dtype).view(1, 1, -1, 1)
        return y * keep

    def causal(y, i, groups):
        return F.conv2d(F.pad(y, (2, 1, 2, 1)), t("conv.%d.weight" % i), t("conv.%d.bias" % i), stride=2,
                        groups=groups)

    layers = [("c", 0, 1), ("relu",), ("c", 2, C), ("p", 3), ("relu",), ("c", 5, C), ("p", 6), ("relu",)]
    for layer in layers:
        x = mask(x)
        if layer[0] == "c":
            x = causal(x, layer[1], layer[2])
            length = (length + 2 + 1 - 3) // 2 + 1
        elif layer[0] == "p":
            x = F.conv2d(x, t("conv.%d.weight" % layer[1]), t("conv.%d.bias" % layer[1]))
        else:
            x = F.relu(x)
    x = mask(x)
    _, Cc, T, Fq = x.shape
    x = x.transpose(1, 2).reshape(1, T, Cc * Fq)
    return F.linear(x, t("out.weight"), t("out.bias"))[0]


def rnnt_greedy_nemo(f, w, state=None, max_symbols=10):
    """NeMo greedy RNN-T (reference/nemo/check_spec.py:176-207 structure; docs/specs/nemotron.md:210-244)
    on projected encoder frames f [T, H] (joint.enc applied), float64 torch with torch.nn.LSTMCell,
    with no prediction cache: the prediction is recomputed from the committed state whenever the
    loop needs it.  state (dict h, c: lists of [H], token) carries across calls; returns tokens."""
    import torch
    import torch.nn.functional as F
    t_ = lambda n: torch.as_tensor(np.asarray(w[n]), dtype=torch.float64)
    emb = t_("decoder.prediction.embed.weight")
    V, H = emb.shape
    blank = V - 1
    L = 0
    while "decoder.prediction.dec_rnn.lstm.weight_ih_l%d" % L in w:
        L += 1
    cells = []
    for l in range(L):
        cell = torch.nn.LSTMCell(H, H).double()
        with torch.no_grad():
            cell.weight_ih.copy_(t_("decoder.prediction.dec_rnn.lstm.weight_ih_l%d" % l))
            cell.weight_hh.copy_(t_("decoder.prediction.dec_rnn.lstm.weight_hh_l%d" % l))
            cell.bias_ih.copy_(t_("decoder.prediction.dec_rnn.lstm.bias_ih_l%d" % l))
            cell.bias_hh.copy_(t_("decoder.prediction.dec_rnn.lstm.bias_hh_l%d" % l))
        cells.append(cell)
    if state is None:
        state = dict(h=[torch.zeros(H, dtype=torch.float64) for _ in range(L)],
                     c=[torch.zeros(H, dtype=torch.float64) for _ in range(L)], token=blank)

    def pred(tok, hs, cs):
        x = torch.zeros(H, dtype=torch.float64) if tok == blank else emb[tok]
        nh, nc = [], []
        with torch.no_grad():
            for l, cell in enumerate(cells):
                hh, cc = cell(x[None], (hs[l][None], cs[l][None]))
                nh.append(hh[0])
                nc.append(cc[0])
                x = hh[0]
        return F.linear(x, t_("joint.pred.weight"), t_("joint.pred.bias")), nh, nc

    f = torch.as_tensor(np.asarray(f), dtype=torch.float64)
    toks = []
    for t in range(f.shape[0]):
        n = 0
        while n < max_symbols:
            g, nh, nc = pred(state["token"], state["h"], state["c"])
            logits = F.linear(F.relu(f[t] + g), t_("joint.joint_net.2.weight"), t_("joint.joint_net.2.bias"))
            k = int(torch.argmax(logits))
            if k == blank:
                break
            toks.append(k)
            state["h"], state["c"], state["token"] = nh, nc, k
            n += 1
    return toks, state


def mel_nemo(audio, fb, window, dtype=None):
    """NeMo FilterbankFeatures at inference (dither off, no normalization; docs/specs/nemotron.md
    §9.1): x[0] = a[0], x[i] = a[i] - 0.97 a[i-1] (fp32, as NeMo runs it); torch.stft(n_fft=512,
    hop 160, win_length 400, the symmetric window centred in 512, center=True, constant padding);
    |X|^2; fb @ power; log(x + 2^-24); frames >= n // 160 zeroed.  The STFT onward in float64.
    Returns [n // 160 + 1, n_mels]."""
    import torch
    a = torch.from_numpy(np.ascontiguousarray(audio, np.float32))
    x = torch.cat([a[:1], a[1:] - 0.97 * a[:-1]]).double()
    X = torch.stft(x, n_fft=512, hop_length=160, win_length=400, window=torch.from_numpy(window).double(),
                   center=True, pad_mode="constant", return_complex=True)
    power = X.abs().pow(2.0)                                   # [257, T]
    mel = torch.from_numpy(np.asarray(fb, np.float64).reshape(-1, 257)) @ power
    out = torch.log(mel + 2.0 ** -24).T.contiguous()
    out[a.numel() // 160:] = 0
    return out.numpy()


def mel_rfft(audio, fb, window):
    """The same features through numpy.fft.rfft of each zero-padded 512-sample frame (the window
    zero-padded to 512, centred), float64 from the fp32 preemphasized signal."""
    a = np.asarray(audio, np.float32)
    x = np.concatenate([a[:1], a[1:] - np.float32(0.97) * a[:-1]]).astype(np.float64)
    n = a.size
    xp = np.concatenate([np.zeros(256), x, np.zeros(256)])
    T = n // 160 + 1
    w = np.zeros(512)
    w[56:456] = np.asarray(window, np.float64)
    frames = np.stack([xp[t * 160:t * 160 + 512] * w for t in range(T)])
    power = np.abs(np.fft.rfft(frames, axis=1)) ** 2
    out = np.log(power @ np.asarray(fb, np.float64).reshape(-1, 257).T + 2.0 ** -24)
    out[n // 160:] = 0
    return out


def slaney_mel_fb(sr=16000, n_fft=512, n_mels=128):
    """librosa.filters.mel(sr, n_fft, n_mels, htk=False, norm='slaney') restated (the checkpoint's
    preprocessor.featurizer.fb is this matrix up to 1e-8, docs/specs/nemotron.md:291)."""
    def hz_to_mel(f):
        f = np.asarray(f, np.float64)
        f_sp = 200.0 / 3
        mels = f / f_sp
        min_log_hz = 1000.0
        min_log_mel = min_log_hz / f_sp
        logstep = np.log(6.4) / 27.0
        return np.where(f >= min_log_hz, min_log_mel + np.log(np.maximum(f, 1e-10) / min_log_hz) / logstep, mels)

    def mel_to_hz(m):
        m = np.asarray(m, np.float64)
        f_sp = 200.0 / 3
        freqs = f_sp * m
        min_log_hz = 1000.0
        min_log_mel = min_log_hz / f_sp
        logstep = np.log(6.4) / 27.0
        return np.where(m >= min_log_mel, min_log_hz * np.exp(logstep * (m - min_log_mel)), freqs)

    fftfreqs = np.linspace(0, sr / 2, 1 + n_fft // 2)
    mel_f = mel_to_hz(np.linspace(hz_to_mel(0.0), hz_to_mel(sr / 2.0), n_mels + 2))
    fdiff = np.diff(mel_f)
    ramps = mel_f[:, None] - fftfreqs[None, :]
    lower = -ramps[:-2] / fdiff[:-1, None]
    upper = ramps[2:] / fdiff[1:, None]
    w = np.maximum(0, np.minimum(lower, upper))
    w *= (2.0 / (mel_f[2:n_mels + 2] - mel_f[:n_mels]))[:, None]
    return w.astype(np.float32)


def hann_symmetric(n=400):
    """torch.hann_window(400, periodic=False): 0.5 - 0.5 cos(2 pi i / 399)."""
    return (0.5 - 0.5 * np.cos(2 * np.pi * np.arange(n) / (n - 1))).astype(np.float32)
