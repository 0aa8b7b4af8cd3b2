"""GPU check of the safetensors loaders (ud_encoder_load_safetensors, ud_rnnt_load_safetensors):
one file holding NeMo names and HF aliases (docs/specs/nemotron.md:246-287), F32 / BF16 / F16 tensors,
a layer beyond the encoder's depth and tensors of other modules must give an encoder and a decoder
whose outputs are bit-identical to ones whose weights were set tensor by tensor (set_weight with the
same widened values)."""
import numpy as np
import pytest

import harness

pytestmark = pytest.mark.gpu

# NeMo suffix -> HF suffix where the HF checkpoint renames a layer tensor
HF_LAYER = {
    "self_attn.linear_q.weight": "self_attn.q_proj.weight", "self_attn.linear_k.weight": "self_attn.k_proj.weight",
    "self_attn.linear_v.weight": "self_attn.v_proj.weight", "self_attn.linear_out.weight": "self_attn.o_proj.weight",
    "self_attn.linear_pos.weight": "self_attn.relative_k_proj.weight", "self_attn.pos_bias_u": "self_attn.bias_u",
    "self_attn.pos_bias_v": "self_attn.bias_v", "conv.batch_norm.weight": "conv.norm.weight",
    "conv.batch_norm.bias": "conv.norm.bias",
}
HF_SUB = {"conv.0": "conv_in", "conv.2": "layers.0.depthwise_conv", "conv.3": "layers.0.pointwise_conv",
          "conv.5": "layers.1.depthwise_conv", "conv.6": "layers.1.pointwise_conv", "out": "linear"}


def _hf_rnnt(name):
    p = "decoder.prediction."
    if name.startswith(p + "dec_rnn.lstm."):
        return "decoder.lstm." + name[len(p + "dec_rnn.lstm."):]
    if name == p + "embed.weight":
        return "decoder.embedding.weight"
    for nemo, hf in (("joint.pred.", "decoder.decoder_projector."), ("joint.enc.", "encoder_projector."),
                     ("joint.joint_net.2.", "joint.head.")):
        if name.startswith(nemo):
            return hf + name[len(nemo):]
    return name


def _write(ud, path, entries):
    """Writes a safetensors file (8-byte little-endian header length, JSON header, raw data) without
    torch, which must not load into a GPU test process.  entries: name -> (fp32 array, 'F32' |
    'BF16' | 'F16').  Returns name -> the fp32 values a reader widens the stored tensor to."""
    import json
    import struct
    header, blobs, widened, off = {"__metadata__": {"format": "pt"}}, [], {}, 0
    for name, (a, d) in entries.items():
        a = np.ascontiguousarray(a, np.float32)
        if d == "F32":
            raw, w = a.tobytes(), a
        elif d == "F16":
            h = a.astype(np.float16)
            raw, w = h.tobytes(), h.astype(np.float32)
        else:
            w = ud.round_bf16(a)
            raw = (w.view(np.uint32) >> 16).astype(np.uint16).tobytes()
        header[name] = {"dtype": d, "shape": list(a.shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        widened[name] = w.reshape(a.shape)
        off += len(raw)
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + b"".join(blobs))
    return widened


def test_encoder_loader_matches_set_weight(gpu, tmp_path):
    ud = gpu
    cfg = ud.EncoderConfig(layers=2, max_chunk=2, max_streams=2, dtype="bf16")
    lw = [ud.synthetic_layer_weights(cfg, 61, l) for l in range(3)]
    sw = ud.synthetic_subsampling_weights(62)
    rw = ud.synthetic_rnnt_weights(63)
    entries, expect = {}, {}
    for l, w in enumerate(lw):
        for suf, a in w.items():
            nemo = "encoder.layers.%d.%s" % (l, suf)
            if l == 1:            # HF names, linear weights stored in BF16
                name = "encoder.layers.1." + HF_LAYER.get(suf, suf)
                d = "BF16" if suf in harness.BF16_WEIGHTS else "F32"
            else:
                name, d = nemo, "F32"
            entries[name] = (a, d)
            expect[name] = nemo
    for k, a in sw.items():      # pre-encode under HF names, the output Linear in F16
        mod, field = k[len("encoder.pre_encode."):].rsplit(".", 1)
        name = "encoder.subsampling.%s.%s" % (HF_SUB[mod], field)
        entries[name] = (a, "F16" if mod == "out" and field == "weight" else "F32")
        expect[name] = k
    for k, a in rw.items():      # other modules: the encoder loader skips them
        entries[k] = (a, "F32")
    entries["preprocessor.featurizer.fb"] = (np.ones((1, 128, 257), np.float32), "F32")
    p = str(tmp_path / "enc.safetensors")
    widened = _write(ud, p, entries)

    st = ud.SafeTensors(p)
    a = ud.Encoder(cfg)
    n = a.load_safetensors(st)
    assert n == 2 * 26 + 12                       # layer 2 and the decoder / preprocessor tensors skipped
    a.finalize()
    b = ud.Encoder(cfg)
    for name, nemo in expect.items():
        if not nemo.startswith("encoder.layers.2."):
            b.set_weight(nemo, widened[name])
    b.finalize()

    S = 2
    rng = np.random.default_rng(64)
    mel = rng.standard_normal((S, 9 + 16, 128)).astype(np.float32)
    outs = []
    for enc in (a, b):
        streams = [enc.new_stream() for _ in range(S)]
        xb, ob = ud.DeviceBuffer(S * 2 * 1024 * 4), ud.DeviceBuffer(S * 2 * 1024 * 4)
        got = []
        for start, rows, drop in ((0, 9, 0), (0, 25, 2)):
            chunk = ud.DeviceBuffer.from_numpy(np.ascontiguousarray(mel[:, start:start + rows]))
            T, vt = enc.subsample(S, chunk, xb, drop=drop)
            enc.encode_stream_step(streams, xb, ob, valid=vt, T=T)
            got.append(ob.download((S, T, 1024)).copy())
        outs.append(got)
    for ga, gb in zip(*outs):
        assert np.isfinite(ga).all()
        assert np.array_equal(ga.view(np.uint32), gb.view(np.uint32))
    st.close()
    a.close()
    b.close()


def test_rnnt_loader_matches_set_weight(gpu, tmp_path):
    ud = gpu
    rw = ud.synthetic_rnnt_weights(71, blank_bias=0.95)
    entries, expect = {}, {}
    for i, (k, a) in enumerate(sorted(rw.items())):
        name = _hf_rnnt(k) if i % 2 else k      # every other tensor under its HF name
        entries[name] = (a, "BF16" if k == "joint.joint_net.2.weight" else "F32")
        expect[name] = k
    entries["encoder.layers.0.norm_out.weight"] = (np.ones(1024, np.float32), "F32")
    p = str(tmp_path / "dec.safetensors")
    widened = _write(ud, p, entries)
    assert sum(n != expect[n] for n in entries if n in expect) >= 7   # HF aliases in the file

    st = ud.SafeTensors(p)
    a = ud.Rnnt(max_streams=3)
    assert a.load_safetensors(st) == len(rw)
    b = ud.Rnnt(max_streams=3)
    b.set_weights({nemo: widened[name] for name, nemo in expect.items()})
    rng = np.random.default_rng(72)
    x = ud.DeviceBuffer.from_numpy(rng.standard_normal((3 * 4, 1024)).astype(np.float32))
    res = []
    for r in (a, b):
        pb = ud.DeviceBuffer(3 * 4 * 640 * 4)
        r.project(12, x, pb)
        toks, cnt = r.greedy([0, 1, 2], pb, 4, [4, 3, 4], cap=64)
        res.append((pb.download((12, 640)).copy(), toks, list(cnt)))
    assert np.array_equal(res[0][0].view(np.uint32), res[1][0].view(np.uint32))
    assert res[0][1] == res[1][1] and res[0][2] == res[1][2]
    assert sum(res[0][2]) > 0
    st.close()
    a.close()
    b.close()


def test_mel_loader_matches_direct(gpu, tmp_path):
    """ud_mel_load_safetensors reads preprocessor.featurizer.fb [1, 128, 257] and .window [400]
    (NemotronModel.init, Sources/DictatorEngine/Models/Nemotron.swift:45-46): its features equal
    those of a frontend built from the same arrays, bit for bit; a file without them is rejected."""
    import refimpl
    ud = gpu
    fb, win = refimpl.slaney_mel_fb(), refimpl.hann_symmetric()
    p = str(tmp_path / "mel.safetensors")
    _write(ud, p, {"preprocessor.featurizer.fb": (fb.reshape(1, 128, 257), "F32"),
                   "preprocessor.featurizer.window": (win, "F32"),
                   "joint.enc.bias": (np.zeros(640, np.float32), "F32")})
    st = ud.SafeTensors(p)
    a = ud.MelFrontend.from_safetensors(st)
    b = ud.MelFrontend(fb, win)
    assert a.n_mels == 128
    audio = np.sin(np.arange(7777, dtype=np.float32) * 0.05).astype(np.float32)
    fa, fbb = a.features([audio])[0], b.features([audio])[0]
    assert np.array_equal(fa.view(np.uint32), fbb.view(np.uint32))
    st.close()
    q = str(tmp_path / "nomel.safetensors")
    _write(ud, q, {"joint.enc.bias": (np.zeros(640, np.float32), "F32")})
    st = ud.SafeTensors(q)
    with pytest.raises(ud.EngineError) as e:
        ud.MelFrontend.from_safetensors(st)
    assert e.value.status == -6
    st.close()
    a.close()
    b.close()
