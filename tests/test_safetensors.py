"""The safetensors reader and NeMo name map of the library (include/ud_safetensors.h), host-only,
pinned against the safetensors package (files written by safetensors.torch / safetensors.numpy):
dtypes F32/F16/BF16 widened bit-exactly, shapes, names, metadata, malformed files, and the HF ->
NeMo name map of docs/specs/nemotron.md:246-287."""
import json
import os
import struct

import numpy as np
import pytest

from conftest import load_pkg


@pytest.fixture(scope="module")
def ud():
    m = load_pkg()
    m.load_library()
    return m


def _save_torch(path, tensors, metadata=None):
    import torch
    from safetensors.torch import save_file
    save_file({k: v.contiguous() for k, v in tensors.items()}, path, metadata=metadata)


def test_dtypes_shapes_and_values(ud, tmp_path):
    import torch
    rng = np.random.default_rng(0)
    a = rng.standard_normal((3, 5, 7)).astype(np.float32)
    b = rng.standard_normal((11,)).astype(np.float32)
    c = rng.standard_normal((4, 6)).astype(np.float32)
    edge = np.array([0.0, -0.0, 1e-8, 6.1e-5, 65504.0, -np.inf, np.inf, 1.0 / 3.0], np.float32)
    p = str(tmp_path / "w.safetensors")
    _save_torch(p, {"a.weight": torch.from_numpy(a), "b": torch.from_numpy(b).to(torch.bfloat16),
                    "c": torch.from_numpy(c).to(torch.float16), "edge16": torch.from_numpy(edge).to(torch.float16),
                    "edgebf": torch.from_numpy(edge).to(torch.bfloat16), "i": torch.arange(5, dtype=torch.int32)},
                metadata={"source": "test", "format": "pt"})
    st = ud.SafeTensors(p)
    assert st.names() == sorted(["a.weight", "b", "c", "edge16", "edgebf", "i"])
    assert st.info("a.weight") == ("F32", (3, 5, 7))
    assert st.info("b") == ("BF16", (11,))
    assert st.info("c") == ("F16", (4, 6))
    assert st.info("i") == ("other", (5,))
    np.testing.assert_array_equal(st.floats("a.weight"), a)
    # widened values equal torch's own conversions back to fp32, bit for bit
    for name, t in (("b", torch.from_numpy(b).to(torch.bfloat16)), ("c", torch.from_numpy(c).to(torch.float16)),
                    ("edge16", torch.from_numpy(edge).to(torch.float16)), ("edgebf", torch.from_numpy(edge).to(torch.bfloat16))):
        ref = t.to(torch.float32).numpy()
        np.testing.assert_array_equal(st.floats(name).view(np.uint32), ref.view(np.uint32), err_msg=name)
    with pytest.raises(ud.EngineError) as e:
        st.floats("i")
    assert e.value.status == -6
    with pytest.raises(ud.EngineError) as e:
        st.floats("missing")
    assert e.value.status == -6
    st.close()


def test_numpy_writer_and_empty_tensor(ud, tmp_path):
    from safetensors.numpy import save_file
    p = str(tmp_path / "n.safetensors")
    z = np.zeros((0, 4), np.float32)
    x = np.arange(12, dtype=np.float32).reshape(3, 4)
    save_file({"z": z, "x": x}, p)
    st = ud.SafeTensors(p)
    assert st.info("z") == ("F32", (0, 4))
    assert st.floats("z").shape == (0, 4)
    np.testing.assert_array_equal(st.floats("x"), x)
    st.close()


def _write_raw(path, header, data=b""):
    h = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + data)


@pytest.mark.parametrize("case", ["short", "header_past_end", "not_json", "offsets_past_end", "size_mismatch",
                                  "bad_dtype", "negative_shape"])
def test_malformed_files(ud, tmp_path, case):
    p = str(tmp_path / ("%s.safetensors" % case))
    if case == "short":
        open(p, "wb").write(b"\x01\x02")
    elif case == "header_past_end":
        open(p, "wb").write(struct.pack("<Q", 1 << 40) + b"{}")
    elif case == "not_json":
        open(p, "wb").write(struct.pack("<Q", 5) + b"{abc:")
    elif case == "offsets_past_end":
        _write_raw(p, {"t": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}, b"\0" * 8)
    elif case == "size_mismatch":
        _write_raw(p, {"t": {"dtype": "F32", "shape": [3], "data_offsets": [0, 16]}}, b"\0" * 16)
    elif case == "bad_dtype":
        _write_raw(p, {"t": {"dtype": "Q4", "shape": [4], "data_offsets": [0, 4]}}, b"\0" * 4)
    elif case == "negative_shape":
        _write_raw(p, {"t": {"dtype": "F32", "shape": [-1], "data_offsets": [0, 4]}}, b"\0" * 4)
    with pytest.raises(ud.EngineError) as e:
        ud.SafeTensors(p)
    assert e.value.status == -6, case


def test_escaped_names_and_metadata(ud, tmp_path):
    p = str(tmp_path / "e.safetensors")
    # json.dumps writes the key as "a\"b\u00e9x" (escaped quote, \u escape of a non-ASCII letter)
    _write_raw(p, {"__metadata__": {"k": "v"}, 'a"b\u00e9x': {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}},
               struct.pack("<f", 2.5))
    st = ud.SafeTensors(p)
    assert st.names() == ['a"b\u00e9x']
    assert st.floats('a"b\u00e9x')[0] == 2.5
    st.close()


# docs/specs/nemotron.md:246-287: HF model.safetensors name -> NeMo state_dict name
HF_TO_NEMO = [
    ("encoder.subsampling.conv_in.weight", "encoder.pre_encode.conv.0.weight"),
    ("encoder.subsampling.conv_in.bias", "encoder.pre_encode.conv.0.bias"),
    ("encoder.subsampling.layers.0.depthwise_conv.weight", "encoder.pre_encode.conv.2.weight"),
    ("encoder.subsampling.layers.0.pointwise_conv.bias", "encoder.pre_encode.conv.3.bias"),
    ("encoder.subsampling.layers.1.depthwise_conv.bias", "encoder.pre_encode.conv.5.bias"),
    ("encoder.subsampling.layers.1.pointwise_conv.weight", "encoder.pre_encode.conv.6.weight"),
    ("encoder.subsampling.linear.weight", "encoder.pre_encode.out.weight"),
    ("encoder.layers.7.self_attn.q_proj.weight", "encoder.layers.7.self_attn.linear_q.weight"),
    ("encoder.layers.0.self_attn.k_proj.weight", "encoder.layers.0.self_attn.linear_k.weight"),
    ("encoder.layers.23.self_attn.v_proj.weight", "encoder.layers.23.self_attn.linear_v.weight"),
    ("encoder.layers.1.self_attn.o_proj.weight", "encoder.layers.1.self_attn.linear_out.weight"),
    ("encoder.layers.12.self_attn.relative_k_proj.weight", "encoder.layers.12.self_attn.linear_pos.weight"),
    ("encoder.layers.3.self_attn.bias_u", "encoder.layers.3.self_attn.pos_bias_u"),
    ("encoder.layers.3.self_attn.bias_v", "encoder.layers.3.self_attn.pos_bias_v"),
    ("encoder.layers.5.conv.norm.weight", "encoder.layers.5.conv.batch_norm.weight"),
    ("encoder.layers.5.conv.norm.bias", "encoder.layers.5.conv.batch_norm.bias"),
    ("decoder.embedding.weight", "decoder.prediction.embed.weight"),
    ("decoder.lstm.weight_ih_l0", "decoder.prediction.dec_rnn.lstm.weight_ih_l0"),
    ("decoder.lstm.bias_hh_l1", "decoder.prediction.dec_rnn.lstm.bias_hh_l1"),
    ("decoder.decoder_projector.weight", "joint.pred.weight"),
    ("encoder_projector.bias", "joint.enc.bias"),
    ("joint.head.weight", "joint.joint_net.2.weight"),
]
SAME = ["encoder.layers.4.feed_forward1.linear1.weight", "encoder.layers.4.norm_self_att.bias",
        "encoder.layers.4.conv.pointwise_conv1.weight", "encoder.layers.4.conv.depthwise_conv.weight",
        "encoder.layers.4.self_attn.linear_q.weight", "encoder.pre_encode.out.bias", "joint.pred.bias",
        "preprocessor.featurizer.fb", "encoder.layers.9.norm_out.weight"]


def test_name_map(ud):
    for hf, nemo in HF_TO_NEMO:
        assert ud.nemo_name(hf) == nemo, hf
        assert ud.nemo_name(nemo) == nemo
    for n in SAME:
        assert ud.nemo_name(n) == n
