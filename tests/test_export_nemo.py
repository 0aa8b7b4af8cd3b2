"""The .nemo extractor (universal-dictator_amd/export_nemo.py; the reference's tools/export_weights.py:
31-62) on a synthetic archive built here: a NeMo-named state dict with fp32, bf16 and fp16 tensors
and an integer buffer, the model config and hash-prefixed tokenizer files, plain and gzipped.  The
written safetensors file is read back with the library's own reader (host code) and the
tokenizer.vocab copy with ud_tokenizer.  CPU only."""
import hashlib
import importlib.util
import io
import json
import os
import tarfile

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytest.importorskip("safetensors")

from conftest import ROOT


def _export_module():
    spec = importlib.util.spec_from_file_location("export_nemo", os.path.join(ROOT, "universal-dictator_amd", "export_nemo.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _state():
    g = torch.Generator().manual_seed(3)
    return {
        "encoder.layers.0.feed_forward1.linear1.weight": torch.randn(8, 4, generator=g),
        "encoder.layers.0.self_attn.pos_bias_u": torch.randn(2, 2, generator=g).to(torch.bfloat16),
        "encoder.pre_encode.conv.0.weight": torch.randn(4, 1, 3, 3, generator=g).to(torch.float16),
        "encoder.layers.0.conv.batch_norm.num_batches_tracked": torch.tensor(7, dtype=torch.int64),
        "decoder.prediction.embed.weight": torch.randn(5, 3, generator=g),
    }


def _write_nemo(path, state, gz):
    buf = io.BytesIO()
    torch.save(state, buf)
    files = {
        "./model_config.yaml": b"encoder:\n  d_model: 1024\n",
        "./model_weights.ckpt": buf.getvalue(),
        "./1a2b3c_tokenizer.model": b"\x00binary-model",
        "./4d5e6f_tokenizer.vocab": "<unk>\t0\n<s>\t0\n</s>\t0\n▁hello\t-1\nworld\t-2\n".encode("utf-8"),
        "./notes.txt": b"not exported",
    }
    with tarfile.open(path, "w:gz" if gz else "w") as tar:
        tar.addfile(tarfile.TarInfo("./"))
        for name, data in files.items():
            info = tarfile.TarInfo(name)
            info.size = len(data)
            tar.addfile(info, io.BytesIO(data))


@pytest.mark.parametrize("gz", [False, True])
def test_export_nemo(ud, tmp_path, gz):
    ex = _export_module()
    state = _state()
    nemo = tmp_path / "model.nemo"
    _write_nemo(nemo, state, gz)
    m = ex.export_nemo(str(nemo))
    out = tmp_path / "nemo_extracted"
    assert sorted(os.listdir(out)) == sorted(["weights.safetensors", "model_config.yaml", "manifest.json",
                                              "1a2b3c_tokenizer.model", "tokenizer.model",
                                              "4d5e6f_tokenizer.vocab", "tokenizer.vocab"])
    assert (out / "tokenizer.vocab").read_bytes() == (out / "4d5e6f_tokenizer.vocab").read_bytes()
    floats = {k: v for k, v in state.items() if v.is_floating_point()}
    assert m == json.loads((out / "manifest.json").read_text())
    assert m["source"] == "model.nemo"
    assert m["source_sha256"] == hashlib.sha256(nemo.read_bytes()).hexdigest()
    assert m["tensors"] == {k: list(floats[k].shape) for k in sorted(floats)}
    assert m["non_float_tensors_skipped"] == {"encoder.layers.0.conv.batch_norm.num_batches_tracked": [[], "torch.int64"]}
    # the library's reader sees NeMo names and fp32 values equal to the checkpoint's (widening exact)
    ud.load_library()
    st = ud.SafeTensors(str(out / "weights.safetensors"))
    assert sorted(st.names()) == sorted(floats)
    for k, v in floats.items():
        dt, shape = st.info(k)
        assert dt == "F32" and shape == tuple(v.shape)
        assert np.array_equal(st.floats(k), v.to(torch.float32).numpy())
    st.close()
    tok = ud.Tokenizer(str(out / "tokenizer.vocab"))
    assert tok.decode([3, 4, 1]) == b"helloworld"
    tok.close()


def test_export_nemo_without_weights(tmp_path):
    ex = _export_module()
    nemo = tmp_path / "empty.nemo"
    with tarfile.open(nemo, "w") as tar:
        info = tarfile.TarInfo("./model_config.yaml")
        info.size = 3
        tar.addfile(info, io.BytesIO(b"x: 1"[:3]))
    with pytest.raises(SystemExit):
        ex.export_nemo(str(nemo), str(tmp_path / "out"))
