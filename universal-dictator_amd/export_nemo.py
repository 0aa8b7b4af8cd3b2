"""Unpacks a NeMo .nemo checkpoint into the plain files the weight loaders read.

    python universal-dictator_amd/export_nemo.py <model>.nemo [out_dir]

The counterpart of the reference's extractor (tools/export_weights.py:31-62).  It writes, into
out_dir (default: `nemo_extracted/` next to the .nemo file):

  weights.safetensors   every floating-point tensor of model_weights.ckpt under its NeMo name,
                        as fp32 (the encoder, decoder and mel loaders take NeMo names:
                        ud_encoder_load_safetensors and friends, include/ud_safetensors.h)
  model_config.yaml     the model config
  <tokenizer files>     as named in the archive, plus a copy under the stable names
                        tokenizer.model / tokenizer.vocab / vocab.txt (ud_tokenizer_load reads
                        tokenizer.vocab)
  manifest.json         source name and sha256, name -> shape of the exported tensors, and the
                        non-float tensors left out (name -> [shape, dtype])

The checkpoint is read with torch.load(weights_only=True): tensors and plain containers only,
nothing from the file is executed.  Plain and gzip-compressed archives are both accepted.
"""
import hashlib
import io
import json
import os
import sys
import tarfile

STABLE_TOKENIZER_NAMES = ("tokenizer.model", "tokenizer.vocab", "vocab.txt")


def _sha256(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        while True:
            block = f.read(1 << 24)
            if not block:
                return h.hexdigest()
            h.update(block)


def _is_side_file(base):
    return base == "model_config.yaml" or "tokenizer" in base or base.endswith("vocab.txt")


def export_nemo(nemo_path, out_dir=None):
    """Writes the files listed in the module docstring; returns the manifest (a dict)."""
    import torch
    from safetensors.torch import save_file

    src = os.path.abspath(nemo_path)
    out = out_dir or os.path.join(os.path.dirname(src), "nemo_extracted")
    os.makedirs(out, exist_ok=True)
    state = None
    with tarfile.open(src, "r:*") as tar:
        for member in tar:
            if not member.isfile():
                continue
            base = os.path.basename(member.name)
            blob = tar.extractfile(member).read()
            if base == "model_weights.ckpt":
                state = torch.load(io.BytesIO(blob), map_location="cpu", weights_only=True)
            elif _is_side_file(base):
                # tokenizer files carry a hash prefix inside the archive: keep that name and a
                # stable one
                with open(os.path.join(out, base), "wb") as f:
                    f.write(blob)
                for stable in STABLE_TOKENIZER_NAMES:
                    if base.endswith(stable) and base != stable:
                        with open(os.path.join(out, stable), "wb") as f:
                            f.write(blob)
    if state is None:
        raise SystemExit("%s: no model_weights.ckpt in the archive" % nemo_path)
    floats, skipped = {}, {}
    for name, t in state.items():
        if not torch.is_tensor(t):
            continue
        if t.is_floating_point():
            floats[name] = t.detach().to(torch.float32).contiguous()
        else:
            skipped[name] = [list(t.shape), str(t.dtype)]
    save_file(floats, os.path.join(out, "weights.safetensors"))
    manifest = {
        "source": os.path.basename(src),
        "source_sha256": _sha256(src),
        "tensors": {k: list(floats[k].shape) for k in sorted(floats)},
        "non_float_tensors_skipped": {k: skipped[k] for k in sorted(skipped)},
    }
    with open(os.path.join(out, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1)
    return manifest


def main(argv):
    if len(argv) not in (2, 3):
        print(__doc__.strip().splitlines()[2].strip())
        return 2
    m = export_nemo(argv[1], argv[2] if len(argv) == 3 else None)
    print("wrote %d tensors (%d non-float left out)" % (len(m["tensors"]), len(m["non_float_tensors_skipped"])))
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
