"""Shared set-up for GPU parity tests: the same seeded weights go to the HIP encoder and to the
oracle (fp32 activations).  For a 16-bit encoder the oracle gets the rounded linear weights that
the encoder computes with: bf16-rounded for dtype "bf16" (the reference's bf16-weight setting,
Core/Kernels.swift:79-112), f16-rounded for dtype "f16" (WeightConverter.convert(.f16),
Core/Convert.swift:76-112).  Either way the encoder holds the weights, its activations and its K/V
caches as IEEE half."""
import os

import numpy as np

# Linear weights that a 16-bit encoder stores rounded (the rest stay fp32: norms, pos_bias, depthwise
# conv -- Sources/DictatorEngine/Core/Convert.swift:76-83).
BF16_WEIGHTS = {
    "feed_forward1.linear1.weight", "feed_forward1.linear2.weight", "self_attn.linear_q.weight",
    "self_attn.linear_k.weight", "self_attn.linear_v.weight", "self_attn.linear_out.weight",
    "self_attn.linear_pos.weight", "conv.pointwise_conv1.weight", "conv.pointwise_conv2.weight",
    "feed_forward2.linear1.weight", "feed_forward2.linear2.weight",
}


def is16(cfg):
    """A 16-bit encoder (dtype bf16 or f16): half activations and caches."""
    return cfg.dtype in ("bf16", "f16")


def round_weights(ud, cfg, lw):
    """The layer weights as the encoder of cfg computes with them (linear weights rounded)."""
    if cfg.dtype == "bf16":
        return [{k: (ud.round_bf16(v) if k in BF16_WEIGHTS else v) for k, v in w.items()} for w in lw]
    if cfg.dtype == "f16":
        return [{k: (ud.round_f16(v) if k in BF16_WEIGHTS else v) for k, v in w.items()} for w in lw]
    return lw


def make_encoder(ud, orc, cfg, seed=1234, ln_jitter=0.1, edit=None):
    """(encoder, oracle model, oracle weights); edit(layer, weights) may change the synthetic
    weights before both sides get them."""
    lw = [ud.synthetic_layer_weights(cfg, seed, l, ln_jitter=ln_jitter) for l in range(cfg.layers)]
    if edit is not None:
        for l, w in enumerate(lw):
            edit(l, w)
    enc = ud.Encoder(cfg)
    for l, w in enumerate(lw):
        enc.set_layer_weights(l, w)
    enc.finalize()
    lw = round_weights(ud, cfg, lw)
    model = orc.Model(lw, cfg.d_model, cfg.heads, cfg.ff_dim, cfg.conv_kernel)
    model.prepare(-(cfg.max_chunk - 1), cfg.left_context + cfg.max_chunk - 1)
    return enc, model, lw


def oracle_sub_weights(sw, half):
    """The subsampling weights the oracle gets for an encoder whose front-end GEMMs run on half
    operands (half=True) -- the reference's f16 checkpoint policy, WeightConverter.keepF32 and
    convert(.f16) (Sources/DictatorEngine/Core/Convert.swift:76-112): pre_encode.out.weight
    rounded to f16, and every encoder.pre_encode.conv.* tensor kept fp32 (the library holds
    conv.3 and conv.6 as half too; that rounding shows up in the measured error)."""
    if not half:
        return dict(sw)
    return {k: (np.asarray(v, np.float32).astype(np.float16).astype(np.float32)
                if k == "encoder.pre_encode.out.weight" else v) for k, v in sw.items()}


# Achieved errors of the parity checks of this session, printed by the terminal summary of
# tests/conftest.py so that the margins against the bars are on record: (test, what, kind, values).
MARGINS = []


def _test_id():
    cur = os.environ.get("PYTEST_CURRENT_TEST", "?")
    return cur.split(" ")[0].split("::", 1)[-1]


def rel_err(got, ref):
    """Max abs error relative to max |ref| (the fp32 path's <= 1e-4 bar)."""
    e = float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))
    MARGINS.append((_test_id(), "", "fp32", e, None))
    return e


def cosine(a, b):
    a = a.ravel().astype(np.float64)
    b = b.ravel().astype(np.float64)
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-300))


def assert_bf16_close(got, ref, what=""):
    """The bf16 bar: max abs error <= 2e-2 and cosine >= 0.9995."""
    err = float(np.abs(got - ref).max())
    cos = cosine(got, ref)
    MARGINS.append((_test_id(), what, "bf16", err, cos))
    assert err <= 2e-2 and cos >= 0.9995, "%s: max abs err %.3g, cosine %.6f" % (what, err, cos)
    return err, cos


class OracleState:
    """Oracle-side caches of S streams in logical order."""

    def __init__(self, S, cfg):
        L, D, KC = cfg.left_context, cfg.d_model, cfg.conv_kernel - 1
        self.k = np.zeros((S, cfg.layers, L, D), np.float32)
        self.v = np.zeros((S, cfg.layers, L, D), np.float32)
        self.c = np.zeros((S, cfg.layers, KC, D), np.float32)
        self.len = np.zeros(S, np.int32)

    def seed_random(self, rng, cache_len, blocks=None):
        """N(0,1) caches.  blocks: draw only that many distinct [L, D] K and V windows and deal them
        to the (stream, layer) pairs in a fixed scrambled order (cheap for hundreds of streams x 24
        layers; neighbouring streams and layers still get different windows)."""
        if blocks is None:
            self.k[:] = rng.standard_normal(self.k.shape, dtype=np.float32)
            self.v[:] = rng.standard_normal(self.v.shape, dtype=np.float32)
        else:
            S, layers = self.k.shape[:2]
            kb = rng.standard_normal((blocks,) + self.k.shape[2:], dtype=np.float32)
            vb = rng.standard_normal((blocks,) + self.v.shape[2:], dtype=np.float32)
            for s in range(S):
                for l in range(layers):
                    self.k[s, l] = kb[(7 * s + 13 * l) % blocks]
                    self.v[s, l] = vb[(11 * s + 5 * l + 3) % blocks]
        self.c[:] = rng.standard_normal(self.c.shape, dtype=np.float32)
        self.len[:] = cache_len

    def import_into(self, streams, ud, bf16):
        """Loads these caches into the encoder's streams (a 16-bit encoder's K/V caches are IEEE
        half, rounded on import, so the oracle copy is rounded the same way)."""
        if bf16:
            self.k[:] = ud.round_f16(self.k)
            self.v[:] = ud.round_f16(self.v)
        for s, st in enumerate(streams):
            for l in range(self.k.shape[1]):
                st.import_cache(l, self.k[s, l], self.v[s, l], self.c[s, l], int(self.len[s]))


def speechlike(n, seed, scale=0.3):
    """Harmonics of a gliding 120 Hz pitch under a slow envelope, over low-level noise: a test
    signal with ~60 dB of spectral dynamic range (16 kHz)."""
    rng = np.random.default_rng(seed)
    t = np.arange(n) / 16000.0
    f0 = 120 + 40 * np.sin(2 * np.pi * 0.7 * t)
    ph = 2 * np.pi * np.cumsum(f0) / 16000.0
    x = sum(np.sin(h * ph) / h for h in range(1, 12)) * (0.2 + 0.15 * np.sin(2 * np.pi * 1.3 * t))
    return (scale * x + 1e-3 * rng.standard_normal(n)).astype(np.float32)
