"""ctypes binding of the CPU oracle (oracle/ud_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by the smoke entry point and by the benchmark's
cpu_baseline leg, as the parity reference and the timed CPU baseline.  The product path never imports it.

Each wrapper takes and returns float32/int32 numpy arrays (C-contiguous).  The reference file:line
each function restates is in the C source.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# UD_ORACLE_LIB: another build of ud_oracle.c (the mutation tests load planted-mistake builds)
LIB_PATH = os.environ.get("UD_ORACLE_LIB") or os.path.join(_HERE, "_build", "libud_oracle.so")

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)
_lib = None

# Per-layer weight order of the oracle (ConformerLayerWeights, FastConformer.swift:41-54), with the
# NeMo state_dict suffix of each slot.
WEIGHT_SUFFIXES = [
    "norm_feed_forward1.weight", "norm_feed_forward1.bias", "feed_forward1.linear1.weight",
    "feed_forward1.linear2.weight", "norm_self_att.weight", "norm_self_att.bias", "self_attn.linear_q.weight",
    "self_attn.linear_k.weight", "self_attn.linear_v.weight", "self_attn.linear_out.weight",
    "self_attn.linear_pos.weight", "self_attn.pos_bias_u", "self_attn.pos_bias_v", "norm_conv.weight",
    "norm_conv.bias", "conv.pointwise_conv1.weight", "conv.depthwise_conv.weight", "conv.batch_norm.weight",
    "conv.batch_norm.bias", "conv.pointwise_conv2.weight", "norm_feed_forward2.weight", "norm_feed_forward2.bias",
    "feed_forward2.linear1.weight", "feed_forward2.linear2.weight", "norm_out.weight", "norm_out.bias",
]

ACT_NONE, ACT_RELU, ACT_SILU, ACT_GELU_ERF = 0, 1, 2, 4

# Subsampling tensors (FastConformer.swift:56-95), in the order orc_subsample takes them.
SUB_WEIGHT_NAMES = [
    "encoder.pre_encode.conv.0.weight", "encoder.pre_encode.conv.0.bias",
    "encoder.pre_encode.conv.2.weight", "encoder.pre_encode.conv.2.bias",
    "encoder.pre_encode.conv.3.weight", "encoder.pre_encode.conv.3.bias",
    "encoder.pre_encode.conv.5.weight", "encoder.pre_encode.conv.5.bias",
    "encoder.pre_encode.conv.6.weight", "encoder.pre_encode.conv.6.bias",
    "encoder.pre_encode.out.weight", "encoder.pre_encode.out.bias",
]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            import importlib.util
            spec = importlib.util.spec_from_file_location("_ud_oracle_build", os.path.join(_HERE, "build.py"))
            mod = importlib.util.module_from_spec(spec)
            spec.loader.exec_module(mod)
            mod.build()
        _lib = ctypes.CDLL(LIB_PATH)
        _lib.orc_bf16_bits.restype = ctypes.c_uint16
        _lib.orc_bf16_bits.argtypes = [ctypes.c_float]
        _lib.orc_bf16_to_float.restype = ctypes.c_float
        _lib.orc_bf16_to_float.argtypes = [ctypes.c_uint16]
        _lib.orc_weight_count.restype = ctypes.c_int
    return _lib


def _p(a):
    return a.ctypes.data_as(_f32p) if a is not None else None


def _ip(a):
    return a.ctypes.data_as(_i32p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def set_threads(n):
    """Sets the OpenMP thread count of the oracle (the CPU baseline's core count)."""
    os.environ["OMP_NUM_THREADS"] = str(n)
    try:
        ctypes.CDLL("libgomp.so.1").omp_set_num_threads(int(n))
    except OSError:
        pass


class store_limit:
    """Context manager: the storage-range model of a 16-bit encoder (orc_set_store_limit) -- values
    stored in 16 bits clamp to [-limit, limit] -- for the duration of the block; 0 = off."""

    def __init__(self, limit):
        self.limit = float(limit)

    def __enter__(self):
        lib().orc_set_store_limit(ctypes.c_float(self.limit))
        return self

    def __exit__(self, *exc):
        lib().orc_set_store_limit(ctypes.c_float(0.0))
        return False


def lcg_floats(n, seed):
    out = np.empty(n, np.float32)
    lib().orc_lcg_floats(_p(out), ctypes.c_int64(n), ctypes.c_uint64(seed))
    return out


def bf16_bits(x):
    x = _f32(x).ravel()
    out = np.empty(x.shape, np.uint16)
    lib().orc_to_bf16(_p(x), out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), ctypes.c_int64(x.size))
    return out


def round_bf16(x):
    x = _f32(x).copy()
    lib().orc_round_bf16(_p(x), ctypes.c_int64(x.size))
    return x


def layer_norm(x, g, b, eps=1e-5, act=ACT_NONE):
    x = _f32(x)
    D = x.shape[-1]
    out = np.empty_like(x)
    lib().orc_layer_norm(_p(x), _p(_f32(g)), _p(_f32(b)) if b is not None else None, _p(out),
                         ctypes.c_int64(x.size // D), D, ctypes.c_float(eps), act)
    return out


def gemm_nt(A, W, bias=None, R=None, alpha=1.0, act=ACT_NONE, out_scale=1.0, res_scale=1.0):
    A, W = _f32(A), _f32(W)
    M, K = A.shape
    N = W.shape[0]
    C = np.empty((M, N), np.float32)
    lib().orc_gemm_nt(_p(A), _p(W), _p(_f32(bias)) if bias is not None else None,
                      _p(_f32(R)) if R is not None else None, _p(C), M, N, K, ctypes.c_float(alpha), act,
                      ctypes.c_float(out_scale), ctypes.c_float(res_scale))
    return C


def glu(x):
    x = _f32(x)
    T, D2 = x.shape
    out = np.empty((T, D2 // 2), np.float32)
    lib().orc_glu(_p(x), _p(out), ctypes.c_int64(T), D2 // 2)
    return out


def dwconv1d(x, w, bias=None, act=ACT_NONE):
    x, w = _f32(x), _f32(w)
    D, K = w.shape
    Tout = x.shape[0] - K + 1
    out = np.empty((Tout, D), np.float32)
    lib().orc_dwconv1d(_p(x), _p(w), _p(_f32(bias)) if bias is not None else None, _p(out), Tout, D, K, act)
    return out


def sinusoid(pos, D):
    out = np.empty(D, np.float32)
    lib().orc_sinusoid(int(pos), D, _p(out))
    return out


def pe_rows(lo, hi, D):
    out = np.empty((hi - lo + 1, D), np.float32)
    lib().orc_pe_rows(lo, hi, D, _p(out))
    return out


def pos_table(wpos, lo, hi):
    wpos = _f32(wpos)
    D = wpos.shape[0]
    P = np.empty((hi - lo + 1, D), np.float32)
    lib().orc_pos_table(_p(wpos), lo, hi, D, _p(P))
    return P


def relpos_attention(q, k, v, P, u, vb, ranges, rel_offset, H):
    """q [Tq, H*dk], k/v [Tk, H*dk], P [n_rel, H*dk], u/vb [H, dk], ranges int32 [Tq, 2]."""
    q, k, v, P = _f32(q), _f32(k), _f32(v), _f32(P)
    Tq, HD = q.shape
    Tk = k.shape[0]
    dk = HD // H
    out = np.empty_like(q)
    rr = np.ascontiguousarray(ranges, dtype=np.int32)
    lib().orc_relpos_attention(_p(q), _p(k), _p(v), _p(P), _p(_f32(u)), _p(_f32(vb)), _ip(rr), _p(out),
                               Tq, Tk, H, dk, HD, HD, HD, HD, rel_offset, P.shape[0],
                               ctypes.c_float(1.0 / np.sqrt(np.float32(dk))))
    return out


def gqa_attention(q, k, v, ranges, Hq, Hkv, scale=None):
    """attention_gqa (30_voxtral.metal:45-101): q [Tq, Hq*d], k/v [Tk, Hkv*d], ranges int32 [Tq, 2]."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    Tq, QW = q.shape
    d = QW // Hq
    Tk = k.shape[0]
    out = np.empty_like(q)
    rr = np.ascontiguousarray(ranges, dtype=np.int32)
    if scale is None:
        scale = 1.0 / np.sqrt(np.float32(d))
    lib().orc_gqa_attention(_p(q), _p(k), _p(v), _ip(rr), _p(out), Tq, Tk, Hq, Hkv, d, QW, Hkv * d, QW,
                            ctypes.c_float(scale))
    return out


def rope_rotate_half(x, H, d, inv_freq, positions=None, pos0=0):
    """rope_rotate_half (30_voxtral.metal:20-36) on a copy of x [T, ld]."""
    y = _f32(x).copy()
    T, ld = y.shape
    pos = None if positions is None else np.ascontiguousarray(positions, dtype=np.int32)
    lib().orc_rope_rotate_half(_p(y), T, H, d, ld, _ip(pos) if pos is not None else None, pos0, _p(_f32(inv_freq)))
    return y


def chunked_limited_ranges(T, left, right):
    r = np.empty((T, 2), np.int32)
    lib().orc_chunked_limited_ranges(T, left, right, _ip(r))
    return r


class Model:
    """Oracle-side model: per-layer fp32 weight arrays (keyed by NeMo suffix) and the position
    tables P_l over rel = lo..hi (FastConformer.swift:161-178)."""

    def __init__(self, layer_weights, D, H, ff, Kc):
        self.layers = [[_f32(lw[s]) for s in WEIGHT_SUFFIXES] for lw in layer_weights]
        self.D, self.H, self.ff, self.Kc = D, H, ff, Kc
        self._ptrs = None
        self.P = None

    def prepare(self, lo, hi):
        D = self.D
        self.lo, self.hi = lo, hi
        self.rel_offset = -lo
        self.P = [pos_table(lw[WEIGHT_SUFFIXES.index("self_attn.linear_pos.weight")], lo, hi) for lw in self.layers]
        flat = [w for lw in self.layers for w in lw]
        self._keep = flat
        self._wptrs = (_f32p * len(flat))(*[_p(w) for w in flat])
        self._pptrs = (_f32p * len(self.P))(*[_p(p) for p in self.P])
        return self

    @property
    def n_rel(self):
        return self.P[0].shape[0]


def stream_step(model, x, valid, kcache, vcache, ccache, cache_len):
    """encodeStreamStep for S streams (FastConformer.swift:441-480).

    x [S, T, D]; valid int32 [S]; kcache/vcache [S, layers, L, D]; ccache [S, layers, K-1, D];
    cache_len int32 [S].  The caches and cache_len are updated in place; returns out [S, T, D]."""
    x = _f32(x)
    S, T, D = x.shape
    layers = len(model.layers)
    L = kcache.shape[2]
    for a in (kcache, vcache, ccache):
        assert a.dtype == np.float32 and a.flags.c_contiguous
    assert cache_len.dtype == np.int32
    out = np.empty_like(x)
    lib().orc_stream_step(model._wptrs, model._pptrs, model.rel_offset, model.n_rel, layers, S, T, L, D,
                          model.H, model.ff, model.Kc, _p(x), _ip(np.ascontiguousarray(valid, np.int32)),
                          _p(kcache), _p(vcache), _p(ccache), _ip(cache_len), _p(out))
    return out


def encoder_offline(model, x, ranges, valid):
    """forwardOffline after the subsampling (FastConformer.swift:361-398); x [T, D], ranges [T, 2]."""
    x = _f32(x)
    T, D = x.shape
    out = np.empty_like(x)
    lib().orc_encoder_offline(model._wptrs, model._pptrs, model.rel_offset, model.n_rel, len(model.layers), T, D,
                              model.H, model.ff, model.Kc, _p(x), _ip(np.ascontiguousarray(ranges, np.int32)),
                              int(valid), _p(out))
    return out


def conv2d_cl(x, w, bias, stride, pad_top, pad_left, groups, act=ACT_NONE, valid_h=None, out_hw=None):
    """conv2d_cl (20_conformer.metal:104-138): x [Hin, Win, Cin] channel-last, w [Cout, Cin/groups,
    KH, KW]; out [Hout, Wout, Cout] with Hout/Wout from out_hw or the causal rule (L + 2 pads - K)/s + 1
    with one bottom/right pad row (Ops.swift callers)."""
    x = _f32(x)
    w = _f32(w)
    Hin, Win, Cin = x.shape
    Cout, _, KH, KW = w.shape
    if out_hw is None:
        Hout = (Hin + pad_top + 1 - KH) // stride + 1
        Wout = (Win + pad_left + 1 - KW) // stride + 1
    else:
        Hout, Wout = out_hw
    out = np.empty((Hout, Wout, Cout), np.float32)
    lib().orc_conv2d_cl(_p(x), Hin, Win, Cin, _p(w), _p(_f32(bias)), _p(out), Hout, Wout, Cout, KH, KW, stride,
                        pad_top, pad_left, groups, act, Hout if valid_h is None else valid_h)
    return out


def sub_next_len(t):
    """Causal stride-2 stage length (FastConformer.swift:219): t // 2 + 1."""
    return t // 2 + 1


def subsample(mel, valid_mel, sw, C=256, D=1024):
    """encodeSubsampling (FastConformer.swift:219-243): mel [T0, 128] -> [T3, D].  sw maps the
    names in SUB_WEIGHT_NAMES to arrays in the checkpoint layout (out.weight columns in
    (channel, freq) order)."""
    mel = _f32(mel)
    T0, F0 = mel.shape
    T3 = sub_next_len(sub_next_len(sub_next_len(T0)))
    ws = [_f32(sw[n]).reshape(-1) for n in SUB_WEIGHT_NAMES]
    ptrs = (_f32p * len(ws))(*[_p(w) for w in ws])
    out = np.empty((T3, D), np.float32)
    got = lib().orc_subsample(_p(mel), T0, F0, int(valid_mel), ptrs, C, D, _p(out))
    assert got == T3
    return out


def rnnt_weight_names(layers=2):
    """RNN-T prediction + joint tensors (RNNTDecoder.init, RNNT.swift:27-63) in the oracle's order."""
    names = ["decoder.prediction.embed.weight"]
    for l in range(layers):
        names += ["decoder.prediction.dec_rnn.lstm.%s_l%d" % (k, l) for k in ("weight_ih", "weight_hh", "bias_ih", "bias_hh")]
    return names + ["joint.pred.weight", "joint.pred.bias", "joint.joint_net.2.weight", "joint.joint_net.2.bias"]


class RnntState:
    """RNNTDecoder.State (RNNT.swift:18-26) of one stream: committed h, c [L, H], last token, and
    the cached prediction for it (committed when a non-blank token is emitted)."""

    def __init__(self, H, V, L):
        self.h = np.zeros((L, H), np.float32)
        self.c = np.zeros((L, H), np.float32)
        self.last = np.array([V - 1], np.int32)
        self.pending = np.zeros(1, np.int32)
        self.pproj = np.zeros(H, np.float32)
        self.ph = np.zeros((L, H), np.float32)
        self.pc = np.zeros((L, H), np.float32)


class Rnnt:
    """Oracle RNN-T decoder over a dict of checkpoint tensors."""

    def __init__(self, w, max_symbols=10):
        self.V, self.H = np.asarray(w["decoder.prediction.embed.weight"]).shape
        self.L = 0
        while "decoder.prediction.dec_rnn.lstm.weight_ih_l%d" % self.L in w:
            self.L += 1
        self._keep = [_f32(w[n]).reshape(-1) for n in rnnt_weight_names(self.L)]
        self._ptrs = (_f32p * len(self._keep))(*[_p(a) for a in self._keep])
        self.max_symbols = max_symbols

    def state(self):
        return RnntState(self.H, self.V, self.L)

    def greedy(self, enc_proj, st, cap=4096):
        """Greedy decode of projected frames [frames, H] from state st (updated); returns the tokens."""
        enc_proj = _f32(enc_proj)
        toks = np.zeros(cap, np.int32)
        n = lib().orc_rnnt_greedy(self._ptrs, self.H, self.V, self.L, _p(enc_proj), enc_proj.shape[0], self.max_symbols,
                                  _p(st.h), _p(st.c), _ip(st.last), _ip(st.pending), _p(st.pproj), _p(st.ph),
                                  _p(st.pc), _ip(toks), cap)
        return [int(t) for t in toks[:min(n, cap)]]

    def predict(self, token, h, c):
        proj = np.zeros(self.H, np.float32)
        ho = np.zeros((self.L, self.H), np.float32)
        co = np.zeros((self.L, self.H), np.float32)
        lib().orc_rnnt_predict(self._ptrs, self.H, self.V, self.L, int(token), _p(_f32(h)), _p(_f32(c)), _p(proj),
                               _p(ho), _p(co))
        return proj, ho, co


# ---------------------------------------------------------------- mel frontend and streaming

MEL_FFT, MEL_HOP, MEL_WIN, MEL_FFT_BINS = 512, 160, 400, 257


class MelFrontend:
    """NemoMelFrontend (Sources/DictatorCore/Audio/NemoMel.swift:11-108) over the C restatement:
    fb [n_mels, 257], window [400] (the checkpoint's preprocessor.featurizer buffers)."""

    def __init__(self, fb, window):
        self.fb = _f32(fb).reshape(-1, MEL_FFT_BINS)
        self.n_mels = self.fb.shape[0]
        self.window = _f32(window).reshape(MEL_WIN)
        self.cos_t = np.empty((MEL_FFT_BINS, MEL_WIN), np.float32)
        self.sin_t = np.empty((MEL_FFT_BINS, MEL_WIN), np.float32)
        lib().orc_mel_tables(_p(self.window), _p(self.cos_t), _p(self.sin_t))

    @staticmethod
    def valid_frames(samples):
        return samples // MEL_HOP

    def frames(self, audio, f0, nf, valid_end):
        audio = _f32(audio)
        out = np.empty((nf, self.n_mels), np.float32)
        lib().orc_mel_frames(_p(audio), ctypes.c_int64(audio.size), ctypes.c_int64(f0), int(nf),
                             ctypes.c_int64(valid_end), _p(self.cos_t), _p(self.sin_t), _p(self.fb), self.n_mels,
                             _p(out))
        return out

    def features(self, audio):
        """Full-utterance features [n // 160 + 1, n_mels], the last frame zero (NemoMel.swift:46-67)."""
        n = int(np.asarray(audio).size)
        return self.frames(audio, 0, n // MEL_HOP + 1, n // MEL_HOP)


class MelStream:
    """NemoMelStream (NemoMel.swift:113-161): push audio in any sizes, frames come out once their
    window is complete; finish() emits the tail exactly as features() would."""

    def __init__(self, fe):
        self.fe = fe
        self.audio = np.zeros(0, np.float32)
        self.emitted = 0

    def _emit(self, end, valid):
        if end <= self.emitted:
            return np.zeros((0, self.fe.n_mels), np.float32)
        out = self.fe.frames(self.audio, self.emitted, end - self.emitted, valid)
        self.emitted = end
        return out

    def push(self, samples):
        self.audio = np.concatenate([self.audio, _f32(samples).ravel()])
        n = self.audio.size
        ready = (n - 200) // MEL_HOP + 1 if n >= 200 else 0
        return self._emit(ready, 1 << 62)

    def finish(self):
        n = self.audio.size
        return self._emit(n // MEL_HOP + 1, n // MEL_HOP)


class Schedule:
    """NemotronSchedule (Sources/DictatorCore/Nemotron/NemotronSchedule.swift:7-17)."""

    def __init__(self, lookahead):
        self.lookahead = lookahead
        self.left_context = 70
        self.pre_encode_cache = 9
        self.drop_extra = 2
        self.first_chunk = 1 + 8 * lookahead
        self.chunk = 8 + 8 * lookahead
        self.out_frames_per_chunk = lookahead + 1


class Streamer:
    """NemotronStreamer (Sources/DictatorCore/Nemotron/NemotronStreamer.swift:16-153) driving the
    oracle encoder step of MetalNemotronEncoder.step (Sources/DictatorEngine/Models/Nemotron.swift:
    74-92): subsampling + drop, the stream step, joint.enc on the kept frames, greedy RNN-T.
    One stream; every chunk runs at its own (unpadded) size, as the reference does.

    model: an oracle Model prepared for the rel range of the schedule; sw: subsampling weights;
    rw: RNN-T weights (joint.enc included); fe: a MelFrontend (live input only)."""

    def __init__(self, model, sw, rw, lookahead, fe=None, layers=None):
        self.model, self.sw, self.fe = model, sw, fe
        self.schedule = Schedule(lookahead)
        self.dec = Rnnt(rw)
        self.dec_state = self.dec.state()
        self.w_enc = _f32(rw["joint.enc.weight"])
        self.b_enc = _f32(rw["joint.enc.bias"])
        nl = len(model.layers)
        L, D, Kc = self.schedule.left_context, model.D, model.Kc
        self.k = np.zeros((1, nl, L, D), np.float32)
        self.v = np.zeros((1, nl, L, D), np.float32)
        self.c = np.zeros((1, nl, Kc, D), np.float32)
        self.len = np.zeros(1, np.int32)
        self.steps = 0
        self.tokens = []
        self.enc_rows = []          # kept encoder output rows per chunk
        self.proj_rows = []         # kept joint.enc rows per chunk
        self.end_padding = True
        self.live_mel = MelStream(fe) if fe is not None else None
        self.live_buffer = np.zeros((0, fe.n_mels if fe is not None else 128), np.float32)
        self.live_start = 0
        self.live_next = 0

    def encoder_step(self, mel_rows, n_rows, valid_rows, keep_all):
        s = self.schedule
        drop = 0 if self.steps == 0 else s.drop_extra
        x = subsample(mel_rows[:n_rows], valid_rows, self.sw)[drop:]
        T = x.shape[0]
        vs = sub_next_len(sub_next_len(sub_next_len(valid_rows)))
        valid_t = max(0, min(vs - drop, T))
        y = stream_step(self.model, x[None], np.array([valid_t], np.int32), self.k, self.v, self.c, self.len)[0]
        self.steps += 1
        keep = valid_t if keep_all else min(valid_t, s.out_frames_per_chunk)
        if keep == 0:
            return np.zeros((0, self.w_enc.shape[0]), np.float32), y[:0]
        proj = gemm_nt(y[:keep], self.w_enc, bias=self.b_enc)
        return proj, y[:keep]

    def step(self, mel_rows, n_rows, valid_rows, keep_all):
        proj, y = self.encoder_step(mel_rows, n_rows, valid_rows, keep_all)
        new = self.dec.greedy(proj, self.dec_state) if proj.shape[0] > 0 else []
        self.tokens += new
        self.enc_rows.append(y)
        self.proj_rows.append(proj)
        return new

    def run_buffered(self, mel, frames, valid_frames):
        """runBuffered (NemotronStreamer.swift:70-91)."""
        s = self.schedule
        idx = 0
        while idx < frames:
            first = idx == 0
            size = s.first_chunk if first else s.chunk
            end = min(idx + size, frames)
            chunk_len = end - idx
            if chunk_len < (1 if first else 8):
                return
            cache_start = idx if first else max(0, idx - s.pre_encode_cache)
            added = idx - cache_start
            rows = added + chunk_len
            valid = max(0, min(valid_frames - idx + added, rows))
            idx += size
            self.step(mel[cache_start:cache_start + rows], rows, valid, idx >= frames)

    def push(self, samples):
        self.live_buffer = np.concatenate([self.live_buffer, self.live_mel.push(samples)])
        return self._drain(False)

    def flush(self):
        self.live_buffer = np.concatenate([self.live_buffer, self.live_mel.finish()])
        return self._drain(True)

    def _drain(self, final):
        """drainChunks (NemotronStreamer.swift:109-153)."""
        s = self.schedule
        have = self.live_buffer.shape[0] + self.live_start
        out = []
        while True:
            idx = self.live_next
            first = idx == 0
            size = s.first_chunk if first else s.chunk
            end = idx + size
            if end > have and not final:
                break
            chunk_end = min(end, have)
            chunk_len = chunk_end - idx
            min_len = 1 if first else 8
            if chunk_len <= 0 or (chunk_len < min_len and not (final and self.end_padding)):
                break
            cache_start = idx if first else max(0, idx - s.pre_encode_cache)
            rows = chunk_end - cache_start
            pad_rows = max(0, min_len - chunk_len)
            is_last = final and end >= have
            a = cache_start - self.live_start
            m = self.live_buffer[a:a + rows]
            if pad_rows > 0:
                m = np.concatenate([m, np.zeros((pad_rows, m.shape[1]), np.float32)])
                out += self.step(m, rows + pad_rows, rows, True)
            else:
                out += self.step(m, rows, rows, is_last)
            self.live_next = end
            keep_from = self.live_next - s.pre_encode_cache
            if keep_from > self.live_start:
                drop = min(self.live_buffer.shape[0], keep_from - self.live_start)
                self.live_buffer = self.live_buffer[drop:]
                self.live_start = keep_from
            if is_last:
                break
        return out


# ---------------------------------------------------------------- SentencePiece detokenizer
# Pure Python restatement of SentencePieceDecoder (Sources/DictatorCore/Decoding/SentencePiece.swift:
# 5-31).  Pinned by the sentencepiece package's own decoder on a trained model (byte fallback
# included), by the Unicode Standard's maximal-subpart example for ill-formed UTF-8, and by
# hand-built cases of the Swift rules (tests/test_tokenizer.py).

def sp_parse_vocab(data):
    """SentencePiece.swift:8-13: the vocabulary file's bytes -> pieces (str), id = index.  The text
    must be UTF-8 (String(contentsOf:encoding: .utf8) throws otherwise: UnicodeDecodeError here).
    Lines end at a '\n' not preceded by '\r' ("\r\n" is one Swift Character, which '\n' does not
    match); empty lines are dropped; a line's piece is its first non-empty tab-separated field
    (Swift's split omits empty subsequences), '' when there is none."""
    text = bytes(data).decode("utf-8")
    lines, start = [], 0
    for i, ch in enumerate(text):
        if ch == "\n" and not (i > 0 and text[i - 1] == "\r"):
            lines.append(text[start:i])
            start = i + 1
    lines.append(text[start:])
    pieces = []
    for line in lines:
        if not line:
            continue
        fields = [f for f in line.split("\t") if f]
        pieces.append(fields[0] if fields else "")
    return pieces


def sp_decode(pieces, ids):
    """SentencePiece.swift:17-30: ids -> UTF-8 bytes of the text.  Out-of-range ids are skipped;
    "<0xHH>" (two hex digits) is a raw byte; <unk>, <s>, </s>, <pad> add nothing; other pieces add
    their UTF-8 with U+2581 replaced by a space.  The bytes are read as UTF-8 with each maximal
    ill-formed subpart replaced by U+FFFD (CPython's errors="replace" follows the same Unicode
    practice as Swift's String(decoding:as:)), and one leading space is dropped."""
    out = bytearray()
    hexd = "0123456789abcdefABCDEF"
    for i in ids:
        i = int(i)
        if i < 0 or i >= len(pieces):
            continue
        p = pieces[i]
        if len(p) == 6 and p.startswith("<0x") and p.endswith(">") and p[3] in hexd and p[4] in hexd:
            out.append(int(p[3:5], 16))
        elif p in ("<unk>", "<s>", "</s>", "<pad>"):
            continue
        else:
            out += p.replace("\u2581", " ").encode("utf-8")
    s = bytes(out).decode("utf-8", errors="replace")
    if s.startswith(" "):
        s = s[1:]
    return s.encode("utf-8")
