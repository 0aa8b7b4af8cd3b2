"""Host-side binding of the MI355X (gfx950) streaming FastConformer encoder step.

Mirrors the reference's encoder-step interface over the C ABI in include/ud_encoder.h:

  Encoder            FastConformerEncoder (Sources/DictatorEngine/Models/FastConformer.swift:62-144)
  Encoder.new_stream FastConformerEncoder.makeStreamState (FastConformer.swift:431-435)
  Encoder.encode_stream_step
                     encodeStreamStep (FastConformer.swift:441-480), batched over streams
  rel_pos_attention  Step.relPosAttention (Sources/DictatorEngine/Core/Ops.swift:80-90)
  EngineError        EngineError.io (Sources/DictatorCore/Errors.swift:3-11)

All compute runs in libud_encoder.so (hand-written HIP for gfx950).  There is no CPU fallback:
loading raises EngineError when the library is missing or no HIP device is present.
Device buffers are DeviceBuffer objects (HBM allocations owned by the library's allocator).
"""
import ctypes
import dataclasses
import os

import numpy as np

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "lib", "libud_encoder.so")
INCLUDE_DIR = os.path.join(os.path.dirname(PKG_DIR), "include")

UD_F32, UD_BF16, UD_F16 = 0, 1, 2
_DTYPES = {"f32": UD_F32, "fp32": UD_F32, "float32": UD_F32, "bf16": UD_BF16, "bfloat16": UD_BF16,
           "f16": UD_F16, "float16": UD_F16}

STATUS = {0: "ok", -1: "invalid argument", -2: "shape", -3: "out of memory", -4: "HIP error", -5: "state",
          -6: "weight", -7: "capacity"}


class EngineError(RuntimeError):
    """A failed library call: status code and the library's message (EngineError.io)."""

    def __init__(self, status, message):
        super().__init__("%s (%d): %s" % (STATUS.get(status, "error"), status, message))
        self.status = status


class _Config(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("layers", "d_model", "heads", "ff_dim", "conv_kernel",
                                               "left_context", "max_chunk", "max_streams", "dtype")]


_lib = None
_vp = ctypes.c_void_p
_i32 = ctypes.c_int32


def _sig(lib):
    i, v, p, f = ctypes.c_int, None, _vp, ctypes.POINTER(ctypes.c_float)
    ip = ctypes.POINTER(_i32)
    sigs = {
        "ud_last_error": (ctypes.c_char_p, []),
        "ud_encoder_create": (i, [ctypes.POINTER(_Config), ctypes.POINTER(_vp)]),
        "ud_encoder_destroy": (v, [p]),
        "ud_encoder_set_weight": (i, [p, ctypes.c_char_p, f, ctypes.c_int64]),
        "ud_encoder_finalize": (i, [p]),
        "ud_stream_create": (i, [p, ctypes.POINTER(_vp)]),
        "ud_stream_reset": (i, [p]),
        "ud_stream_destroy": (v, [p]),
        "ud_stream_info": (i, [p, ip, ip]),
        "ud_encoder_step": (i, [p, ctypes.POINTER(_vp), _i32, _i32, p, ip, p, p]),
        "ud_encoder_subsample": (i, [p, _i32, _i32, p, ip, _i32, p, ip, ip, p]),
        "ud_stream_export_cache": (i, [p, _i32, f, f, f, ip]),
        "ud_stream_import_cache": (i, [p, _i32, f, f, f, _i32]),
        "ud_relpos_attention": (i, [_i32, p, p, p, p, p, p, p, p, _i32, _i32, _i32, _i32, _i32, _i32, p]),
        "ud_relpos_attention_batched": (i, [_i32, p, p, p, p, p, p, p, p, _i32, _i32, _i32, _i32, _i32, _i32, p]),
        "ud_layer_attention": (i, [p, ctypes.POINTER(_vp), _i32, _i32, _i32, p, ip, p, p]),
        "ud_chunked_limited_ranges": (i, [_i32, _i32, _i32, ip, _i32, _i32, _i32, ip]),
        "ud_stream_advance": (i, [ctypes.POINTER(_vp), _i32, _i32]),
        "ud_time_projection": (i, [p, _i32, _i32, _i32, p, f, ctypes.POINTER(ctypes.c_double)]),
        "ud_measure_hbm": (i, [ctypes.c_size_t, _i32, p, f, f]),
        "ud_measure_mfma": (i, [_i32, p, f, f]),
        "ud_time_layer_attention": (i, [p, ctypes.POINTER(_vp), _i32, _i32, _i32, p, p, _i32, p, f]),
        "ud_time_ring_read_floor": (i, [p, ctypes.POINTER(_vp), _i32, _i32, _i32, p, p, _i32, p, f]),
        "ud_device_count": (i, [ip]),
        "ud_device_arch": (i, [ctypes.c_char_p, _i32]),
        "ud_malloc": (i, [ctypes.POINTER(_vp), ctypes.c_size_t]),
        "ud_free": (i, [p]),
        "ud_memcpy_htod": (i, [p, p, ctypes.c_size_t]),
        "ud_memcpy_dtoh": (i, [p, p, ctypes.c_size_t]),
        "ud_memcpy_dtod": (i, [p, p, ctypes.c_size_t]),
        "ud_memset": (i, [p, _i32, ctypes.c_size_t]),
        "ud_device_synchronize": (i, []),
        "ud_mem_get_info": (i, [ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]),
        "ud_graph_capture_begin": (i, [p]),
        "ud_graph_capture_end": (i, [p, ctypes.POINTER(_vp)]),
        "ud_graph_launch": (i, [p, p]),
        "ud_graph_destroy": (i, [p]),
        "ud_hip_stream_create": (i, [ctypes.POINTER(_vp)]),
        "ud_hip_stream_destroy": (i, [p]),
        "ud_hip_stream_synchronize": (i, [p]),
        "ud_event_create": (i, [ctypes.POINTER(_vp)]),
        "ud_event_destroy": (i, [p]),
        "ud_event_record": (i, [p, p]),
        "ud_event_synchronize": (i, [p]),
        "ud_event_elapsed_ms": (i, [f, p, p]),
        "ud_gqa_workspace_bytes": (ctypes.c_size_t, [_i32, _i32, _i32, _i32]),
        "ud_gqa_attention_paged": (i, [_i32, p, p, p, p, _i32, p, p, _i32, _i32, _i32, _i32, _i32, _i32, p,
                                       ctypes.c_size_t, p]),
        "ud_gqa_attention_paged_noalloc": (i, [_i32, p, p, p, p, _i32, p, p, _i32, _i32, _i32, _i32, _i32, _i32,
                                               p]),
        "ud_gqa_attention_paged_mq": (i, [_i32, p, p, p, p, _i32, p, p, _i32, _i32, _i32, _i32, _i32, _i32, _i32, p,
                                          ctypes.c_size_t, p]),
        "ud_rope_rotate_half": (i, [_i32, p, _i32, _i32, _i32, _i32, p, _i32, p, p]),
        "ud_paged_kv_append": (i, [_i32, p, p, p, p, p, _i32, p, _i32, _i32, _i32, _i32, p]),
        "ud_encoder_get_config": (i, [p, ctypes.POINTER(_Config)]),
        "ud_safetensors_open": (i, [ctypes.c_char_p, ctypes.POINTER(_vp)]),
        "ud_safetensors_close": (v, [p]),
        "ud_safetensors_count": (_i32, [p]),
        "ud_safetensors_name": (ctypes.c_char_p, [p, _i32]),
        "ud_safetensors_info": (i, [p, ctypes.c_char_p, ip, ctypes.POINTER(ctypes.c_int64), ip]),
        "ud_safetensors_read_f32": (i, [p, ctypes.c_char_p, f, ctypes.c_int64]),
        "ud_nemo_name": (i, [ctypes.c_char_p, ctypes.c_char_p, _i32]),
        "ud_encoder_load_safetensors": (i, [p, p, ip]),
        "ud_rnnt_load_safetensors": (i, [p, p, ip]),
        "ud_rnnt_create": (i, [_i32, _i32, _i32, _i32, _i32, _i32, ctypes.POINTER(_vp)]),
        "ud_rnnt_destroy": (v, [p]),
        "ud_rnnt_set_weight": (i, [p, ctypes.c_char_p, f, ctypes.c_int64]),
        "ud_rnnt_reset": (i, [p, _i32]),
        "ud_rnnt_project": (i, [p, _i32, p, p, p]),
        "ud_rnnt_greedy": (i, [p, _i32, ip, p, _i32, ip, ip, _i32, ip, p]),
        "ud_rnnt_get_info": (i, [p, ip, ip, ip, ip, ip, ip]),
        "ud_mel_create": (i, [f, _i32, f, ctypes.POINTER(_vp)]),
        "ud_mel_destroy": (v, [p]),
        "ud_mel_bins": (_i32, [p]),
        "ud_mel_features": (i, [p, _i32, p, ctypes.c_int64, ctypes.POINTER(ctypes.c_int64), p, _i32, ip, p]),
        "ud_mel_load_safetensors": (i, [p, ctypes.POINTER(_vp)]),
        "ud_streamer_create": (i, [p, p, p, _i32, _i32, ctypes.POINTER(_vp)]),
        "ud_streamer_destroy": (v, [p]),
        "ud_streamer_open": (i, [p, ip]),
        "ud_streamer_close": (i, [p, _i32]),
        "ud_streamer_set_options": (i, [p, _i32, _i32]),
        "ud_streamer_push": (i, [p, _i32, p, p, p]),       # ids int32[n], samples float*[n], counts int64[n]
        "ud_streamer_flush": (i, [p, _i32, ip]),
        "ud_streamer_run_buffered": (i, [p, _i32, ip, ctypes.POINTER(f), ip, ip]),
        "ud_streamer_tokens": (i, [p, _i32, ip, _i32, ip]),
        "ud_streamer_recorded": (i, [p, _i32, _i32, f, ctypes.c_int64, ctypes.POINTER(ctypes.c_int64)]),
        "ud_streamer_stats": (i, [p, ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64)]),
        "ud_streamer_emissions": (i, [p, _i32, ip, ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_double), _i32, ip]),
        "ud_streamer_step_times": (i, [p, _i32, ctypes.POINTER(ctypes.c_double), _i32, ip]),
        "ud_nemotron_step": (i, [p, p, ctypes.POINTER(_vp), _i32, _i32, p, ip, ip, _i32, _i32, p, _i32, ip, p]),
        "ud_tokenizer_load": (i, [ctypes.c_char_p, ctypes.POINTER(_vp)]),
        "ud_tokenizer_parse": (i, [ctypes.c_char_p, ctypes.c_int64, ctypes.POINTER(_vp)]),
        "ud_tokenizer_destroy": (v, [p]),
        "ud_tokenizer_size": (i, [p, ip]),
        "ud_tokenizer_piece": (i, [p, _i32, ctypes.c_char_p, ctypes.c_int64, ctypes.POINTER(ctypes.c_int64)]),
        "ud_tokenizer_decode": (i, [p, ip, _i32, ctypes.c_char_p, ctypes.c_int64, ctypes.POINTER(ctypes.c_int64)]),
        "ud_streamer_text": (i, [p, _i32, p, ctypes.c_char_p, ctypes.c_int64, ctypes.POINTER(ctypes.c_int64)]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def load_library(path=LIB_PATH):
    """Loads libud_encoder.so (no device check).  Raises EngineError if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(path):
            raise EngineError(-5, "libud_encoder.so is not built (run universal-dictator_amd/build.py): " + path)
        _lib = _sig(ctypes.CDLL(path))
    return _lib


def _check(rc):
    if rc != 0:
        raise EngineError(rc, (_lib.ud_last_error() or b"").decode())


def lib():
    """The library, after checking that a HIP device is present."""
    l = load_library()
    n = _i32(0)
    rc = l.ud_device_count(ctypes.byref(n))
    if rc != 0 or n.value < 1:
        raise EngineError(-4, "no HIP device visible: the encoder step runs only on the GPU")
    return l


def measure_hbm(nbytes=1 << 30, iters=10, hip_stream=None):
    """(read GB/s, copy GB/s) of this device: streaming kernels over nbytes buffers."""
    r, c = ctypes.c_float(0), ctypes.c_float(0)
    _check(lib().ud_measure_hbm(nbytes, iters, hip_stream.ptr if hip_stream else None, ctypes.byref(r), ctypes.byref(c)))
    return r.value, c.value


def measure_mfma(iters=20000, hip_stream=None):
    """(f16 TFLOP/s, bf16 TFLOP/s) of dense register-only MFMA chains on this device."""
    h, b = ctypes.c_float(0), ctypes.c_float(0)
    _check(lib().ud_measure_mfma(iters, hip_stream.ptr if hip_stream else None, ctypes.byref(h), ctypes.byref(b)))
    return h.value, b.value


def device_arch():
    buf = ctypes.create_string_buffer(64)
    _check(lib().ud_device_arch(buf, 64))
    return buf.value.decode()


def synchronize():
    _check(lib().ud_device_synchronize())


def mem_get_info():
    """(free, total) bytes of device memory (hipMemGetInfo)."""
    f, t = ctypes.c_size_t(0), ctypes.c_size_t(0)
    _check(lib().ud_mem_get_info(ctypes.byref(f), ctypes.byref(t)))
    return f.value, t.value


class Graph:
    """Work captured from a HipStream into a HIP graph: `with Graph.capture(stream) as g:` records
    the calls made on that stream inside the block; g.launch(stream) replays them."""

    def __init__(self):
        self.ptr = None

    @classmethod
    def capture(cls, stream):
        g = cls()
        g._stream = stream
        return g

    def __enter__(self):
        _check(lib().ud_graph_capture_begin(self._stream.ptr))
        return self

    def __exit__(self, exc_type, exc, tb):
        p = _vp()
        rc = _lib.ud_graph_capture_end(self._stream.ptr, ctypes.byref(p))
        self.ptr = p.value
        if exc_type is None:
            _check(rc)
        return False

    def launch(self, stream):
        _check(_lib.ud_graph_launch(self.ptr, stream.ptr))

    def __del__(self):
        try:
            if self.ptr:
                _lib.ud_graph_destroy(self.ptr)
        except Exception:
            pass


# ---------------------------------------------------------------- device memory, streams, events

class DeviceBuffer:
    """An HBM allocation."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        p = _vp()
        _check(lib().ud_malloc(ctypes.byref(p), self.nbytes))
        self.ptr = p.value

    @classmethod
    def from_numpy(cls, a):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    @classmethod
    def zeros(cls, nbytes):
        b = cls(nbytes)
        _check(lib().ud_memset(b.ptr, 0, b.nbytes))
        return b

    def upload(self, a):
        a = np.ascontiguousarray(a)
        if a.nbytes > self.nbytes:
            raise EngineError(-2, "upload of %d bytes into a %d-byte buffer" % (a.nbytes, self.nbytes))
        _check(_lib.ud_memcpy_htod(self.ptr, a.ctypes.data, a.nbytes))

    def download(self, shape, dtype=np.float32):
        out = np.empty(shape, dtype)
        if out.nbytes > self.nbytes:
            raise EngineError(-2, "download of %d bytes from a %d-byte buffer" % (out.nbytes, self.nbytes))
        _check(_lib.ud_memcpy_dtoh(out.ctypes.data, self.ptr, out.nbytes))
        return out

    def free(self):
        if self.ptr:
            _lib.ud_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class HipStream:
    def __init__(self):
        p = _vp()
        _check(lib().ud_hip_stream_create(ctypes.byref(p)))
        self.ptr = p.value

    def synchronize(self):
        _check(_lib.ud_hip_stream_synchronize(self.ptr))

    def __del__(self):
        try:
            if self.ptr:
                _lib.ud_hip_stream_destroy(self.ptr)
        except Exception:
            pass


class Event:
    def __init__(self):
        p = _vp()
        _check(lib().ud_event_create(ctypes.byref(p)))
        self.ptr = p.value

    def record(self, stream=None):
        _check(_lib.ud_event_record(self.ptr, stream.ptr if stream else None))

    def synchronize(self):
        _check(_lib.ud_event_synchronize(self.ptr))

    def elapsed_ms(self, end):
        ms = ctypes.c_float(0)
        _check(_lib.ud_event_elapsed_ms(ctypes.byref(ms), self.ptr, end.ptr))
        return ms.value

    def __del__(self):
        try:
            if self.ptr:
                _lib.ud_event_destroy(self.ptr)
        except Exception:
            pass


# ---------------------------------------------------------------- encoder

@dataclasses.dataclass
class EncoderConfig:
    """FastConformerConfig.nemotron (FastConformer.swift:5-38) plus streaming geometry.

    dtype: "f32"; "bf16" (bf16-valued linear weights held as IEEE half; half activations, K/V
    caches and tables; fp32 accumulation); or "f16" (the same, with the weights rounded straight
    to half, the reference's f16 checkpoint, Core/Convert.swift:76-112).  16-bit stores saturate
    at +-65504."""
    layers: int = 24
    d_model: int = 1024
    heads: int = 8
    ff_dim: int = 4096
    conv_kernel: int = 9
    left_context: int = 70
    max_chunk: int = 2
    max_streams: int = 64
    dtype: str = "bf16"

    def _c(self):
        return _Config(self.layers, self.d_model, self.heads, self.ff_dim, self.conv_kernel, self.left_context,
                       self.max_chunk, self.max_streams, _DTYPES[self.dtype])


LAYER_WEIGHT_SUFFIXES = (
    "norm_feed_forward1.weight", "norm_feed_forward1.bias", "feed_forward1.linear1.weight",
    "feed_forward1.linear2.weight", "norm_self_att.weight", "norm_self_att.bias", "self_attn.linear_q.weight",
    "self_attn.linear_k.weight", "self_attn.linear_v.weight", "self_attn.linear_out.weight",
    "self_attn.linear_pos.weight", "self_attn.pos_bias_u", "self_attn.pos_bias_v", "norm_conv.weight",
    "norm_conv.bias", "conv.pointwise_conv1.weight", "conv.depthwise_conv.weight", "conv.batch_norm.weight",
    "conv.batch_norm.bias", "conv.pointwise_conv2.weight", "norm_feed_forward2.weight", "norm_feed_forward2.bias",
    "feed_forward2.linear1.weight", "feed_forward2.linear2.weight", "norm_out.weight", "norm_out.bias",
)


class Stream:
    """One audio stream's encoder state (StreamState, FastConformer.swift:406-429)."""

    def __init__(self, encoder):
        self.encoder = encoder
        p = _vp()
        _check(lib().ud_stream_create(encoder.handle, ctypes.byref(p)))
        self.handle = p.value

    @property
    def cache_len(self):
        c, s = _i32(0), _i32(0)
        _check(_lib.ud_stream_info(self.handle, ctypes.byref(c), ctypes.byref(s)))
        return c.value

    @property
    def step(self):
        c, s = _i32(0), _i32(0)
        _check(_lib.ud_stream_info(self.handle, ctypes.byref(c), ctypes.byref(s)))
        return s.value

    def reset(self):
        _check(_lib.ud_stream_reset(self.handle))

    def export_cache(self, layer):
        """(k [L, D], v [L, D], conv [K-1, D], cache_len) in logical order, fp32."""
        cfg = self.encoder.config
        L, D, KC = cfg.left_context, cfg.d_model, cfg.conv_kernel - 1
        k = np.empty((L, D), np.float32)
        v = np.empty((L, D), np.float32)
        c = np.empty((KC, D), np.float32)
        n = _i32(0)
        fp = ctypes.POINTER(ctypes.c_float)
        _check(_lib.ud_stream_export_cache(self.handle, layer, k.ctypes.data_as(fp), v.ctypes.data_as(fp),
                                           c.ctypes.data_as(fp), ctypes.byref(n)))
        return k, v, c, n.value

    def import_cache(self, layer, k, v, conv, cache_len):
        fp = ctypes.POINTER(ctypes.c_float)
        k, v, conv = (np.ascontiguousarray(a, np.float32) for a in (k, v, conv))
        _check(_lib.ud_stream_import_cache(self.handle, layer, k.ctypes.data_as(fp), v.ctypes.data_as(fp),
                                           conv.ctypes.data_as(fp), int(cache_len)))

    def close(self):
        if self.handle:
            _lib.ud_stream_destroy(self.handle)
            self.handle = None


def _handles(streams):
    arr = (_vp * len(streams))(*[s.handle for s in streams])
    return arr


def _valid_arr(valid, n, T):
    if valid is None:
        valid = [T] * n
    return np.ascontiguousarray(valid, np.int32)


class Encoder:
    """Device weights, position tables, workspace and stream pool of one encoder."""

    def __init__(self, config=None):
        self.config = config or EncoderConfig()
        p = _vp()
        c = self.config._c()
        _check(lib().ud_encoder_create(ctypes.byref(c), ctypes.byref(p)))
        self.handle = p.value

    def set_weight(self, name, array):
        a = np.ascontiguousarray(array, np.float32)
        _check(_lib.ud_encoder_set_weight(self.handle, name.encode(), a.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                          a.size))

    def set_layer_weights(self, layer, weights):
        """weights: dict NeMo-suffix -> array (as synthetic_layer_weights returns)."""
        for suffix, a in weights.items():
            self.set_weight("encoder.layers.%d.%s" % (layer, suffix), a)

    def load_safetensors(self, st):
        """Sets every encoder tensor of a SafeTensors file (NeMo or HF names; layers beyond this
        encoder's depth skipped); returns the count.  Call finalize() afterwards."""
        n = _i32(0)
        _check(_lib.ud_encoder_load_safetensors(self.handle, st.handle, ctypes.byref(n)))
        return n.value

    def set_subsampling_weights(self, weights):
        """weights: dict of the 12 encoder.pre_encode.* tensors (as synthetic_subsampling_weights
        returns), checkpoint layout."""
        for name, a in weights.items():
            self.set_weight(name, a)

    def finalize(self):
        _check(_lib.ud_encoder_finalize(self.handle))

    def subsample(self, n, mel, out, valid_mel=None, drop=0, mel_rows=None, hip_stream=None):
        """encodeSubsampling + drop (ud_encoder_subsample): mel a DeviceBuffer of fp32
        [n, mel_rows, 128]; out a DeviceBuffer of fp32 [n, T, d_model].  Returns (T, valid_T)."""
        mel_rows = mel_rows or mel.nbytes // (4 * n * MEL_BINS)
        vm = None if valid_mel is None else np.ascontiguousarray(valid_mel, np.int32)
        T = _i32(0)
        vt = np.zeros(n, np.int32)
        _check(_lib.ud_encoder_subsample(self.handle, n, mel_rows, mel.ptr,
                                         vm.ctypes.data_as(ctypes.POINTER(_i32)) if vm is not None else None,
                                         int(drop), out.ptr, ctypes.byref(T), vt.ctypes.data_as(ctypes.POINTER(_i32)),
                                         hip_stream.ptr if hip_stream else None))
        return T.value, vt

    def new_stream(self):
        return Stream(self)

    def encode_stream_step(self, streams, x, out, valid=None, T=None, hip_stream=None):
        """One chunk step for `streams`: x/out are DeviceBuffers of fp32 [n, T, d_model]."""
        n = len(streams)
        T = T or x.nbytes // (4 * n * self.config.d_model)
        va = _valid_arr(valid, n, T)
        _check(_lib.ud_encoder_step(self.handle, _handles(streams), n, T, x.ptr,
                                    va.ctypes.data_as(ctypes.POINTER(_i32)), out.ptr,
                                    hip_stream.ptr if hip_stream else None))

    def layer_attention(self, streams, T, layer, qkv, att, valid=None, hip_stream=None):
        n = len(streams)
        va = _valid_arr(valid, n, T)
        _check(_lib.ud_layer_attention(self.handle, _handles(streams), n, T, layer, qkv.ptr,
                                       va.ctypes.data_as(ctypes.POINTER(_i32)), att.ptr,
                                       hip_stream.ptr if hip_stream else None))

    def time_layer_attention(self, streams, T, layer, qkv, att, iters, hip_stream=None):
        """Average duration (ms) of the fused attention kernel over `iters` back-to-back launches,
        from HIP events on hip_stream."""
        ms = ctypes.c_float(0)
        _check(_lib.ud_time_layer_attention(self.handle, _handles(streams), len(streams), T, layer, qkv.ptr, att.ptr,
                                            iters, hip_stream.ptr if hip_stream else None, ctypes.byref(ms)))
        return ms.value

    def time_ring_read_floor(self, streams, T, layer, qkv, att, iters, hip_stream=None):
        """Average duration (ms) of a kernel that performs only the attention kernel's loads (bf16,
        T <= 2): the memory floor of that access pattern."""
        ms = ctypes.c_float(0)
        _check(_lib.ud_time_ring_read_floor(self.handle, _handles(streams), len(streams), T, layer, qkv.ptr, att.ptr,
                                            iters, hip_stream.ptr if hip_stream else None, ctypes.byref(ms)))
        return ms.value

    PROJECTIONS = ("ff_linear1", "ff_linear2", "qkv", "linear_out", "pointwise_conv1", "pointwise_conv2")

    def time_projection(self, which, rows, iters, hip_stream=None):
        """(average ms per launch, flops per launch) of one of the step's projection GEMMs
        (PROJECTIONS index) launched as the step launches it for `rows` rows."""
        ms = ctypes.c_float(0)
        fl = ctypes.c_double(0)
        _check(_lib.ud_time_projection(self.handle, which, rows, iters, hip_stream.ptr if hip_stream else None,
                                       ctypes.byref(ms), ctypes.byref(fl)))
        return ms.value, fl.value

    @staticmethod
    def advance(streams, T):
        _check(_lib.ud_stream_advance(_handles(streams), len(streams), T))

    def close(self):
        if self.handle:
            _lib.ud_encoder_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def rel_pos_attention(q, k, v, pos_table, rel_offset, bias_u, bias_v, ranges, out, heads, Tq, Tk, head_dim,
                      n_rel, dtype="f32", hip_stream=None):
    """Step.relPosAttention (Ops.swift:80-90) on DeviceBuffers: q [Tq, H*dk], k/v [Tk, H*dk],
    pos_table [n_rel, H*dk] (dtype f32 or bf16), bias_u/bias_v fp32 [H, dk], ranges int32 [Tq, 2]."""
    _check(lib().ud_relpos_attention(_DTYPES[dtype], q.ptr, k.ptr, v.ptr, pos_table.ptr, bias_u.ptr, bias_v.ptr,
                                     ranges.ptr, out.ptr, Tq, Tk, heads, head_dim, rel_offset, n_rel,
                                     hip_stream.ptr if hip_stream else None))


MASK_CHUNKED_LIMITED, MASK_CHUNKED_LIMITED_RC = 0, 1


def chunked_limited_ranges(T, left, right, valid=None, chunk=None):
    """Key ranges int32 [B, T, 2] of the offline streaming masks (MaskSpec.ranges +
    forwardOffline's clip to the valid length, FastConformer.swift:324-357, 380-381).  chunk None:
    chunked_limited [left, right]; else chunked_limited_with_rc [left, chunk, right].  valid: None
    (one utterance, no clip), an int, or a sequence of B valid lengths.  Host computation only."""
    if valid is None:
        vals = None
        B = 1
    else:
        vals = np.atleast_1d(np.asarray(valid, np.int32))
        B = len(vals)
    out = np.empty((B, T, 2), np.int32)
    ip = ctypes.POINTER(_i32)
    kind = MASK_CHUNKED_LIMITED if chunk is None else MASK_CHUNKED_LIMITED_RC
    _check(load_library().ud_chunked_limited_ranges(
        kind, B, T, vals.ctypes.data_as(ip) if vals is not None else None, left, 0 if chunk is None else chunk, right,
        out.ctypes.data_as(ip)))
    return out


def rel_pos_attention_batched(q, k, v, pos_table, rel_offset, bias_u, bias_v, ranges, out, B, T, heads,
                              n_rel, head_dim=128, hip_stream=None):
    """Offline relPosAttention over B whole utterances (bf16): q/k/v/out [B, T, H*128], pos_table
    [n_rel, H*128], bias_u/bias_v fp32 [H, 128], ranges int32 [B, T, 2]."""
    _check(lib().ud_relpos_attention_batched(UD_BF16, q.ptr, k.ptr, v.ptr, pos_table.ptr, bias_u.ptr, bias_v.ptr,
                                             ranges.ptr, out.ptr, B, T, heads, head_dim, rel_offset, n_rel,
                                             hip_stream.ptr if hip_stream else None))


# ---------------------------------------------------------------- decoder attention (ud_decode.h)

def rope_inv_freq(head_dim, theta=1e6):
    """inv_freq_i = 1 / theta^(2i/d), evaluated in float64 and rounded to float32 as the reference
    builds it (Sources/DictatorEngine/Models/Voxtral.swift:176-179)."""
    i = np.arange(head_dim // 2, dtype=np.float64)
    return (1.0 / np.power(float(theta), 2.0 * i / head_dim)).astype(np.float32)


def gqa_workspace_bytes(n, q_heads, head_dim, max_keys):
    return int(lib().ud_gqa_workspace_bytes(n, q_heads, head_dim, max_keys))


def gqa_attention_paged(q, k_pages, v_pages, block_table, max_blocks, ranges, out, n, q_heads, kv_heads, head_dim,
                        max_keys, workspace, kv_dtype="bf16", block_size=16, hip_stream=None):
    """Step.attention (Ops.swift:136-169) for one query token per sequence over a paged K/V cache:
    q/out fp32 [n, q_heads*head_dim]; k_pages/v_pages [num_blocks, kv_heads, block_size, head_dim]
    (kv_dtype bf16 or f16); block_table int32 [n, max_blocks]; ranges int32 [n, 2]."""
    _check(lib().ud_gqa_attention_paged(_DTYPES[kv_dtype], q.ptr, k_pages.ptr, v_pages.ptr, block_table.ptr,
                                        max_blocks, ranges.ptr, out.ptr, n, q_heads, kv_heads, head_dim, block_size,
                                        max_keys, workspace.ptr, workspace.nbytes,
                                        hip_stream.ptr if hip_stream else None))


def gqa_attention_paged_mq(q, k_pages, v_pages, block_table, max_blocks, ranges, out, n, n_queries, q_heads, kv_heads,
                           head_dim, max_keys, workspace, kv_dtype="bf16", block_size=16, hip_stream=None):
    """Step.attention with n_queries (1 .. 8) positions per sequence (Ops.swift:141-162,
    attention_mq_split): q/out fp32 [n, n_queries, q_heads*head_dim], ranges int32 [n, n_queries, 2],
    each K/V page read once for all of a sequence's queries; workspace of
    gqa_workspace_bytes(n * n_queries, q_heads, head_dim, max_keys) bytes."""
    _check(lib().ud_gqa_attention_paged_mq(_DTYPES[kv_dtype], q.ptr, k_pages.ptr, v_pages.ptr, block_table.ptr,
                                           max_blocks, ranges.ptr, out.ptr, n, n_queries, q_heads, kv_heads, head_dim,
                                           block_size, max_keys, workspace.ptr, workspace.nbytes,
                                           hip_stream.ptr if hip_stream else None))


# Static scratch of ud_gqa_attention_paged_noalloc (UD_GQA_NOALLOC_SCRATCH_BYTES in ud_decode.h).
GQA_NOALLOC_SCRATCH_BYTES = 40 << 20


def gqa_attention_paged_noalloc(q, k_pages, v_pages, block_table, max_blocks, ranges, out, n, q_heads, kv_heads,
                                head_dim, max_keys, kv_dtype="bf16", block_size=16, hip_stream=None):
    """gqa_attention_paged without a workspace: the split partials live in the library's static
    per-device scratch, so the call allocates nothing (calls overlapping on one device race)."""
    _check(lib().ud_gqa_attention_paged_noalloc(_DTYPES[kv_dtype], q.ptr, k_pages.ptr, v_pages.ptr,
                                                block_table.ptr, max_blocks, ranges.ptr, out.ptr, n, q_heads,
                                                kv_heads, head_dim, block_size, max_keys,
                                                hip_stream.ptr if hip_stream else None))


def rope_rotate_half(x, rows, heads, head_dim, ld, inv_freq, positions=None, pos0=0, dtype="f32", hip_stream=None):
    """Step.rope / rope_rotate_half (30_voxtral.metal:20-36) in place on x [rows, ld]; positions is
    an int32 DeviceBuffer [rows] or None for pos0 + row."""
    _check(lib().ud_rope_rotate_half(_DTYPES[dtype], x.ptr, rows, heads, head_dim, ld,
                                     positions.ptr if positions is not None else None, pos0, inv_freq.ptr,
                                     hip_stream.ptr if hip_stream else None))


def paged_kv_append(k_new, v_new, k_pages, v_pages, block_table, max_blocks, positions, n, kv_heads, head_dim,
                    kv_dtype="bf16", block_size=16, hip_stream=None):
    """Writes row i of k_new / v_new [n, kv_heads*head_dim] at logical position positions[i] of
    sequence i in the paged cache."""
    _check(lib().ud_paged_kv_append(_DTYPES[kv_dtype], k_new.ptr, v_new.ptr, k_pages.ptr, v_pages.ptr, block_table.ptr,
                                    max_blocks, positions.ptr, n, kv_heads, head_dim, block_size,
                                    hip_stream.ptr if hip_stream else None))


# ---------------------------------------------------------------- synthetic weights

def synthetic_layer_weights(cfg, seed, layer, ln_jitter=0.1):
    """Random-init weights of one Nemotron FastConformer layer in the checkpoint layout.

    Linear and conv weights are Xavier-uniform; pos_bias_u/v ~ N(0, 0.02^2); LayerNorm gamma =
    1 + ln_jitter*U(-1,1), beta = ln_jitter*U(-1,1) (ln_jitter=0 gives gamma=1, beta=0)."""
    rng = np.random.default_rng([int(seed), int(layer)])
    D, ff, K, H = cfg.d_model, cfg.ff_dim, cfg.conv_kernel, cfg.heads

    def xavier(shape, fan_in, fan_out):
        b = np.float32(np.sqrt(6.0 / (fan_in + fan_out)))
        return ((rng.random(shape, dtype=np.float32) * 2 - 1) * b).astype(np.float32)

    def ln():
        g = (1 + ln_jitter * (rng.random(D, dtype=np.float32) * 2 - 1)).astype(np.float32)
        b = (ln_jitter * (rng.random(D, dtype=np.float32) * 2 - 1)).astype(np.float32)
        return g, b

    w = {}
    for name in ("norm_feed_forward1", "norm_self_att", "norm_conv", "conv.batch_norm", "norm_feed_forward2",
                 "norm_out"):
        g, b = ln()
        w[name + ".weight"], w[name + ".bias"] = g, b
    w["feed_forward1.linear1.weight"] = xavier((ff, D), D, ff)
    w["feed_forward1.linear2.weight"] = xavier((D, ff), ff, D)
    for n in ("q", "k", "v", "out", "pos"):
        w["self_attn.linear_%s.weight" % n] = xavier((D, D), D, D)
    w["self_attn.pos_bias_u"] = (rng.standard_normal((H, D // H), dtype=np.float32) * 0.02).astype(np.float32)
    w["self_attn.pos_bias_v"] = (rng.standard_normal((H, D // H), dtype=np.float32) * 0.02).astype(np.float32)
    w["conv.pointwise_conv1.weight"] = xavier((2 * D, D), D, 2 * D)
    w["conv.depthwise_conv.weight"] = xavier((D, K), K, K)
    w["conv.pointwise_conv2.weight"] = xavier((D, D), D, D)
    w["feed_forward2.linear1.weight"] = xavier((ff, D), D, ff)
    w["feed_forward2.linear2.weight"] = xavier((D, ff), ff, D)
    return w


ST_DTYPES = {0: "F32", 1: "BF16", 2: "F16", 3: "other"}


class SafeTensors:
    """A memory-mapped safetensors file (include/ud_safetensors.h), mirroring SafeTensorsReader
    (Sources/DictatorCore/Weights/WeightSource.swift): names, info, tensors widened to fp32."""

    def __init__(self, path):
        p = _vp()
        _check(load_library().ud_safetensors_open(os.fsencode(path), ctypes.byref(p)))
        self.handle = p.value

    def names(self):
        return [_lib.ud_safetensors_name(self.handle, i).decode() for i in range(_lib.ud_safetensors_count(self.handle))]

    def info(self, name):
        dt = _i32(0)
        nd = _i32(0)
        shape = (ctypes.c_int64 * 8)()
        _check(_lib.ud_safetensors_info(self.handle, name.encode(), ctypes.byref(dt), shape, ctypes.byref(nd)))
        return ST_DTYPES[dt.value], tuple(shape[i] for i in range(nd.value))

    def floats(self, name):
        _, shape = self.info(name)
        out = np.empty(shape, np.float32)
        _check(_lib.ud_safetensors_read_f32(self.handle, name.encode(),
                                            out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), out.size))
        return out

    def close(self):
        if self.handle:
            _lib.ud_safetensors_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def nemo_name(name):
    """The NeMo state_dict name of a tensor name (HF model.safetensors aliases mapped)."""
    buf = ctypes.create_string_buffer(512)
    _check(load_library().ud_nemo_name(name.encode(), buf, 512))
    return buf.value.decode()


class Rnnt:
    """RNN-T joint + greedy decoder for a pool of stream slots (include/ud_rnnt.h), mirroring
    RNNTDecoder (Sources/DictatorCore/Decoding/RNNT.swift): set_weights, project (joint.enc),
    greedy over projected frames with per-slot state carried across calls."""

    def __init__(self, max_streams, hidden=640, vocab=1025, layers=2, enc_dim=1024, max_symbols=10):
        p = _vp()
        _check(lib().ud_rnnt_create(hidden, vocab, layers, enc_dim, max_streams, max_symbols, ctypes.byref(p)))
        self.handle = p.value
        self.H, self.V, self.L, self.E, self.S = hidden, vocab, layers, enc_dim, max_streams

    def set_weights(self, weights):
        """weights: dict of checkpoint tensors (as synthetic_rnnt_weights returns)."""
        for name, a in weights.items():
            a = np.ascontiguousarray(a, np.float32)
            _check(_lib.ud_rnnt_set_weight(self.handle, name.encode(),
                                           a.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), a.size))

    def reset(self, slot):
        _check(_lib.ud_rnnt_reset(self.handle, int(slot)))

    def load_safetensors(self, st):
        """Sets every decoder.prediction.* / joint.* tensor of a SafeTensors file; returns the count."""
        n = _i32(0)
        _check(_lib.ud_rnnt_load_safetensors(self.handle, st.handle, ctypes.byref(n)))
        return n.value

    def project(self, rows, enc, out, hip_stream=None):
        """out [rows, hidden] = joint.enc(enc [rows, enc_dim]); DeviceBuffers of fp32."""
        _check(_lib.ud_rnnt_project(self.handle, int(rows), enc.ptr, out.ptr, hip_stream.ptr if hip_stream else None))

    def nemotron_step(self, enc, streams, mel, mel_rows, valid_rows, keep_all, drop_extra, out_frames, proj,
                      proj_rows, hip_stream=None):
        """NemotronEncoder.step for len(streams) streams (include/ud_streamer.h ud_nemotron_step):
        mel a DeviceBuffer of fp32 [n, mel_rows, 128], proj a DeviceBuffer of fp32
        [n, proj_rows, hidden]; returns the kept frames per stream."""
        n = len(streams)
        vr = np.ascontiguousarray(valid_rows, np.int32)
        ka = np.ascontiguousarray([1 if k else 0 for k in keep_all], np.int32)
        fr = np.zeros(n, np.int32)
        P = ctypes.POINTER(_i32)
        _check(_lib.ud_nemotron_step(enc.handle, self.handle, _handles(streams), n, int(mel_rows), mel.ptr,
                                     vr.ctypes.data_as(P), ka.ctypes.data_as(P), int(drop_extra), int(out_frames),
                                     proj.ptr, int(proj_rows), fr.ctypes.data_as(P),
                                     hip_stream.ptr if hip_stream else None))
        return [int(x) for x in fr]

    def greedy(self, slots, proj, rows_per_stream, frames, cap=4096, hip_stream=None):
        """Greedy decode: proj a DeviceBuffer of fp32 [len(slots) * rows_per_stream, hidden];
        returns a list of token lists (and the full emitted counts)."""
        n = len(slots)
        sl = np.ascontiguousarray(slots, np.int32)
        fr = np.ascontiguousarray(frames, np.int32)
        toks = np.zeros((n, max(cap, 1)), np.int32)
        cnt = np.zeros(n, np.int32)
        P = ctypes.POINTER(_i32)
        _check(_lib.ud_rnnt_greedy(self.handle, n, sl.ctypes.data_as(P), proj.ptr, int(rows_per_stream),
                                   fr.ctypes.data_as(P), toks.ctypes.data_as(P), int(cap), cnt.ctypes.data_as(P),
                                   hip_stream.ptr if hip_stream else None))
        return [list(map(int, toks[b, :min(cnt[b], cap)])) for b in range(n)], cnt

    def close(self):
        if self.handle:
            _lib.ud_rnnt_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


SUB_CHANNELS, MEL_BINS = 256, 128


def synthetic_subsampling_weights(seed, D=1024, C=SUB_CHANNELS, mel_bins=MEL_BINS):
    """Random-init weights of the causal dw_striding subsampling (encoder.pre_encode.*) in the
    checkpoint layout: conv weights Xavier-uniform over torch's fan_in/fan_out
    (in_channels/groups * k * k, out_channels/groups * k * k), biases U(-1/sqrt(fan_in), +), the
    output Linear [D, C*F3] with columns in NeMo's (channel, freq) order."""
    rng = np.random.default_rng([int(seed), 1 << 20])
    F3 = mel_bins
    for _ in range(3):
        F3 = F3 // 2 + 1

    def xavier(shape, fan_in, fan_out):
        b = np.float32(np.sqrt(6.0 / (fan_in + fan_out)))
        return ((rng.random(shape, dtype=np.float32) * 2 - 1) * b).astype(np.float32)

    def bias(n, fan_in):
        return ((rng.random(n, dtype=np.float32) * 2 - 1) / np.float32(np.sqrt(fan_in))).astype(np.float32)

    p = "encoder.pre_encode."
    w = {}
    w[p + "conv.0.weight"], w[p + "conv.0.bias"] = xavier((C, 1, 3, 3), 9, 9 * C), bias(C, 9)
    for i in (2, 5):
        w[p + "conv.%d.weight" % i], w[p + "conv.%d.bias" % i] = xavier((C, 1, 3, 3), 9, 9), bias(C, 9)
    for i in (3, 6):
        w[p + "conv.%d.weight" % i], w[p + "conv.%d.bias" % i] = xavier((C, C, 1, 1), C, C), bias(C, C)
    w[p + "out.weight"], w[p + "out.bias"] = xavier((D, C * F3), C * F3, D), bias(D, C * F3)
    return w


def synthetic_rnnt_weights(seed, H=640, V=1025, L=2, enc_dim=1024, blank_bias=0.0):
    """Random-init RNN-T prediction and joint networks in the checkpoint layout (torch's LSTM and
    Linear init: U(-1/sqrt(H), 1/sqrt(H)) for the LSTM, U(-1/sqrt(fan_in), +) for the Linears,
    embedding N(0, 1) with the blank row zero), joint.enc included.  blank_bias is added to the
    blank logit's bias, which sets how often the greedy loop emits."""
    rng = np.random.default_rng([int(seed), 1 << 21])

    def u(shape, bound):
        return ((rng.random(shape, dtype=np.float32) * 2 - 1) * np.float32(bound)).astype(np.float32)

    w = {}
    emb = rng.standard_normal((V, H), dtype=np.float32)
    emb[V - 1] = 0.0
    w["decoder.prediction.embed.weight"] = emb
    k = 1.0 / np.sqrt(H)
    for l in range(L):
        p = "decoder.prediction.dec_rnn.lstm."
        w[p + "weight_ih_l%d" % l] = u((4 * H, H), k)
        w[p + "weight_hh_l%d" % l] = u((4 * H, H), k)
        w[p + "bias_ih_l%d" % l] = u(4 * H, k)
        w[p + "bias_hh_l%d" % l] = u(4 * H, k)
    w["joint.pred.weight"], w["joint.pred.bias"] = u((H, H), k), u(H, k)
    w["joint.enc.weight"], w["joint.enc.bias"] = u((H, enc_dim), 1 / np.sqrt(enc_dim)), u(H, 1 / np.sqrt(enc_dim))
    w["joint.joint_net.2.weight"], w["joint.joint_net.2.bias"] = u((V, H), k), u(V, k)
    w["joint.joint_net.2.bias"][V - 1] += np.float32(blank_bias)
    return w


def round_f16(a):
    """IEEE-half rounding (round to nearest even) of float32 values, returned as float32: the
    storage format of a 16-bit (bf16 or f16) encoder's activations, K/V caches and position tables,
    and the weight rounding of an f16 encoder."""
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


def f16_bits(a):
    """uint16 bit patterns of IEEE half(a) (round to nearest even)."""
    return np.ascontiguousarray(np.asarray(a, np.float32).astype(np.float16)).view(np.uint16)


def from_f16_bits(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


def round_bf16(a):
    """Round-to-nearest-even to bfloat16 and back to fp32 (the upload rule of bf16 encoders,
    Sources/DictatorEngine/Core/Tensor.swift:116-122)."""
    a = np.ascontiguousarray(a, np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32) << 16
    r = np.where(np.isnan(a), np.uint32(0x7FC00000), r.astype(np.uint32))
    return r.astype(np.uint32).view(np.float32).reshape(a.shape)


# ---------------------------------------------------------------- mel frontend and streaming


class MelFrontend:
    """NeMo log-mel frontend on the GPU (include/ud_mel.h), mirroring NemoMelFrontend
    (Sources/DictatorCore/Audio/NemoMel.swift:11-108): fb [n_mels, 257] and window [400] are the
    checkpoint's preprocessor.featurizer buffers."""

    HOP = 160

    def __init__(self, fb=None, window=None, handle=None):
        if handle is None:
            fb = np.ascontiguousarray(fb, np.float32).reshape(-1, 257)
            window = np.ascontiguousarray(window, np.float32).reshape(400)
            p = _vp()
            F = ctypes.POINTER(ctypes.c_float)
            _check(lib().ud_mel_create(fb.ctypes.data_as(F), fb.shape[0], window.ctypes.data_as(F), ctypes.byref(p)))
            handle = p.value
        self.handle = handle
        self.n_mels = int(_lib.ud_mel_bins(self.handle))

    @classmethod
    def from_safetensors(cls, st):
        p = _vp()
        _check(lib().ud_mel_load_safetensors(st.handle, ctypes.byref(p)))
        return cls(handle=p.value)

    @staticmethod
    def valid_frames(samples):
        return samples // MelFrontend.HOP

    def features_device(self, n, audio, stride, n_samples, out, out_rows, hip_stream=None):
        """ud_mel_features on DeviceBuffers: audio fp32 [n, stride]; out fp32 [n, out_rows, n_mels].
        Returns the frame counts."""
        ns = np.ascontiguousarray(n_samples, np.int64)
        fr = np.zeros(n, np.int32)
        _check(_lib.ud_mel_features(self.handle, n, audio.ptr, int(stride), ns.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
                                    out.ptr, int(out_rows), fr.ctypes.data_as(ctypes.POINTER(_i32)),
                                    hip_stream.ptr if hip_stream else None))
        return fr

    def features(self, clips):
        """Full-utterance features of a list of 1-D fp32 clips: a list of [n // 160 + 1, n_mels]."""
        clips = [np.ascontiguousarray(c, np.float32).ravel() for c in clips]
        n = len(clips)
        stride = max(1, max(c.size for c in clips))
        a = np.zeros((n, stride), np.float32)
        for b, c in enumerate(clips):
            a[b, :c.size] = c
        rows = stride // self.HOP + 1
        ab = DeviceBuffer.from_numpy(a)
        ob = DeviceBuffer(n * rows * self.n_mels * 4)
        fr = self.features_device(n, ab, stride, [c.size for c in clips], ob, rows)
        synchronize()
        out = ob.download((n, rows, self.n_mels))
        return [out[b, :fr[b]].copy() for b in range(n)]

    def close(self):
        if self.handle:
            _lib.ud_mel_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _sized_bytes(call):
    """Runs call(buf, cap, len_ptr) once to size the output and once to fill it."""
    n = ctypes.c_int64(0)
    _check(call(None, 0, ctypes.byref(n)))
    buf = ctypes.create_string_buffer(max(1, n.value))
    _check(call(buf, n.value, ctypes.byref(n)))
    return buf.raw[:n.value]


class Tokenizer:
    """SentencePieceDecoder (Sources/DictatorCore/Decoding/SentencePiece.swift:5-31) through the C ABI
    (include/ud_tokenizer.h): host code, no device needed.  Build from a tokenizer.vocab path, or
    from the file's bytes with Tokenizer.from_bytes.  decode() returns UTF-8 bytes."""

    def __init__(self, vocab_path=None, _handle=None):
        load_library()
        if _handle is not None:
            self.handle = _handle
            return
        h = _vp()
        _check(_lib.ud_tokenizer_load(os.fsencode(vocab_path), ctypes.byref(h)))
        self.handle = h

    @classmethod
    def from_bytes(cls, data):
        load_library()
        data = bytes(data)
        h = _vp()
        _check(_lib.ud_tokenizer_parse(data, len(data), ctypes.byref(h)))
        return cls(_handle=h)

    def __len__(self):
        n = _i32(0)
        _check(_lib.ud_tokenizer_size(self.handle, ctypes.byref(n)))
        return n.value

    def piece(self, i):
        return _sized_bytes(lambda buf, cap, n: _lib.ud_tokenizer_piece(self.handle, int(i), buf, cap, n))

    def decode(self, ids):
        a = np.ascontiguousarray(np.asarray(ids, np.int32).reshape(-1))
        P = ctypes.POINTER(_i32)
        ptr = a.ctypes.data_as(P) if a.size else None
        return _sized_bytes(lambda buf, cap, n: _lib.ud_tokenizer_decode(self.handle, ptr, a.size, buf, cap, n))

    def close(self):
        if getattr(self, "handle", None):
            _lib.ud_tokenizer_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Streamer:
    """Cache-aware streaming transcription of many streams at once (include/ud_streamer.h), mirroring
    NemotronStreamer (Sources/DictatorCore/Nemotron/NemotronStreamer.swift): open() gives a stream
    id; push / flush / run_buffered / tokens act per stream id, and every stream with a complete
    chunk joins one batched step."""

    def __init__(self, encoder, rnnt, mel=None, lookahead=1, max_streams=None):
        max_streams = max_streams or encoder.config.max_streams
        p = _vp()
        _check(lib().ud_streamer_create(encoder.handle, rnnt.handle, mel.handle if mel is not None else None,
                                        int(lookahead), int(max_streams), ctypes.byref(p)))
        self.handle = p.value
        self.lookahead = lookahead
        self._end_padding, self._record = True, False
        self._keep = (encoder, rnnt, mel)

    def _opts(self):
        _check(_lib.ud_streamer_set_options(self.handle, int(self._end_padding), int(self._record)))

    @property
    def end_padding(self):
        return self._end_padding

    @end_padding.setter
    def end_padding(self, on):
        self._end_padding = bool(on)
        self._opts()

    @property
    def record(self):
        return self._record

    @record.setter
    def record(self, on):
        self._record = bool(on)
        self._opts()

    def open(self):
        i = _i32(0)
        _check(_lib.ud_streamer_open(self.handle, ctypes.byref(i)))
        return i.value

    def close_stream(self, sid):
        _check(_lib.ud_streamer_close(self.handle, int(sid)))

    class Pushed:
        """The arguments of one ud_streamer_push (ids, sample pointers, counts), packed once: a
        caller that pushes many streams from Python can pack ahead of its time-critical loop."""

        def __init__(self, chunks):
            self.ids = np.fromiter(chunks.keys(), np.int32, len(chunks))
            arrs = []
            for a in chunks.values():
                if not (isinstance(a, np.ndarray) and a.dtype == np.float32 and a.ndim == 1 and a.flags.c_contiguous):
                    a = np.ascontiguousarray(a, np.float32).ravel()
                arrs.append(a)
            self.arrs = arrs                        # keeps the samples alive
            self.ptrs = np.fromiter((a.__array_interface__["data"][0] for a in arrs), np.uintp, len(arrs))
            self.counts = np.fromiter((a.size for a in arrs), np.int64, len(arrs))
            self.n = len(arrs)
            self.args = (self.ids.ctypes.data, self.ptrs.ctypes.data, self.counts.ctypes.data)

    def push(self, chunks):
        """chunks: {stream id: fp32 samples}, or a Streamer.Pushed of them.  Runs every chunk that
        became complete."""
        pk = chunks if isinstance(chunks, Streamer.Pushed) else Streamer.Pushed(chunks)
        _check(_lib.ud_streamer_push(self.handle, pk.n, *pk.args))

    def flush(self, ids):
        ids = np.ascontiguousarray(ids, np.int32)
        _check(_lib.ud_streamer_flush(self.handle, ids.size, ids.ctypes.data_as(ctypes.POINTER(_i32))))

    def run_buffered(self, runs):
        """runs: {stream id: (mel [frames, n_mels], frames, valid_frames)} for fresh streams."""
        ids = np.array(list(runs.keys()), np.int32)
        mels = [np.ascontiguousarray(r[0], np.float32) for r in runs.values()]
        F = ctypes.POINTER(ctypes.c_float)
        ptrs = (F * max(1, len(mels)))(*[m.ctypes.data_as(F) for m in mels])
        fr = np.array([r[1] for r in runs.values()], np.int32)
        vf = np.array([r[2] for r in runs.values()], np.int32)
        P = ctypes.POINTER(_i32)
        _check(_lib.ud_streamer_run_buffered(self.handle, ids.size, ids.ctypes.data_as(P), ptrs, fr.ctypes.data_as(P),
                                             vf.ctypes.data_as(P)))

    def tokens(self, sid):
        n = _i32(0)
        _check(_lib.ud_streamer_tokens(self.handle, int(sid), None, 0, ctypes.byref(n)))
        out = np.zeros(max(1, n.value), np.int32)
        _check(_lib.ud_streamer_tokens(self.handle, int(sid), out.ctypes.data_as(ctypes.POINTER(_i32)), n.value,
                                       ctypes.byref(n)))
        return [int(t) for t in out[:n.value]]

    def text(self, sid, tokenizer):
        """NemotronStreamer.text: the stream's tokens so far decoded by `tokenizer` (a Tokenizer), as
        UTF-8 bytes."""
        return _sized_bytes(lambda buf, cap, n: _lib.ud_streamer_text(self.handle, int(sid), tokenizer.handle, buf, cap, n))

    def recorded(self, sid, which):
        """Recorded kept rows (record = True): which 'enc' [rows, d_model] or 'proj' [rows, hidden]."""
        w = 0 if which == "enc" else 1
        r = ctypes.c_int64(0)
        _check(_lib.ud_streamer_recorded(self.handle, int(sid), w, None, 0, ctypes.byref(r)))
        width = self._keep[0].config.d_model if w == 0 else self._keep[1].H
        out = np.zeros((r.value, width), np.float32)
        _check(_lib.ud_streamer_recorded(self.handle, int(sid), w, out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                         r.value, ctypes.byref(r)))
        return out

    def emissions(self, sid):
        """NemotronStreamer's emissions of a live stream: (token, samples_seen, compute_seconds) per
        emitted token, in order."""
        n = _i32(0)
        _check(_lib.ud_streamer_emissions(self.handle, int(sid), None, None, None, 0, ctypes.byref(n)))
        k = max(1, n.value)
        tok, seen, secs = np.zeros(k, np.int32), np.zeros(k, np.int64), np.zeros(k, np.float64)
        _check(_lib.ud_streamer_emissions(self.handle, int(sid), tok.ctypes.data_as(ctypes.POINTER(_i32)),
                                          seen.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
                                          secs.ctypes.data_as(ctypes.POINTER(ctypes.c_double)), n.value, ctypes.byref(n)))
        return [(int(tok[e]), int(seen[e]), float(secs[e])) for e in range(n.value)]

    def step_times(self, sid):
        """NemotronStreamer.wallTimes of a stream: wall seconds of each of its chunks' batched steps."""
        n = _i32(0)
        _check(_lib.ud_streamer_step_times(self.handle, int(sid), None, 0, ctypes.byref(n)))
        out = np.zeros(max(1, n.value), np.float64)
        _check(_lib.ud_streamer_step_times(self.handle, int(sid), out.ctypes.data_as(ctypes.POINTER(ctypes.c_double)),
                                           n.value, ctypes.byref(n)))
        return [float(x) for x in out[:n.value]]

    def stats(self):
        b, c = ctypes.c_int64(0), ctypes.c_int64(0)
        _check(_lib.ud_streamer_stats(self.handle, ctypes.byref(b), ctypes.byref(c)))
        return b.value, c.value

    def close(self):
        if self.handle:
            _lib.ud_streamer_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
