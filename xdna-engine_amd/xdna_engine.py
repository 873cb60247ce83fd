"""Python host mirror of the xdna-engine decode backend, over libxdna_engine.so.

The classes follow the reference's host interface for this path so tests and
callers read like the reference's own:

  Device      rust/npu-xrt Device (open/close) over the C ABI device layer
  Buf         rust/npu-xrt Bo (alloc/write/read)
  CtxDecode   rust/npu-asr/src/ctx_decode.rs:142-694 CtxDecode
              (register_weight / gemv / register_fused / fused_norm_gemv /
               attn / dispatches), plus the int8-activation and W8A8 forms
  Norm        ctx_decode.rs:74-79 (Rms / Ln) + Gemma's (1 + w) RMSNorm
  Decoder     the decode-backend contract (reset / precompute_cross /
              step / generate) of whisper_decoder.rs and opt125m_decode.rs
  presets     OPT_125M, WHISPER_SMALL, GEMMA3_1B (npu-gemma/src/config.rs)

Errors raise XdnaError carrying xe_last_error().  There is no CPU fallback:
if the library is missing, loading raises.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libxdna_engine.so")

XE_F32, XE_BF16, XE_I8, XE_BFP16, XE_I32, XE_I4 = 0, 1, 2, 3, 4, 5
XE_EPI_NONE, XE_EPI_BIAS, XE_EPI_SILU_BIAS = 0, 1, 2
XE_Q8_LIN, XE_Q8_ELF = 0, 1
XE_NORM_NONE, XE_NORM_LN, XE_NORM_RMS, XE_NORM_RMS1P = 0, 1, 2, 3
XE_LAYOUT_MK, XE_LAYOUT_KN = 0, 1
XE_OPT, XE_WHISPER, XE_GEMMA3 = 0, 1, 2
EXECUTORS = {0: "graph", 2: "eager", 3: "ll"}

EXPORTS = [
    "xe_last_error", "xe_abi_version", "xe_device_count", "xe_device_open", "xe_device_close",
    "xe_device_synchronize", "xe_device_name", "xe_buf_alloc", "xe_buf_free", "xe_buf_write",
    "xe_buf_read", "xe_buf_device_ptr", "xe_buf_size", "xe_buf_fill_synthetic", "xe_buf_copy", "xe_register_weight_view", "xe_probe_gemv",
    "xe_probe_attn", "xe_ctx_create",
    "xe_ctx_destroy",
    "xe_ctx_dispatches", "xe_ctx_reset_dispatches", "xe_register_weight",
    "xe_register_weight_q8", "xe_register_weight_q4", "xe_register_weight_q4_kn", "xe_register_weight_q8_rule",
    "xe_register_weight_bfp16", "xe_register_weight_bf16",
    "xe_register_fused", "xe_weight_set_norm", "xe_weight_free", "xe_weight_shape", "xe_gemv",
    "xe_fused_norm_gemv", "xe_gemv_dev", "xe_gemv_i8act", "xe_gemv_i8act_dev", "xe_w8a8_linear",
    "xe_w8a8_linear_dev",
    "xe_attn_decode", "xe_attn_decode_dev", "xe_attn_decode_dev_static", "xe_ctx_synchronize", "xe_decoder_create",
    "xe_decoder_destroy", "xe_decoder_init_synthetic", "xe_decoder_set_tensor",
    "xe_decoder_get_tensor_q8", "xe_decoder_reset", "xe_decoder_prime_kv", "xe_decoder_set_cross",
    "xe_decoder_set_cross_int8",
    "xe_decoder_step",
    "xe_decoder_generate", "xe_decoder_last_step_us", "xe_decoder_weight_bytes", "xe_decoder_set_stop",
    "xe_decoder_generate_until",
    "xe_decoder_feed", "xe_decoder_decode", "xe_decoder_profile_step", "xe_decoder_executor",
    "xe_model_tensor_shape", "xe_decoder_config", "xe_decoder_load_safetensors", "xe_safetensors_plan",
    "xe_ctx_record", "xe_run_query", "xe_run_wait", "xe_run_free", "xe_resident_open", "xe_resident_close",
    "xe_resident_write", "xe_resident_dispatch", "xe_resident_dispatch_start", "xe_resident_read",
]


class XdnaError(RuntimeError):
    pass


class ModelConfig(C.Structure):
    """xe_model_config (include/xdna_engine.h)."""
    _fields_ = [(n, C.c_int) for n in ("family", "n_layers", "d_model", "n_heads",
                                       "n_kv_heads", "head_dim", "ffn", "vocab",
                                       "max_pos", "max_ctx", "wdtype")] + \
               [("eps", C.c_float), ("rope_theta", C.c_float), ("n_cross", C.c_int)]

    def replace(self, **kw):
        c = ModelConfig()
        for name, _ in self._fields_:
            setattr(c, name, kw.get(name, getattr(self, name)))
        return c

    def as_dict(self):
        return {name: getattr(self, name) for name, _ in self._fields_}


def _cfg(**kw):
    c = ModelConfig()
    for k, v in kw.items():
        setattr(c, k, v)
    return c


# OPT-125m architecture (opt125m_decode.rs:17-21).
OPT_125M = _cfg(family=XE_OPT, n_layers=12, d_model=768, n_heads=12, n_kv_heads=12, head_dim=64,
                ffn=3072, vocab=50272, max_pos=2048, max_ctx=2048, wdtype=XE_I8, eps=1e-5,
                rope_theta=0.0, n_cross=0)
# Whisper-small decoder (whisper_decoder.rs D/N_HEADS/FFN/VOCAB).
WHISPER_SMALL = _cfg(family=XE_WHISPER, n_layers=12, d_model=768, n_heads=12, n_kv_heads=12,
                     head_dim=64, ffn=3072, vocab=51865, max_pos=448, max_ctx=448, wdtype=XE_I8,
                     eps=1e-5, rope_theta=0.0, n_cross=1500)
# Gemma-3-1B (npu-gemma/src/config.rs:156-170; one RoPE theta 1e6).
GEMMA3_1B = _cfg(family=XE_GEMMA3, n_layers=26, d_model=1152, n_heads=4, n_kv_heads=1,
                 head_dim=256, ffn=6912, vocab=262144, max_pos=0, max_ctx=4096, wdtype=XE_I8,
                 eps=1e-6, rope_theta=1e6, n_cross=0)

_lib = None


def lib():
    """Load libxdna_engine.so (raises if it was not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise XdnaError("libxdna_engine.so not built: run `make -C xdna-engine_amd` "
                        "or __graft_entry__.build()")
    L = C.CDLL(LIB_PATH)
    vp, i, f, sz, u64 = C.c_void_p, C.c_int, C.c_float, C.c_size_t, C.c_uint64
    sig = {
        "xe_last_error": (C.c_char_p, []),
        "xe_abi_version": (i, []),
        "xe_device_count": (i, []),
        "xe_device_open": (vp, [i]),
        "xe_device_close": (None, [vp]),
        "xe_device_synchronize": (i, [vp]),
        "xe_device_name": (i, [vp, C.c_char_p, i]),
        "xe_buf_alloc": (vp, [vp, sz]),
        "xe_buf_free": (None, [vp]),
        "xe_buf_write": (i, [vp, vp, sz, sz]),
        "xe_buf_read": (i, [vp, vp, sz, sz]),
        "xe_buf_device_ptr": (vp, [vp]),
        "xe_buf_size": (sz, [vp]),
        "xe_buf_fill_synthetic": (i, [vp, sz, i, u64, C.c_uint32, u64, f, f, sz]),
        "xe_buf_copy": (i, [vp, sz, vp, sz, sz]),
        "xe_register_weight_view": (vp, [vp, i, i, i, vp, vp, vp, vp]),
        "xe_probe_gemv": (i, [vp, vp, i, vp, i, i, vp, i, i, C.POINTER(C.c_double)]),
        "xe_probe_attn": (i, [vp, vp, vp, vp, vp, i, i, i, i, i, f, vp, i, i, C.POINTER(C.c_double)]),
        "xe_ctx_create": (vp, [vp]),
        "xe_ctx_destroy": (None, [vp]),
        "xe_ctx_dispatches": (u64, [vp]),
        "xe_ctx_reset_dispatches": (None, [vp]),
        "xe_ctx_synchronize": (i, [vp]),
        "xe_register_weight": (vp, [vp, i, i, i, vp, i, vp]),
        "xe_register_weight_q8": (vp, [vp, i, i, vp, vp, vp]),
        "xe_register_weight_bfp16": (vp, [vp, i, i, vp, vp, vp]),
        "xe_register_weight_q4": (vp, [vp, i, i, vp, vp, vp]),
        "xe_register_weight_q8_rule": (vp, [vp, i, i, vp, i, vp, i]),
        "xe_register_weight_q4_kn": (vp, [vp, i, i, vp, vp, vp]),
        "xe_register_weight_bf16": (vp, [vp, i, i, vp, vp]),
        "xe_register_fused": (vp, [vp, i, i, i, vp, i, i, vp, vp, f, vp]),
        "xe_weight_set_norm": (i, [vp, i, vp, vp, f]),
        "xe_weight_free": (None, [vp]),
        "xe_weight_shape": (i, [vp, C.POINTER(i), C.POINTER(i), C.POINTER(i)]),
        "xe_gemv": (i, [vp, vp, vp, i, i, vp]),
        "xe_fused_norm_gemv": (i, [vp, vp, vp, i, i, vp]),
        "xe_gemv_dev": (i, [vp, vp, vp, i, i, vp]),
        "xe_gemv_i8act": (i, [vp, vp, vp, i, vp]),
        "xe_gemv_i8act_dev": (i, [vp, vp, vp, i, vp]),
        "xe_w8a8_linear": (i, [vp, vp, vp, i, vp, C.POINTER(f)]),
        "xe_w8a8_linear_dev": (i, [vp, vp, vp, i, i, vp, vp]),
        "xe_attn_decode": (i, [vp, vp, vp, vp, vp, i, i, i, i, i, f, vp]),
        "xe_attn_decode_dev": (i, [vp, vp, vp, vp, vp, i, i, i, i, i, f, vp]),
        "xe_attn_decode_dev_static": (i, [vp, vp, vp, vp, vp, i, i, i, i, i, f, vp]),
        "xe_decoder_create": (vp, [vp, C.POINTER(ModelConfig), i]),
        "xe_decoder_destroy": (None, [vp]),
        "xe_decoder_init_synthetic": (i, [vp, u64]),
        "xe_decoder_set_tensor": (i, [vp, i, i, vp, sz]),
        "xe_decoder_get_tensor_q8": (i, [vp, i, i, vp, vp]),
        "xe_decoder_reset": (i, [vp]),
        "xe_decoder_prime_kv": (i, [vp, i, i, u64]),
        "xe_decoder_set_cross": (i, [vp, vp]),
        "xe_decoder_set_cross_int8": (i, [vp, i, i]),
        "xe_decoder_step": (i, [vp, vp, vp, i, vp, vp]),
        "xe_decoder_generate": (i, [vp, vp, i, i, i, vp]),
        "xe_decoder_set_stop": (i, [vp, C.c_int32]),
        "xe_decoder_generate_until": (i, [vp, vp, i, i, i, C.c_int32, vp, vp]),
        "xe_decoder_last_step_us": (C.c_double, [vp]),
        "xe_decoder_feed": (i, [vp, vp, i, i]),
        "xe_decoder_decode": (i, [vp, i, i, vp, C.POINTER(C.c_double)]),
        "xe_decoder_profile_step": (i, [vp, i, i, vp, vp, vp]),
        "xe_decoder_weight_bytes": (u64, [vp]),
        "xe_decoder_executor": (i, [vp, i]),
        "xe_ctx_record": (vp, [vp]),
        "xe_run_query": (i, [vp]),
        "xe_run_wait": (i, [vp]),
        "xe_run_free": (None, [vp]),
        "xe_resident_open": (vp, [vp, i]),
        "xe_resident_close": (None, [vp]),
        "xe_resident_write": (i, [vp, vp, vp]),
        "xe_resident_dispatch": (i, [vp]),
        "xe_resident_dispatch_start": (vp, [vp]),
        "xe_resident_read": (i, [vp, vp, vp]),
        "xe_model_tensor_shape": (i, [C.POINTER(ModelConfig), i, i, C.POINTER(i), C.POINTER(i)]),
        "xe_decoder_config": (i, [vp, C.POINTER(ModelConfig)]),
        "xe_decoder_load_safetensors": (i, [vp, C.c_char_p]),
        "xe_safetensors_plan": (i, [C.c_char_p, C.POINTER(ModelConfig), C.c_char_p, i]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name, None)
        if fn is None:
            continue
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def last_error():
    return lib().xe_last_error().decode()


def _check(rc):
    if rc is None or (isinstance(rc, int) and rc < 0):
        raise XdnaError(last_error())
    return rc


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _f32(a):
    return None if a is None else np.ascontiguousarray(a, np.float32)


def device_count():
    return lib().xe_device_count()


class Device:
    """rust/npu-xrt Device: one GPU and its default-priority stream."""

    def __init__(self, ordinal=0):
        self.h = lib().xe_device_open(ordinal)
        if not self.h:
            raise XdnaError(last_error())

    def name(self):
        buf = C.create_string_buffer(64)
        _check(lib().xe_device_name(self.h, buf, 64))
        return buf.value.decode()

    def synchronize(self):
        _check(lib().xe_device_synchronize(self.h))

    def close(self):
        if self.h:
            lib().xe_device_close(self.h)
            self.h = None


class Buf:
    """rust/npu-xrt Bo: device memory."""

    def __init__(self, dev, nbytes):
        self.dev = dev
        self.h = lib().xe_buf_alloc(dev.h, nbytes)
        if not self.h:
            raise XdnaError(last_error())
        self.nbytes = nbytes

    @classmethod
    def from_array(cls, dev, a):
        a = np.ascontiguousarray(a)
        b = cls(dev, max(a.nbytes, 1))
        b.write(a)
        return b

    @property
    def ptr(self):
        return lib().xe_buf_device_ptr(self.h)

    def write(self, a, offset=0):
        a = np.ascontiguousarray(a)
        _check(lib().xe_buf_write(self.h, _p(a), a.nbytes, offset))

    def read(self, dtype, count, offset=0):
        out = np.empty(count, dtype)
        _check(lib().xe_buf_read(self.h, _p(out), out.nbytes, offset))
        return out

    def copy_from(self, src, nbytes, dst_off=0, src_off=0):
        """Device-to-device copy by the library's streaming copy kernel."""
        _check(lib().xe_buf_copy(self.h, dst_off, src.h, src_off, nbytes))

    def fill_synthetic(self, dtype, seed, stream, count, mean=0.0, std=1.0, start=0, offset=0):
        """Elements [start, start+count) of the synthetic stream (seed, stream)
        written at byte offset, as XE_F32 / XE_BF16 / XE_I8 (on the device)."""
        _check(lib().xe_buf_fill_synthetic(self.h, offset, dtype, seed, stream, start, mean, std,
                                           count))

    def free(self):
        if self.h:
            lib().xe_buf_free(self.h)
            self.h = None


class Norm:
    """ctx_decode.rs:74-79 Norm, plus Gemma's (1 + w) RMSNorm."""

    def __init__(self, kind, gamma, beta=None, eps=1e-5):
        self.kind, self.gamma, self.beta, self.eps = kind, _f32(gamma), _f32(beta), eps

    @staticmethod
    def Ln(gamma, beta, eps=1e-5):
        return Norm(XE_NORM_LN, gamma, beta, eps)

    @staticmethod
    def Rms(gamma, eps=1e-5):
        return Norm(XE_NORM_RMS, gamma, None, eps)

    @staticmethod
    def Rms1p(w, eps=1e-6):
        return Norm(XE_NORM_RMS1P, w, None, eps)


class Weight:
    def __init__(self, h):
        if not h:
            raise XdnaError(last_error())
        self.h = h
        m, k, d = C.c_int(), C.c_int(), C.c_int()
        _check(lib().xe_weight_shape(h, C.byref(m), C.byref(k), C.byref(d)))
        self.m, self.k, self.wdtype = m.value, k.value, d.value

    def free(self):
        if self.h:
            lib().xe_weight_free(self.h)
            self.h = None


class CtxDecode:
    """ctx_decode.rs:142-694 CtxDecode over the GPU: resident weights, GEMV,
    fused norm+GEMV and single-query attention."""

    def __init__(self, dev):
        self.dev = dev
        self.h = lib().xe_ctx_create(dev.h)
        if not self.h:
            raise XdnaError(last_error())

    def close(self):
        if self.h:
            lib().xe_ctx_destroy(self.h)
            self.h = None

    def dispatches(self):
        return lib().xe_ctx_dispatches(self.h)

    def reset_dispatches(self):
        lib().xe_ctx_reset_dispatches(self.h)

    def synchronize(self):
        _check(lib().xe_ctx_synchronize(self.h))

    def record(self):
        """A run handle on the work queued so far (xe_ctx_record)."""
        return Run(lib().xe_ctx_record(self.h))

    # -- registration (ctx_decode.rs:269-317, 566-612) --
    def register_weight(self, w, wdtype=XE_I8, layout=XE_LAYOUT_MK, bias=None):
        w = _f32(w)
        m, k = (w.shape if layout == XE_LAYOUT_MK else w.shape[::-1])
        b = _f32(bias)
        return Weight(lib().xe_register_weight(self.h, wdtype, m, k, _p(w), layout, _p(b)))

    def register_weight_q8(self, q, scales, bias=None):
        q = np.ascontiguousarray(q, np.int8)
        s, b = _f32(scales), _f32(bias)
        m, k = q.shape
        return Weight(lib().xe_register_weight_q8(self.h, m, k, _p(q), _p(s), _p(b)))

    def register_weight_q8_rule(self, w, rule, layout=XE_LAYOUT_MK, bias=None):
        """int8 under a reference rule: XE_Q8_LIN (Lin::load) or XE_Q8_ELF
        (gen_decode.py qrow: half-even, bf16 scale)."""
        w = _f32(w)
        m, k = (w.shape if layout == XE_LAYOUT_MK else w.shape[::-1])
        b = _f32(bias)
        return Weight(lib().xe_register_weight_q8_rule(self.h, m, k, _p(w), layout, _p(b), rule))

    def register_weight_q4(self, packed, scales, bias=None):
        """int4 [m, k/2] packed along k (opt125m_decode.rs:63-105 codes)."""
        packed = np.ascontiguousarray(packed, np.uint8)
        s, b = _f32(scales), _f32(bias)
        m, k2 = packed.shape
        return Weight(lib().xe_register_weight_q4(self.h, m, 2 * k2, _p(packed), _p(s), _p(b)))

    def register_weight_q4_kn(self, packed_kn, scales, bias=None):
        """int4 in the reference's own [K, N/2] packing (Lin::load)."""
        packed_kn = np.ascontiguousarray(packed_kn, np.uint8)
        s, b = _f32(scales), _f32(bias)
        k, m2 = packed_kn.shape
        return Weight(lib().xe_register_weight_q4_kn(self.h, 2 * m2, k, _p(packed_kn), _p(s), _p(b)))

    def register_weight_bfp16(self, mant, exps, bias=None):
        mant = np.ascontiguousarray(mant, np.int8)
        exps = np.ascontiguousarray(exps, np.uint8)
        m, k = mant.shape
        b = _f32(bias)
        return Weight(lib().xe_register_weight_bfp16(self.h, m, k, _p(mant), _p(exps), _p(b)))

    def register_weight_bf16(self, bits, bias=None):
        bits = np.ascontiguousarray(bits, np.uint16)
        m, k = bits.shape
        b = _f32(bias)
        return Weight(lib().xe_register_weight_bf16(self.h, m, k, _p(bits), _p(b)))

    def register_fused(self, w, norm, wdtype=XE_I8, layout=XE_LAYOUT_MK, bias=None):
        w = _f32(w)
        m, k = (w.shape if layout == XE_LAYOUT_MK else w.shape[::-1])
        b = _f32(bias)
        return Weight(lib().xe_register_fused(self.h, wdtype, m, k, _p(w), layout, norm.kind,
                                              _p(norm.gamma), _p(norm.beta), norm.eps, _p(b)))

    def set_norm(self, weight, norm):
        _check(lib().xe_weight_set_norm(weight.h, norm.kind, _p(norm.gamma), _p(norm.beta),
                                        norm.eps))

    def register_weight_view(self, wdtype, m, k, w_ptr, scale_ptr=None, exps_ptr=None,
                             bias_ptr=None):
        """A weight over device memory (Buf.ptr + offset); no copy."""
        return Weight(lib().xe_register_weight_view(self.h, wdtype, m, k, w_ptr, scale_ptr,
                                                    exps_ptr, bias_ptr))

    def probe_gemv(self, weights, x_ptr, x_dtype, batch, y_ptr, reps, eager=False):
        """Device microseconds per launch of xe_gemv_dev rotating over weights
        (graph replays; eager: plain launches)."""
        arr = (C.c_void_p * len(weights))(*[w.h for w in weights])
        us = C.c_double()
        _check(lib().xe_probe_gemv(self.h, arr, len(weights), x_ptr, x_dtype, batch, y_ptr, reps,
                                   1 if eager else 0, C.byref(us)))
        return us.value

    def probe_attn(self, q_ptr, k_ptr, v_ptr, lens_ptr, b, hq, hkv, hd, max_ctx, scale, out_ptr,
                   reps, eager=False):
        """Device microseconds per xe_attn_decode_dev call."""
        us = C.c_double()
        _check(lib().xe_probe_attn(self.h, q_ptr, k_ptr, v_ptr, lens_ptr, b, hq, hkv, hd, max_ctx,
                                   scale, out_ptr, reps, 1 if eager else 0, C.byref(us)))
        return us.value

    # -- execution (ctx_decode.rs:325-366, 617-643) --
    def _run(self, fn, weight, x):
        x = np.asarray(x)
        squeeze = x.ndim == 1
        x2 = np.atleast_2d(x)
        if x2.dtype == np.uint16:          # bf16 bits
            xd, dt = np.ascontiguousarray(x2), XE_BF16
        else:
            xd, dt = np.ascontiguousarray(x2, np.float32), XE_F32
        b = xd.shape[0]
        y = np.empty((b, weight.m), np.float32)
        _check(fn(self.h, weight.h, _p(xd), dt, b, _p(y)))
        return y[0] if squeeze else y

    def gemv(self, weight, x):
        return self._run(lib().xe_gemv, weight, x)

    def fused_norm_gemv(self, weight, x):
        return self._run(lib().xe_fused_norm_gemv, weight, x)

    def gemv_dev(self, weight, x_buf, batch, y_buf, x_dtype=XE_F32):
        _check(lib().xe_gemv_dev(self.h, weight.h, x_buf.ptr, x_dtype, batch, y_buf.ptr))

    def gemv_i8act(self, weight, xq):
        xq = np.ascontiguousarray(np.atleast_2d(xq), np.int8)
        b = xq.shape[0]
        acc = np.empty((b, weight.m), np.int32)
        _check(lib().xe_gemv_i8act(self.h, weight.h, _p(xq), b, _p(acc)))
        return acc

    def w8a8_linear(self, weight, x):
        x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
        b = x.shape[0]
        y = np.empty((b, weight.m), np.float32)
        sa = C.c_float()
        _check(lib().xe_w8a8_linear(self.h, weight.h, _p(x), b, _p(y), C.byref(sa)))
        return y, sa.value

    def w8a8_linear_dev(self, weight, x_buf, batch, epi, y_buf, sa_buf=None):
        """Device-pointer W8A8 (asynchronous); epi: XE_EPI_NONE/BIAS/SILU_BIAS."""
        _check(lib().xe_w8a8_linear_dev(self.h, weight.h, x_buf.ptr, batch, epi, y_buf.ptr,
                                        None if sa_buf is None else sa_buf.ptr))

    # -- attention (ctx_decode.rs:468-555) --
    def attn(self, q, kc, vc, lens, scale):
        """q fp32 [b, hq, hd]; kc/vc bf16 bits [b, hkv, max_ctx, hd]; lens [b]."""
        q = np.ascontiguousarray(q, np.float32)
        kc = np.ascontiguousarray(kc, np.uint16)
        vc = np.ascontiguousarray(vc, np.uint16)
        lens = np.ascontiguousarray(lens, np.int32)
        b, hq, hd = q.shape
        _, hkv, max_ctx, _ = kc.shape
        out = np.empty_like(q)
        _check(lib().xe_attn_decode(self.h, _p(q), _p(kc), _p(vc), _p(lens), b, hq, hkv, hd,
                                    max_ctx, scale, _p(out)))
        return out

    def attn_dev(self, q_buf, k_buf, v_buf, lens_buf, b, hq, hkv, hd, max_ctx, scale, out_buf):
        _check(lib().xe_attn_decode_dev(self.h, q_buf.ptr, k_buf.ptr, v_buf.ptr, lens_buf.ptr, b,
                                        hq, hkv, hd, max_ctx, scale, out_buf.ptr))


class Run:
    """An asynchronous submission (shim_run_* handles)."""

    def __init__(self, h):
        if not h:
            raise XdnaError(last_error())
        self.h = h

    def query(self):
        return _check(lib().xe_run_query(self.h)) == 1

    def wait(self):
        _check(lib().xe_run_wait(self.h))

    def free(self):
        if self.h:
            lib().xe_run_free(self.h)
            self.h = None


class Resident:
    """ElfResident: the decode step of `batch` streams, bound once."""

    def __init__(self, dec, batch):
        self.dec, self.batch = dec, batch
        self.h = lib().xe_resident_open(dec.h, batch)
        if not self.h:
            raise XdnaError(last_error())

    def write(self, tokens, pos):
        t = np.ascontiguousarray(tokens, np.int32)
        p = np.ascontiguousarray(pos, np.int32)
        assert t.size == self.batch and p.size == self.batch
        _check(lib().xe_resident_write(self.h, _p(t), _p(p)))

    def dispatch(self):
        _check(lib().xe_resident_dispatch(self.h))

    def dispatch_start(self):
        return Run(lib().xe_resident_dispatch_start(self.h))

    def read(self, want_logits=False):
        nxt = np.empty(self.batch, np.int32)
        lg = np.empty((self.batch, self.dec.cfg.vocab), np.float32) if want_logits else None
        _check(lib().xe_resident_read(self.h, _p(nxt), _p(lg)))
        return nxt, lg

    def close(self):
        if self.h:
            lib().xe_resident_close(self.h)
            self.h = None


def tensor_shape(cfg, kind, layer):
    """(rows, cols) of tensor (kind, layer) of cfg, or None if the family has none."""
    r, c = C.c_int(), C.c_int()
    if lib().xe_model_tensor_shape(C.byref(cfg), kind, layer, C.byref(r), C.byref(c)) != 0:
        return None
    return r.value, c.value


def safetensors_plan(path, cfg):
    """Host-only dry run of the loader: {name: (kind, layer, transposed) or None}
    and the naming ("arena" / "hf")."""
    buf = C.create_string_buffer(1 << 20)
    _check(lib().xe_safetensors_plan(os.fsencode(path), C.byref(cfg), buf, len(buf)))
    lines = buf.value.decode().split("\n")
    out = {}
    for ln in lines[1:]:
        name, _, rhs = ln.rpartition(" -> ")
        if rhs == "skipped":
            out[name] = None
        else:
            f = rhs.split()
            out[name] = (int(f[0]), int(f[1]), len(f) > 2)
    return lines[0], out


class Decoder:
    """Decode backend: reset / precompute_cross / step / generate."""

    def __init__(self, dev, cfg, max_batch=1):
        self.dev, self.cfg, self.max_batch = dev, cfg, max_batch
        self.batch = None
        self.h = lib().xe_decoder_create(dev.h, C.byref(cfg), max_batch)
        if not self.h:
            raise XdnaError(last_error())

    def close(self):
        if self.h:
            lib().xe_decoder_destroy(self.h)
            self.h = None

    def init_synthetic(self, seed):
        _check(lib().xe_decoder_init_synthetic(self.h, seed))

    def set_tensor(self, kind, layer, data):
        d = _f32(data).reshape(-1)
        _check(lib().xe_decoder_set_tensor(self.h, kind, layer, _p(d), d.size))

    def load_safetensors(self, path):
        """npu-weights arena / Hugging Face checkpoint -> the decoder's
        weights; returns the number of tensors loaded."""
        return _check(lib().xe_decoder_load_safetensors(self.h, os.fsencode(path)))

    def get_tensor_q8(self, kind, layer, rows, cols):
        q = np.empty((rows, cols), np.int8)
        s = np.empty(rows, np.float32)
        _check(lib().xe_decoder_get_tensor_q8(self.h, kind, layer, _p(q), _p(s)))
        return q, s

    def reset(self):
        _check(lib().xe_decoder_reset(self.h))

    def prime_kv(self, stream, n_pos, seed=0):
        """Synthetic bf16 K/V rows [0, n_pos) of one stream (the oracle's
        prime_kv values); the stream's next position becomes n_pos."""
        _check(lib().xe_decoder_prime_kv(self.h, stream, n_pos, seed))

    def precompute_cross(self, enc=None):
        e = _f32(enc)
        _check(lib().xe_decoder_set_cross(self.h, _p(e)))

    def set_cross_int8(self, k_int8=True, v_int8=True):
        """Per-utterance int8 cross K / V from the next precompute_cross on."""
        _check(lib().xe_decoder_set_cross_int8(self.h, int(bool(k_int8)), int(bool(v_int8))))

    def step(self, tokens, pos, want_logits=True):
        tokens = np.ascontiguousarray(np.atleast_1d(tokens), np.int32)
        pos = np.ascontiguousarray(np.atleast_1d(pos), np.int32)
        b = tokens.shape[0]
        logits = np.empty((b, self.cfg.vocab), np.float32) if want_logits else None
        nxt = np.empty(b, np.int32)
        _check(lib().xe_decoder_step(self.h, _p(tokens), _p(pos), b, _p(logits), _p(nxt)))
        return logits, nxt

    def generate(self, prompt, n_new):
        prompt = np.ascontiguousarray(np.atleast_2d(prompt), np.int32)
        b, n_prompt = prompt.shape
        out = np.empty((b, n_new), np.int32)
        _check(lib().xe_decoder_generate(self.h, _p(prompt), n_prompt, b, n_new, _p(out)))
        return out

    def set_stop(self, stop_id):
        """Stop token of the device greedy loop (-1: none)."""
        _check(lib().xe_decoder_set_stop(self.h, int(stop_id)))

    def generate_until(self, prompt, max_new, stop_id):
        """(out [batch, max_new] padded with stop_id, n_out [batch])."""
        prompt = np.ascontiguousarray(np.atleast_2d(prompt), np.int32)
        b, n_prompt = prompt.shape
        out = np.empty((b, max_new), np.int32)
        n_out = np.empty(b, np.int32)
        _check(lib().xe_decoder_generate_until(self.h, _p(prompt), n_prompt, b, max_new, int(stop_id),
                                               _p(out), _p(n_out)))
        return out, n_out

    def feed(self, prompt):
        prompt = np.ascontiguousarray(np.atleast_2d(prompt), np.int32)
        b, n = prompt.shape
        _check(lib().xe_decoder_feed(self.h, _p(prompt), n, b))
        self.batch = b

    def decode(self, n_steps, batch=None, want_tokens=True):
        """Returns (tokens [batch, n_steps] or None, device microseconds)."""
        b = batch or self.batch
        out = np.empty((b, n_steps), np.int32) if want_tokens else None
        us = C.c_double()
        self.steps_run = _check(lib().xe_decoder_decode(self.h, b, n_steps, _p(out), C.byref(us)))
        return out, us.value

    def profile_step(self, batch=None, max_entries=4096):
        """One eager step, an event after each launch: [(label, us, bytes)]."""
        b = batch or self.batch
        labels = C.create_string_buffer(32 * max_entries)
        us = np.empty(max_entries, np.float64)
        by = np.empty(max_entries, np.float64)
        n = _check(lib().xe_decoder_profile_step(self.h, b, max_entries, labels, _p(us), _p(by)))
        raw = labels.raw
        return [(raw[32 * i:32 * i + 32].split(b"\0")[0].decode(), float(us[i]), float(by[i]))
                for i in range(n)]

    def executor(self, batch=None):
        """Name of the executor a step of `batch` streams runs on."""
        b = batch or self.batch or 1
        return EXECUTORS[_check(lib().xe_decoder_executor(self.h, b))]

    def last_step_us(self):
        return lib().xe_decoder_last_step_us(self.h)

    def weight_bytes(self):
        return lib().xe_decoder_weight_bytes(self.h)
