"""ctypes binding of the CPU oracle (oracle/liboracle.so) -- test infrastructure.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load the
oracle; it is the checker, never the thing measured or shipped.
"""
import ctypes as C
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "liboracle.so")

f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")


class ModelConfig(C.Structure):
    """Mirror of xe_model_config (include/xdna_engine.h)."""
    _fields_ = [(n, C.c_int) for n in ("family", "n_layers", "d_model", "n_heads",
                                       "n_kv_heads", "head_dim", "ffn", "vocab",
                                       "max_pos", "max_ctx", "wdtype")] + \
               [("eps", C.c_float), ("rope_theta", C.c_float), ("n_cross", C.c_int)]


def _build_if_missing():
    if not os.path.exists(ORACLE_SO):
        subprocess.check_call(["make", "-s", "-C", os.path.join(ROOT, "oracle")])


_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    _build_if_missing()
    L = C.CDLL(ORACLE_SO)
    sig = {
        "xo_f32_to_bf16_bits": (C.c_uint16, [C.c_float]),
        "xo_bf16_bits_to_f32": (C.c_float, [C.c_uint16]),
        "xo_bf16_round": (C.c_float, [C.c_float]),
        "xo_pack_bf16": (None, [f32p, u16p, C.c_size_t]),
        "xo_unpack_bf16": (None, [u16p, f32p, C.c_size_t]),
        "xo_layer_norm": (None, [f32p, C.c_int, C.c_int, f32p, f32p, C.c_float, f32p]),
        "xo_layer_norm_normalize": (None, [f32p, C.c_int, C.c_int, C.c_float, f32p]),
        "xo_rmsnorm": (None, [f32p, C.c_int, f32p, C.c_float, f32p]),
        "xo_erf_as": (C.c_float, [C.c_float]),
        "xo_gelu_erf": (C.c_float, [C.c_float]),
        "xo_gelu_tanh": (C.c_float, [C.c_float]),
        "xo_fast_exp_nonpos": (C.c_float, [C.c_float]),
        "xo_quant_i8": (C.c_int8, [C.c_float, C.c_float]),
        "xo_quant_scale": (C.c_float, [f32p, C.c_size_t]),
        "xo_quant_rows_i8": (None, [f32p, C.c_int, C.c_int, i8p, f32p]),
        "xo_quant_cols_i8": (None, [f32p, C.c_int, C.c_int, i8p, f32p]),
        "xo_quant_rows_i8_elf": (None, [f32p, C.c_int, C.c_int, i8p, f32p]),
        "xo_dequant_epi": (None, [i32p, C.c_int, C.c_int, C.c_float, f32p, C.c_void_p, f32p]),
        "xo_gemv_i8": (None, [f32p, C.c_int, C.c_int, C.c_int, i8p, f32p, C.c_void_p, f32p]),
        "xo_gemv_i8_rowblocked": (None, [f32p, C.c_int, C.c_int, C.c_int, i8p, f32p, C.c_void_p, f32p]),
        "xo_lin_fwd_i8_kn": (None, [f32p, C.c_int, C.c_int, C.c_int, i8p, f32p, C.c_void_p, f32p]),
        "xo_quant_cols_i4": (None, [f32p, C.c_int, C.c_int, u8p, f32p]),
        "xo_lin_fwd_i4_kn": (None, [f32p, C.c_int, C.c_int, C.c_int, u8p, f32p, C.c_void_p, f32p]),
        "xo_quant_rows_i4": (None, [f32p, C.c_int, C.c_int, u8p, f32p]),
        "xo_gemv_i4": (None, [f32p, C.c_int, C.c_int, C.c_int, u8p, f32p, C.c_void_p, f32p]),
        "xo_gemv_f32": (None, [f32p, C.c_int, C.c_int, C.c_int, f32p, C.c_void_p, f32p]),
        "xo_gemv_bf16w": (None, [f32p, C.c_int, C.c_int, C.c_int, u16p, C.c_void_p, f32p]),
        "xo_bfp16_encode": (None, [f32p, C.c_int, C.c_int, i8p, u8p]),
        "xo_bfp16_decode": (None, [i8p, u8p, C.c_int, C.c_int, f32p]),
        "xo_gemv_bfp16": (None, [f32p, C.c_int, C.c_int, C.c_int, i8p, u8p, C.c_void_p, f32p]),
        "xo_gemm_i8i8_i32": (None, [i8p, C.c_int, C.c_int, i8p, C.c_int, i32p]),
        "xo_w8a8_linear": (None, [f32p, C.c_int, C.c_int, i8p, f32p, C.c_int, C.c_void_p, f32p,
                                  C.POINTER(C.c_float)]),
        "xo_fast_sigmoid": (C.c_float, [C.c_float]),
        "xo_w8a8_linear_epi": (None, [f32p, C.c_int, C.c_int, i8p, f32p, C.c_int, C.c_void_p, C.c_int,
                                      f32p, C.POINTER(C.c_float)]),
        "xo_norm_row": (None, [f32p, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_float, f32p]),
        "xo_fold_weight": (None, [f32p, C.c_int, C.c_int, f32p, C.c_void_p, C.c_void_p, f32p, f32p]),
        "xo_attend_one": (None, [f32p, f32p, f32p, C.c_int, C.c_int, C.c_int, f32p]),
        "xo_attn_decode": (None, [f32p, u16p, u16p, i32p, C.c_int, C.c_int, C.c_int, C.c_int,
                                  C.c_int, C.c_float, f32p]),
        "xo_attn_online": (None, [f32p, u16p, u16p, C.c_int, C.c_int, C.c_float, f32p]),
        "xo_rope": (None, [f32p, C.c_int, C.c_int, C.c_int, f32p, f32p, f32p]),
        "xo_argmax_first": (C.c_int, [f32p, C.c_int]),
        "xo_argmax_last": (C.c_int, [f32p, C.c_int]),
        "xo_synth_base": (C.c_uint64, [C.c_uint64, C.c_uint32]),
        "xo_synth_value": (C.c_float, [C.c_uint64, C.c_uint64, C.c_float, C.c_float]),
        "xo_synth_fill": (None, [C.c_uint64, C.c_uint32, C.c_float, C.c_float, f32p, C.c_size_t]),
        "xo_synth_fill_range": (None, [C.c_uint64, C.c_uint32, C.c_float, C.c_float, C.c_uint64,
                                       f32p, C.c_size_t]),
        "xo_model_create": (C.c_void_p, [C.POINTER(ModelConfig), C.c_uint64, C.c_int]),
        "xo_model_free": (None, [C.c_void_p]),
        "xo_model_reset": (None, [C.c_void_p]),
        "xo_model_set_kv_f32": (C.c_int, [C.c_void_p, C.c_int]),
        "xo_model_set_mutation": (C.c_int, [C.c_void_p, C.c_int]),
        "xo_model_set_kouter": (C.c_int, [C.c_void_p, C.c_int]),
        "xo_model_prime_kv": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_uint64]),
        "xo_model_set_cross": (C.c_int, [C.c_void_p, C.c_void_p]),
        "xo_model_set_cross_i8": (C.c_int, [C.c_void_p, C.c_int, C.c_int]),
        "xo_quant_cross_i8": (None, [f32p, C.c_int, C.c_int, C.c_int, i8p, f32p]),
        "xo_head_attend_x8": (None, [f32p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                     C.c_void_p, C.c_int, C.c_int, C.c_float, f32p, f32p]),
        "xo_model_step": (None, [C.c_void_p, i32p, i32p, C.c_int, f32p]),
        "xo_model_argmax": (C.c_int, [C.c_void_p, f32p]),
        "xo_model_tensor_numel": (C.c_size_t, [C.c_void_p, C.c_int, C.c_int]),
        "xo_model_tensor_f32": (C.c_int, [C.c_void_p, C.c_int, C.c_int, f32p]),
        "xo_model_tensor_q8": (C.c_int, [C.c_void_p, C.c_int, C.c_int, i8p, f32p]),
        "xo_model_generate": (C.c_int, [C.c_void_p, i32p, C.c_int, C.c_int, C.c_int, i32p,
                                        C.c_void_p]),
        "xo_model_generate_until": (C.c_int, [C.c_void_p, i32p, C.c_int, C.c_int, C.c_int, C.c_int,
                                              i32p, i32p, C.c_void_p]),
        "xo_set_threads": (None, [C.c_int]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def ptr(a):
    """Nullable array argument (None -> NULL)."""
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# ---- numpy-facing helpers -------------------------------------------------

def bf16_bits(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().xo_pack_bf16(x.reshape(-1), out.reshape(-1), x.size)
    return out


def bf16_to_f32(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def quant_rows_i8(w):
    w = np.ascontiguousarray(w, np.float32)
    m, k = w.shape
    q = np.empty((m, k), np.int8)
    s = np.empty(m, np.float32)
    lib().xo_quant_rows_i8(w, m, k, q, s)
    return q, s


def quant_rows_i8_elf(w):
    """gen_decode.py qrow: half-even rounding, scale stored as bf16."""
    w = np.ascontiguousarray(w, np.float32)
    m, k = w.shape
    q = np.empty((m, k), np.int8)
    s = np.empty(m, np.float32)
    lib().xo_quant_rows_i8_elf(w, m, k, q, s)
    return q, s


def quant_cross_i8(x, heads, hd):
    """Per-channel int8 of one layer's cross K or V (whisper_decoder.rs:1186-1219):
    x fp32 [T, heads*hd] -> q int8 [heads, T, hd], scales [heads*hd]."""
    x = np.ascontiguousarray(x, np.float32)
    t = x.shape[0]
    q = np.empty((heads, t, hd), np.int8)
    s = np.empty(heads * hd, np.float32)
    lib().xo_quant_cross_i8(x, t, heads, hd, q, s)
    return q, s


def head_attend_x8(q, scale, k8=None, sk=None, kb=None, v8=None, sv=None, vb=None):
    """One head over int8 (with channel scales) and/or bf16 keys / values [T, hd]."""
    q = np.ascontiguousarray(q, np.float32)
    hd = q.shape[0]
    arrs = [None if a is None else np.ascontiguousarray(a) for a in (k8, sk, kb, v8, sv, vb)]
    t = next(a.shape[0] for a in (arrs[0], arrs[2]) if a is not None)
    sc = np.empty(t, np.float32)
    out = np.empty(hd, np.float32)
    lib().xo_head_attend_x8(q, *[ptr(a) for a in arrs], t, hd, scale, sc, out)
    return out


def gemv_i8(x, q, s, bias=None):
    x = np.ascontiguousarray(x, np.float32)
    b = x.shape[0]
    m, k = q.shape
    y = np.empty((b, m), np.float32)
    lib().xo_gemv_i8(x, b, k, m, np.ascontiguousarray(q), np.ascontiguousarray(s, np.float32),
                     ptr(None if bias is None else np.ascontiguousarray(bias, np.float32)), y)
    return y


EPI_NONE, EPI_BIAS, EPI_SILU_BIAS = 0, 1, 2


def w8a8_linear(a, wq, ws, bias=None, epi=None):
    """forward_view_int8 + dequant_epi (ctx2.rs:771-830, 1386-1435); returns
    (out, scale_a)."""
    a = np.ascontiguousarray(a, np.float32)
    mp, k = a.shape
    m = wq.shape[0]
    if epi is None:
        epi = EPI_BIAS if bias is not None else EPI_NONE
    out = np.empty((mp, m), np.float32)
    sa = C.c_float()
    bb = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().xo_w8a8_linear_epi(a, mp, k, np.ascontiguousarray(wq, np.int8),
                             np.ascontiguousarray(ws, np.float32), m, ptr(bb), epi, out, C.byref(sa))
    return out, sa.value


def quant_rows_i4(w):
    """Lin::load int4 (opt125m_decode.rs:63-79) on an [M, K] matrix: packed
    uint8 [M, K/2] (k = 2j low nibble, 2j+1 high) and scales [M]."""
    w = np.ascontiguousarray(w, np.float32)
    m, k = w.shape
    q = np.empty((m, k // 2), np.uint8)
    s = np.empty(m, np.float32)
    lib().xo_quant_rows_i4(w, m, k, q, s)
    return q, s


def quant_cols_i4(w_kn):
    """Lin::load int4 in the reference's [K, N] layout: packed [K, N/2]."""
    w_kn = np.ascontiguousarray(w_kn, np.float32)
    k, n = w_kn.shape
    q = np.empty((k, n // 2), np.uint8)
    s = np.empty(n, np.float32)
    lib().xo_quant_cols_i4(w_kn, k, n, q, s)
    return q, s


def gemv_i4(x, packed, s, bias=None):
    x = np.ascontiguousarray(x, np.float32)
    b = x.shape[0]
    m, k2 = packed.shape
    y = np.empty((b, m), np.float32)
    bb = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().xo_gemv_i4(x, b, 2 * k2, m, np.ascontiguousarray(packed), np.ascontiguousarray(s, np.float32),
                     ptr(bb), y)
    return y


def lin_fwd_i4_kn(x, packed_kn, s, bias=None):
    x = np.ascontiguousarray(x, np.float32)
    b, k = x.shape
    n = 2 * packed_kn.shape[1]
    y = np.empty((b, n), np.float32)
    bb = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().xo_lin_fwd_i4_kn(x, b, k, n, np.ascontiguousarray(packed_kn),
                           np.ascontiguousarray(s, np.float32), ptr(bb), y)
    return y


def unpack_i4(packed):
    """Sign-extended nibbles of a packed [R, C/2] array as int8 [R, C]."""
    p = np.asarray(packed, np.uint8)
    lo = (p & 0x0F).astype(np.int8)
    hi = (p >> 4).astype(np.int8)
    out = np.empty((p.shape[0], 2 * p.shape[1]), np.int8)
    out[:, 0::2] = np.where(lo >= 8, lo - 16, lo)
    out[:, 1::2] = np.where(hi >= 8, hi - 16, hi)
    return out


def gemv_bf16w(x, wbits, bias=None):
    x = np.ascontiguousarray(x, np.float32)
    b = x.shape[0]
    m, k = wbits.shape
    y = np.empty((b, m), np.float32)
    bb = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().xo_gemv_bf16w(x, b, k, m, np.ascontiguousarray(wbits), ptr(bb), y)
    return y


def bfp16_encode(w):
    w = np.ascontiguousarray(w, np.float32)
    m, k = w.shape
    mant = np.empty((m, k), np.int8)
    exps = np.empty((m, k // 8), np.uint8)
    lib().xo_bfp16_encode(w, m, k, mant, exps)
    return mant, exps


def bfp16_decode(mant, exps):
    m, k = mant.shape
    w = np.empty((m, k), np.float32)
    lib().xo_bfp16_decode(np.ascontiguousarray(mant), np.ascontiguousarray(exps), m, k, w)
    return w


def gemv_bfp16(x, mant, exps, bias=None):
    x = np.ascontiguousarray(x, np.float32)
    b = x.shape[0]
    m, k = mant.shape
    y = np.empty((b, m), np.float32)
    bb = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().xo_gemv_bfp16(x, b, k, m, np.ascontiguousarray(mant), np.ascontiguousarray(exps),
                        ptr(bb), y)
    return y


def norm_rows(x, norm, gamma=None, beta=None, eps=1e-5):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    k = x.shape[-1]
    g = None if gamma is None else np.ascontiguousarray(gamma, np.float32)
    be = None if beta is None else np.ascontiguousarray(beta, np.float32)
    for i in range(x.shape[0]):
        row = np.ascontiguousarray(x[i])
        o = np.empty(k, np.float32)
        lib().xo_norm_row(row, k, norm, ptr(g), ptr(be), eps, o)
        out[i] = o
    return out


def attn_decode(q, kc, vc, lens, scale):
    q = np.ascontiguousarray(q, np.float32)
    b, hq, hd = q.shape
    _, hkv, max_ctx, _ = kc.shape
    out = np.empty_like(q)
    lib().xo_attn_decode(q, np.ascontiguousarray(kc), np.ascontiguousarray(vc),
                         np.ascontiguousarray(lens, np.int32), b, hq, hkv, hd, max_ctx,
                         scale, out)
    return out


def synth_fill(seed, tensor, mean, std, n):
    out = np.empty(n, np.float32)
    lib().xo_synth_fill(seed, tensor, mean, std, out, n)
    return out


def synth_range(seed, tensor, mean, std, start, n):
    """Elements [start, start+n) of a synthetic stream, fp32."""
    out = np.empty(n, np.float32)
    lib().xo_synth_fill_range(seed, tensor, mean, std, start, out, n)
    return out


def round_half_away_i8(v):
    """roundf + clamp(+-127) of fp32 values, as int8."""
    v = np.asarray(v, np.float64)
    r = np.sign(v) * np.floor(np.abs(v) + 0.5)
    return np.clip(r, -127, 127).astype(np.int8)


class OracleModel:
    """The oracle decoder (configs 1, 4, 5)."""

    def __init__(self, cfg, seed, batch=1):
        self.cfg = cfg
        self.batch = batch
        self.h = lib().xo_model_create(C.byref(cfg), seed, batch)
        assert self.h, "oracle model create failed"

    def close(self):
        if self.h:
            lib().xo_model_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def reset(self):
        lib().xo_model_reset(self.h)

    def set_mutation(self, code):
        """Plant a composition mistake (oracle XO_MUT_*), 0 for none."""
        assert lib().xo_model_set_mutation(self.h, code) == 0

    def set_kouter(self, on=True):
        """int8 linears through the reference's k-outer [K, N] loop."""
        assert lib().xo_model_set_kouter(self.h, 1 if on else 0) == 0

    def prime_kv(self, b, n_pos, seed=0):
        """Synthetic K/V rows [0, n_pos) of stream b (timing at long contexts)."""
        assert lib().xo_model_prime_kv(self.h, b, n_pos, seed) == 0

    def set_kv_f32(self, on=True):
        """fp32 K/V caches (the reference CPU decoders' choice) instead of bf16."""
        assert lib().xo_model_set_kv_f32(self.h, 1 if on else 0) == 0

    def set_cross_i8(self, k_int8=True, v_int8=True):
        """int8 per-utterance cross K / V from the next set_cross on."""
        assert lib().xo_model_set_cross_i8(self.h, int(bool(k_int8)), int(bool(v_int8))) == 0

    def set_cross(self, enc=None):
        e = None if enc is None else np.ascontiguousarray(enc, np.float32)
        assert lib().xo_model_set_cross(self.h, ptr(e)) == 0

    def step(self, tokens, pos):
        tokens = np.ascontiguousarray(tokens, np.int32)
        pos = np.ascontiguousarray(pos, np.int32)
        b = tokens.shape[0]
        logits = np.empty((b, self.cfg.vocab), np.float32)
        lib().xo_model_step(self.h, tokens, pos, b, logits)
        return logits

    def argmax(self, logits):
        return lib().xo_model_argmax(self.h, np.ascontiguousarray(logits, np.float32))

    def tensor_f32(self, kind, layer=-1):
        n = lib().xo_model_tensor_numel(self.h, kind, layer)
        out = np.empty(n, np.float32)
        assert lib().xo_model_tensor_f32(self.h, kind, layer, out) == 0
        return out

    def tensor_q8(self, kind, layer=-1):
        n = lib().xo_model_tensor_numel(self.h, kind, layer)
        q = np.empty(n, np.int8)
        rows = n // self._cols(kind)
        s = np.empty(rows, np.float32)
        assert lib().xo_model_tensor_q8(self.h, kind, layer, q, s) == 0
        return q.reshape(rows, -1), s

    def _cols(self, kind):
        c = self.cfg
        from_in = {XE_T_O_W: c.n_heads * c.head_dim, XE_T_FC2_W: c.ffn}
        return from_in.get(kind, c.d_model)

    def generate(self, prompt, n_new):
        prompt = np.ascontiguousarray(prompt, np.int32)
        b, n_prompt = prompt.shape
        out = np.empty((b, n_new), np.int32)
        margins = np.empty((b, n_new), np.float32)
        assert lib().xo_model_generate(self.h, prompt, n_prompt, b, n_new, out,
                                       margins.ctypes.data_as(C.c_void_p)) == 0
        return out, margins

    def generate_until(self, prompt, max_new, stop):
        """EOT rule: (out [b, max_new] padded with stop, n_out [b], margins)."""
        prompt = np.ascontiguousarray(prompt, np.int32)
        b, n_prompt = prompt.shape
        out = np.empty((b, max_new), np.int32)
        n_out = np.empty(b, np.int32)
        margins = np.empty((b, max_new), np.float32)
        assert lib().xo_model_generate_until(self.h, prompt, n_prompt, b, max_new, int(stop), out, n_out,
                                             margins.ctypes.data_as(C.c_void_p)) == 0
        return out, n_out, margins


# tensor kinds (include/xdna_engine.h enum xe_tensor)
XE_T_TOK_EMB, XE_T_POS_EMB, XE_T_LNF_W, XE_T_LNF_B, XE_T_ENC_OUT = 0, 1, 2, 3, 4
(XE_T_LN1_W, XE_T_LN1_B, XE_T_Q_W, XE_T_Q_B, XE_T_K_W, XE_T_K_B, XE_T_V_W, XE_T_V_B,
 XE_T_O_W, XE_T_O_B, XE_T_LN2_W, XE_T_LN2_B, XE_T_FC1_W, XE_T_FC1_B, XE_T_UP_W, XE_T_FC2_W,
 XE_T_FC2_B, XE_T_QNORM_W, XE_T_KNORM_W, XE_T_POST_ATTN_W, XE_T_POST_FFN_W, XE_T_LNX_W,
 XE_T_LNX_B, XE_T_XQ_W, XE_T_XQ_B, XE_T_XK_W, XE_T_XV_W, XE_T_XV_B, XE_T_XO_W,
 XE_T_XO_B) = range(8, 38)


def synth_id(kind, layer):
    return kind if layer < 0 else 64 * (layer + 1) + kind
