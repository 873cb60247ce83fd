"""Pins of the CPU oracle (CPU only).

Each test checks an oracle function against something other than its own
formula: the reference's in-source known-answer vectors
(tests/golden/reference_vectors.json, extracted by extract_reference_vectors.py),
an independent implementation (torch's bfloat16 cast, math.erf, numpy int64),
closed forms, invariants, or brute force.  A plausible mistake (dropped term,
wrong sign/index, transposed operand, wrong rounding mode) fails one of them.
"""
import ctypes as C
import json
import math
import os

import numpy as np
import pytest

import oracle_lib as O

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_vectors.json")))


def L():
    return O.lib()


def lcg_bits(seed, n):
    """The reference's LCG (npu-xrt/src/lib.rs:1109-1113): s = s*1664525 + 1013904223."""
    out = np.empty(n, np.uint32)
    s = seed
    for i in range(n):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = s
    return out


# ---------------------------------------------------------------- bf16 ----

def test_bf16_round_reference_values():
    for case in GOLD["bf16_round"]:
        got = L().xo_bf16_round(case["x"])
        assert abs(got - case["expected"]) <= case["tol"], case
    assert math.isnan(L().xo_bf16_round(float("nan")))


def test_bf16_unpack_exhaustive():
    # every bf16 pattern (npu-xrt/src/lib.rs:1063-1074): unpack is <<16
    bits = np.arange(65536, dtype=np.uint32)
    got = np.empty(65536, np.float32)
    L().xo_unpack_bf16(bits.astype(np.uint16), got, 65536)
    assert np.array_equal(got.view(np.uint32), bits << 16)


def test_bf16_pack_matches_torch_rne_on_lcg_sweep():
    torch = pytest.importorskip("torch")
    specials = np.array([0.0, -0.0, 1.0, -1.0, 0.5, -0.5, 1e-30, -1e-30, 1e30, -1e30,
                         np.finfo(np.float32).tiny, np.finfo(np.float32).max,
                         -np.finfo(np.float32).max, np.inf, -np.inf, 3.14159, 2.71828,
                         65504.0, 1.0 / 3.0, 1.5, -2.5, 0.123], np.float32)
    sweep = lcg_bits(0x12345678, 200_000).view(np.float32)
    x = np.concatenate([specials, sweep])
    got = O.bf16_bits(x)
    finite = ~np.isnan(x)
    want = torch.from_numpy(x[finite].copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got[finite], want)
    # NaN rule of f32_to_bf16_bits: (bits >> 16) | 0x40 (quiet), payload kept
    nb = x[~finite].view(np.uint32)
    assert np.array_equal(got[~finite], ((nb >> 16) | 0x40).astype(np.uint16))


def test_bf16_pack_unpack_roundtrip_idempotent():
    src = (lcg_bits(0xC0FFEE11, 4099) & 0xFFFF0000).view(np.float32)
    ok = ~np.isnan(src)
    back = O.bf16_to_f32(O.bf16_bits(src))
    assert np.array_equal(back[ok].view(np.uint32), src[ok].view(np.uint32))


# ------------------------------------------------------- norms / acts ----

def test_layer_norm_reference_vectors():
    g = GOLD["layer_norm"]
    x = np.array(g["x"], np.float32)
    out = np.empty(8, np.float32)
    L().xo_layer_norm(x, g["rows"], g["d"], np.array(g["gamma"], np.float32),
                      np.array(g["beta"], np.float32), g["eps"], out)
    assert np.max(np.abs(out - np.array(g["expected"], np.float32))) < g["tol"]


def test_layer_norm_normalize_reference_vectors():
    g = GOLD["layer_norm_normalize"]
    x = np.array(g["x"], np.float32)
    out = np.empty(8, np.float32)
    L().xo_layer_norm_normalize(x, g["rows"], g["d"], g["eps"], out)
    assert np.max(np.abs(out - np.array(g["expected"], np.float32))) < g["tol"]


def test_layer_norm_constant_row_gives_beta():
    x = np.full(64, 3.25, np.float32)
    gamma = np.linspace(0.5, 2, 64).astype(np.float32)
    beta = np.linspace(-1, 1, 64).astype(np.float32)
    out = np.empty(64, np.float32)
    L().xo_layer_norm(x, 1, 64, gamma, beta, 1e-5, out)
    assert np.array_equal(out, beta)


def test_rmsnorm_reference_unit_and_closed_form():
    # rmsnorm_unit (npu-gemma/src/lib.rs:83-91)
    x = np.array([3.0, -3.0, 3.0, -3.0], np.float32)
    out = np.empty(4, np.float32)
    L().xo_rmsnorm(x, 4, np.zeros(4, np.float32), 1e-6, out)
    assert np.all(np.abs(np.abs(out) - 1.0) < 1e-3)
    # closed form: +-c with weight w -> sign * c / sqrt(c^2 + eps) * (1 + w)
    w = np.array([0.5, -0.25, 0.0, 1.0], np.float32)
    L().xo_rmsnorm(x, 4, w, 1e-6, out)
    want = np.sign(x) * 3.0 / math.sqrt(9.0 + 1e-6) * (1.0 + w)
    assert np.allclose(out, want, rtol=1e-6)


def test_rope_reference_vectors():
    g = GOLD["rope"]
    x = np.array(g["x"], np.float32)
    out = np.empty_like(x)
    L().xo_rope(x, g["rows"], g["n_heads"], g["head_dim"], np.array(g["cos"], np.float32),
                np.array(g["sin"], np.float32), out)
    assert np.max(np.abs(out - np.array(g["expected"], np.float32))) < g["tol"]


def test_erf_as_published_bound_and_symmetry():
    xs = np.linspace(-6, 6, 4001)
    for v in xs[::7]:
        a = L().xo_erf_as(float(v))
        assert abs(a - math.erf(float(v))) < 5e-7   # A&S 1.5e-7 + f32 evaluation
        assert a == -L().xo_erf_as(float(-v)) or v == 0


def test_gelu_erf_properties():
    assert L().xo_gelu_erf(0.0) == 0.0
    for v in np.linspace(-5, 5, 101):
        v = float(np.float32(v))
        g, gm = L().xo_gelu_erf(v), L().xo_gelu_erf(-v)
        assert abs((g - gm) - v) < 1e-5          # gelu(x) - gelu(-x) = x
        exact = 0.5 * v * (1 + math.erf(v / math.sqrt(2)))
        assert abs(g - exact) < 2e-6 * max(1.0, abs(v))


def test_gelu_tanh_reference_and_bound():
    # geglu_shapes: gelu(0) = 0 (npu-gemma/src/lib.rs:93-99)
    assert L().xo_gelu_tanh(0.0) == 0.0
    for v in np.linspace(-6, 6, 241):
        v = float(v)
        exact = 0.5 * v * (1 + math.erf(v / math.sqrt(2)))
        assert abs(L().xo_gelu_tanh(v) - exact) < 1e-3


def test_fast_exp_accuracy_reference_bound():
    # test_fast_exp_accuracy (npu-asr-host/src/lib.rs:847-859)
    xs = np.arange(-60.0, 0.0, 0.013)
    worst = max(abs(L().xo_fast_exp_nonpos(float(v)) - math.exp(v)) / math.exp(v) for v in xs)
    assert worst < 5e-4


# ------------------------------------------------------------- quant ----

def test_quant_i8_rounding_half_away_and_clamp():
    q = L().xo_quant_i8
    assert q(0.5, 1.0) == 1 and q(-0.5, 1.0) == -1      # Rust round(), not half-even
    assert q(2.5, 1.0) == 3 and q(-2.5, 1.0) == -3
    assert q(1.49, 1.0) == 1 and q(200.0, 1.0) == 127 and q(-200.0, 1.0) == -127


def test_quant_rows_equals_reference_column_layout():
    rng = np.random.default_rng(0)
    w_kn = rng.standard_normal((48, 40)).astype(np.float32) * 0.02
    w_kn[:, 7] = 0.0                               # all-zero column -> scale 1.0
    qk = np.empty((48, 40), np.int8)
    sk = np.empty(40, np.float32)
    L().xo_quant_cols_i8(w_kn, 48, 40, qk, sk)
    qr, sr = O.quant_rows_i8(w_kn.T.copy())
    assert np.array_equal(qr, qk.T) and np.array_equal(sr, sk)
    assert sk[7] == 1.0 and not qk[:, 7].any()
    # the max-magnitude element of each column lands exactly on +-127
    idx = np.argmax(np.abs(w_kn), axis=0)
    cols = [c for c in range(40) if c != 7]
    assert all(abs(int(qk[idx[c], c])) == 127 for c in cols)


def test_gemv_i8_matches_reference_kn_loop_bitwise():
    rng = np.random.default_rng(1)
    k, n, b = 96, 80, 3
    w_kn = rng.standard_normal((k, n)).astype(np.float32)
    qk = np.empty((k, n), np.int8)
    s = np.empty(n, np.float32)
    L().xo_quant_cols_i8(w_kn, k, n, qk, s)
    x = rng.standard_normal((b, k)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    y_kn = np.empty((b, n), np.float32)
    L().xo_lin_fwd_i8_kn(x, b, k, n, qk, s, O.ptr(bias), y_kn)
    y_mk = O.gemv_i8(x, qk.T.copy(), s, bias)
    assert np.array_equal(y_kn.view(np.uint32), y_mk.view(np.uint32))


@pytest.mark.parametrize("m,k", [(1, 7), (8, 64), (37, 96), (97, 200), (257, 1152)])
def test_gemv_i8_rowblocked_equals_scalar_bitwise(m, k):
    """The decoder models' GEMV (row blocks of 8, k-major, vector code) is
    the scalar k-ordered loop bit for bit, ragged row counts included."""
    rng = np.random.default_rng(m * 1000 + k)
    q = rng.integers(-127, 128, (m, k)).astype(np.int8)
    s = rng.uniform(0.001, 0.02, m).astype(np.float32)
    bias = rng.standard_normal(m).astype(np.float32)
    x = rng.standard_normal((2, k)).astype(np.float32)
    want = O.gemv_i8(x, q, s, bias)
    got = np.empty((2, m), np.float32)
    L().xo_gemv_i8_rowblocked(x, 2, k, m, q, s, O.ptr(bias), got)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_gemv_i8_integer_inputs_exact():
    rng = np.random.default_rng(2)
    q = rng.integers(-127, 128, (33, 64)).astype(np.int8)
    x = rng.integers(-8, 9, (2, 64)).astype(np.float32)
    s = np.ones(33, np.float32)
    want = x.astype(np.int64) @ q.astype(np.int64).T
    assert np.array_equal(O.gemv_i8(x, q, s), want.astype(np.float32))


def test_w8a8_int32_bruteforce_and_dequant_order():
    rng = np.random.default_rng(3)
    a = rng.integers(-127, 128, (5, 64)).astype(np.int8)
    w = rng.integers(-127, 128, (24, 64)).astype(np.int8)
    acc = np.empty((5, 24), np.int32)
    L().xo_gemm_i8i8_i32(a, 5, 64, w, 24, acc)
    assert np.array_equal(acc, a.astype(np.int64) @ w.astype(np.int64).T)
    # dequant order (acc * scale_a) * ws + bias: differs from acc * (scale_a * ws)
    sa = np.float32(0.0123)
    ws = rng.uniform(0.001, 0.02, 24).astype(np.float32)
    bias = rng.standard_normal(24).astype(np.float32)
    out = np.empty((5, 24), np.float32)
    L().xo_dequant_epi(acc, 5, 24, sa, ws, O.ptr(bias), out)
    want = (acc.astype(np.float32) * sa) * ws[None, :] + bias[None, :]
    other = acc.astype(np.float32) * (sa * ws[None, :]) + bias[None, :]
    assert np.array_equal(out, want.astype(np.float32))
    assert not np.array_equal(want.astype(np.float32), other.astype(np.float32))


def test_quant_rows_elf_is_numpy_qrow():
    """gen_decode.py:158-165 qrow is numpy code: its own operations (float32
    max / 127, np.round half-to-even, clip), then the scale through the
    reference's bf16 RNE (npu-xrt/src/lib.rs:809-817, pinned above) --
    equal bit for bit; exact ties decide the rounding mode."""
    rng = np.random.default_rng(31)
    w = (rng.standard_normal((40, 96)) * 0.02).astype(np.float32)
    w[3] = 0.0
    # exact ties: amax 127 -> scale 1.0 (row 5), values k + 0.5
    w[5, :8] = [127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5]
    q, s = O.quant_rows_i8_elf(w)
    m = w.astype(np.float32)
    s32 = (np.abs(m).max(axis=1) / 127.0).astype(np.float32)
    s32 = np.where(s32 > 0, s32, np.float32(1.0)).astype(np.float32)
    want_q = np.clip(np.round(m / s32[:, None]), -127, 127).astype(np.int8)
    assert np.array_equal(q, want_q)
    assert np.array_equal(s, O.bf16_to_f32(O.bf16_bits(s32)))
    assert q[5, :8].tolist() == [127, 0, 2, 2, 0, -2, -2, 4]      # half to even
    lin_q, _ = O.quant_rows_i8(w)
    assert lin_q[5, :8].tolist() == [127, 1, 2, 3, -1, -2, -3, 4]  # Lin: half away (differs)
    assert s[3] == 1.0 and not q[3].any()


# -------------------------------------------------------------- int4 ----

def test_i4_quant_nibbles_and_scales_closed_form():
    """Lin::load int4 (opt125m_decode.rs:63-79): scale amax/7 (1.0 for an
    all-zero column), round half away from zero, clamp +-7, two's-complement
    nibbles with the even column low.  Checked against hand-computed codes."""
    # column 0: amax 7 -> scale 1: values land on their own integers (and ties)
    # column 1: all zero -> scale 1.0, code 0
    # column 2: amax 14 -> scale 2: 3 -> 1.5 -> 2 (half away), -3 -> -2
    # column 3: amax 0.7 -> scale 0.1
    w_kn = np.array([[7.0, 0.0, 14.0, 0.7],
                     [-0.5, 0.0, 3.0, -0.7],
                     [2.5, 0.0, -3.0, 0.04],
                     [-7.0, 0.0, -14.0, -0.049]], np.float32)
    q, s = O.quant_cols_i4(w_kn)
    assert s.tolist() == [1.0, 1.0, 2.0, np.float32(0.7) / np.float32(7.0)]
    codes = O.unpack_i4(q)
    assert codes.tolist() == [[7, 0, 7, 7], [-1, 0, 2, -7], [3, 0, -2, 0], [-7, 0, -7, 0]]
    # raw nibbles: -1 -> 0xF, -7 -> 0x9, 7 -> 0x7 (even column in the low nibble)
    assert int(q[1, 0]) == (0x0 << 4) | 0xF and int(q[3, 0]) == (0x0 << 4) | 0x9
    assert int(q[0, 1]) == (0x7 << 4) | 0x7


def test_i4_sign_extension_all_nibbles():
    # ((v ^ 8) - 8) of every nibble, through the GEMV with one-hot x
    packed = np.array([[(v << 4) | v for v in range(16)]], np.uint8).reshape(1, 16)
    want = [0, 1, 2, 3, 4, 5, 6, 7, -8, -7, -6, -5, -4, -3, -2, -1]
    assert O.unpack_i4(packed)[0, 0::2].tolist() == want
    eye = np.eye(32, dtype=np.float32)
    y = O.gemv_i4(eye, packed, np.ones(1, np.float32))[:, 0]
    assert y[0::2].tolist() == want and y[1::2].tolist() == want


def test_i4_rows_equal_reference_column_layout_and_loop_bitwise():
    """[M, K] packing along K is the reference's [K, N/2] packing transposed:
    same codes and scales; the [M, K] GEMV equals the reference's k-outer
    [K, N] loop (opt125m_decode.rs:83-105) bit for bit."""
    rng = np.random.default_rng(11)
    k, n, b = 96, 80, 3
    w_kn = (rng.standard_normal((k, n)) * 0.02).astype(np.float32)
    w_kn[:, 5] = 0.0
    qk, sk = O.quant_cols_i4(w_kn)
    qr, sr = O.quant_rows_i4(w_kn.T.copy())
    assert np.array_equal(sr, sk) and sk[5] == 1.0
    assert np.array_equal(O.unpack_i4(qr), O.unpack_i4(qk).T)
    x = rng.standard_normal((b, k)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    y_kn = O.lin_fwd_i4_kn(x, qk, sk, bias)
    y_mk = O.gemv_i4(x, qr, sr, bias)
    assert np.array_equal(y_kn.view(np.uint32), y_mk.view(np.uint32))


def test_i4_gemv_integer_inputs_exact():
    rng = np.random.default_rng(12)
    codes = rng.integers(-7, 8, (33, 64)).astype(np.int64)
    nib = (codes & 0xF).astype(np.uint8)
    packed = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    x = rng.integers(-8, 9, (2, 64)).astype(np.float32)
    want = x.astype(np.int64) @ codes.T
    assert np.array_equal(O.gemv_i4(x, packed, np.ones(33, np.float32)), want.astype(np.float32))
    # the scale multiplies after the sum
    s = rng.uniform(0.001, 0.02, 33).astype(np.float32)
    got = O.gemv_i4(x, packed, s)
    assert np.array_equal(got, (want.astype(np.float32) * s[None, :]).astype(np.float32))


def test_fast_sigmoid_accuracy_and_symmetry():
    """fast_sigmoid (ctx2.rs:1338-1348) on fast_exp_nonpos: within the
    reference's own fast_exp bound (5e-4 relative, npu-asr-host/src/lib.rs:
    847-859) of the exact logistic, and s(x) + s(-x) = 1."""
    for v in np.linspace(-30, 30, 601):
        v = float(np.float32(v))
        got = O.lib().xo_fast_sigmoid(v)
        exact = 1.0 / (1.0 + math.exp(-v))
        assert abs(got - exact) <= 5e-4 * exact
        assert abs(got + O.lib().xo_fast_sigmoid(-v) - 1.0) < 1e-6


def test_w8a8_epilogues_none_bias_silu():
    """dequant_epi's three epilogues over one product: Bias = None + bias
    exactly (one fp32 add), SiluBias = z * sigmoid(z) of the Bias output."""
    rng = np.random.default_rng(9)
    a = rng.standard_normal((6, 64)).astype(np.float32)
    wf = (rng.standard_normal((40, 64)) * 0.02).astype(np.float32)
    q, s = O.quant_rows_i8(wf)
    bias = rng.standard_normal(40).astype(np.float32)
    y0, sa0 = O.w8a8_linear(a, q, s, bias, O.EPI_NONE)
    y1, sa1 = O.w8a8_linear(a, q, s, bias, O.EPI_BIAS)
    y2, _ = O.w8a8_linear(a, q, s, bias, O.EPI_SILU_BIAS)
    assert sa0 == sa1 == np.float32(np.max(np.abs(a))) / np.float32(127.0)
    assert np.array_equal(y1, (y0 + bias[None, :]).astype(np.float32))
    z = y1.astype(np.float64)
    assert np.allclose(y2, z / (1.0 + np.exp(-z)), rtol=5e-4, atol=1e-7)
    # the product itself is the brute-force integer one
    aq = O.round_half_away_i8(a / np.float32(sa0))
    acc = aq.astype(np.int64) @ q.astype(np.int64).T
    assert np.array_equal(y0, ((acc.astype(np.float32) * np.float32(sa0)) * s[None, :]).astype(np.float32))


def test_quant_scale_zero_guard():
    assert L().xo_quant_scale(np.zeros(16, np.float32), 16) == 1.0
    assert L().xo_quant_scale(np.array([0.0, -2.54, 1.0], np.float32), 3) == np.float32(2.54) / np.float32(127.0)


# ------------------------------------------------------------- bfp16 ----

def test_bfp16_exact_on_representable_blocks():
    rng = np.random.default_rng(4)
    # blocks whose values are integer multiples of their quantum with |q| <= 127
    m, k = 6, 64
    e = rng.integers(-10, 10, (m, k // 8))
    q = rng.integers(-127, 128, (m, k))
    q[:, ::8] = np.where(rng.random((m, k // 8)) < 0.5, 127, 64)  # block max sets exponent
    w = (q * np.ldexp(1.0, np.repeat(e, 8, axis=1) - 6)).astype(np.float32)
    mant, exps = O.bfp16_encode(w)
    back = O.bfp16_decode(mant, exps)
    assert np.array_equal(back, w)
    assert np.array_equal(exps.astype(np.int64) - 127, e)


def test_bfp16_half_even_ties():
    """Exact half-quantum ties round to even (golden_ffn_gemm.py:47 uses
    numpy's round): [64, 2.5, -2.5, 3.5, 0 ...] has e = 6 and quantum 1, so it
    encodes to [64, 2, -2, 4, 0 ...] with exponent byte 133; a half-away
    encoder would give [64, 3, -3, 4].  A second block checks +-0.5 -> 0 and
    1.5 -> 2 under a negative block maximum."""
    w = np.zeros((2, 16), np.float32)
    w[0, :4] = [64.0, 2.5, -2.5, 3.5]
    w[1, 8:12] = [-64.0, 0.5, 1.5, -0.5]
    mant, exps = O.bfp16_encode(w)
    assert list(mant[0, :8]) == [64, 2, -2, 4, 0, 0, 0, 0]
    assert list(mant[1, 8:16]) == [-64, 0, 2, 0, 0, 0, 0, 0]
    assert exps[0, 0] == 133 and exps[1, 1] == 133


def test_bfp16_error_bound_and_saturation():
    rng = np.random.default_rng(5)
    w = rng.standard_normal((16, 128)).astype(np.float32)
    mant, exps = O.bfp16_encode(w)
    back = O.bfp16_decode(mant, exps)
    wb = O.bf16_to_f32(O.bf16_bits(w)).reshape(w.shape)
    quantum = np.repeat(np.ldexp(1.0, exps.astype(np.int64) - 127 - 6), 8, axis=1)
    # within half a quantum, except the saturated +128 case (one quantum)
    err = np.abs(back - wb)
    assert np.all(err <= quantum * 1.0 + 1e-30)
    sat = mant == 127
    assert np.all(err[~sat] <= quantum[~sat] * 0.5 + 1e-30)
    # block max magnitude lies in [64, 128) quanta -> mantissa of the max is 64..127 in size
    blk = np.abs(wb).reshape(16, 16, 8).max(axis=2)
    qmax = np.abs(mant.astype(np.int64)).reshape(16, 16, 8).max(axis=2)
    assert np.all((qmax >= 64) & (qmax <= 128)) and np.all(blk > 0)


# -------------------------------------------------- fused norm + gemv ----

def _selftest_inputs():
    """norm_gemv_probe.rs:79-83 deterministic 8x4 inputs (W as [K,N])."""
    k, n = 8, 4
    x = np.array([((i * 7 % 11) - 5.0) * 0.3 for i in range(k)])
    gamma = np.array([1.0 + 0.1 * i for i in range(k)])
    beta = np.array([0.05 * (i - 3.0) for i in range(k)])
    bias = np.array([0.2 * (i - 1.0) for i in range(n)])
    w = np.array([[(((kk * 5 + nn * 3) % 13) - 6.0) * 0.1 for nn in range(n)] for kk in range(k)])
    return x, gamma, beta, bias, w


def test_fold_identity_reference_selftest():
    x, gamma, beta, bias, w_kn = _selftest_inputs()
    f = lambda a: np.ascontiguousarray(a, np.float32)
    w_mk = f(w_kn.T)
    # direct: LN(x) then W, in f64 (the probe's golden)
    mean, var = x.mean(), ((x - x.mean()) ** 2).mean()
    xn = (x - mean) / math.sqrt(var + 1e-5) * gamma + beta
    direct = w_kn.T @ xn + bias
    # oracle norm + gemv (f32)
    h = np.empty(8, np.float32)
    L().xo_norm_row(f(x), 8, 1, O.ptr(f(gamma)), O.ptr(f(beta)), 1e-5, h)
    y = np.array([float(np.dot(w_mk[r].astype(np.float64), h)) for r in range(4)]) + bias
    assert np.max(np.abs(y - direct)) < 1e-5
    # oracle fold: W'' and bias'; inv_std * ((x - mean) . W'') + bias'
    wf = np.empty_like(w_mk)
    bf = np.empty(4, np.float32)
    L().xo_fold_weight(w_mk, 4, 8, f(gamma), O.ptr(f(beta)), O.ptr(f(bias)), wf, bf)
    folded = (wf.astype(np.float64) @ (x - mean)) / math.sqrt(var + 1e-5) + bf
    assert np.max(np.abs(folded - direct)) < 1e-5


# --------------------------------------------------------- attention ----

def test_attend_one_reference_mha_vectors():
    g = GOLD["mha_no_round"]
    t, H, hd = g["t"], g["n_heads"], g["head_dim"]
    q = np.array(g["q"], np.float32).reshape(t, H * hd)
    k = np.array(g["k"], np.float32)
    v = np.array(g["v"], np.float32)
    exp = np.array(g["expected"], np.float32).reshape(t, H * hd)
    for i in range(t):  # unmasked mha row i = attend_one(q_i, K, V, t)
        ctx = np.empty(H * hd, np.float32)
        L().xo_attend_one(np.ascontiguousarray(q[i]), k, v, t, H, hd, ctx)
        assert np.max(np.abs(ctx - exp[i])) < g["tol"]


def _rand_cache(rng, b, hkv, ctx, hd):
    kf = rng.standard_normal((b, hkv, ctx, hd)).astype(np.float32)
    vf = rng.standard_normal((b, hkv, ctx, hd)).astype(np.float32)
    return O.bf16_bits(kf), O.bf16_bits(vf)


def test_attn_decode_closed_forms():
    rng = np.random.default_rng(6)
    kc, vc = _rand_cache(rng, 1, 1, 16, 64)
    q = rng.standard_normal((1, 1, 64)).astype(np.float32)
    # one key -> the value row
    out = O.attn_decode(q, kc, vc, [1], 0.125)
    assert np.array_equal(out[0, 0], O.bf16_to_f32(vc[0, 0, 0]))
    # identical keys -> mean of the values
    kc2 = np.repeat(kc[:, :, :1], 16, axis=2)
    out = O.attn_decode(q, kc2, vc, [10], 0.125)
    want = O.bf16_to_f32(vc[0, 0, :10]).astype(np.float64).mean(axis=0)
    assert np.allclose(out[0, 0], want, rtol=1e-5, atol=1e-6)


def test_attn_decode_matches_attend_one_and_online():
    rng = np.random.default_rng(7)
    H, hd, S = 4, 64, 37
    kc, vc = _rand_cache(rng, 1, H, S, hd)
    q = rng.standard_normal((1, H, hd)).astype(np.float32)
    out = O.attn_decode(q, kc, vc, [S], 1.0 / math.sqrt(hd))
    # attend_one on [S, H*hd] rows of the same (bf16-valued) data
    kf = O.bf16_to_f32(kc[0]).transpose(1, 0, 2).reshape(S, H * hd).copy()
    vf = O.bf16_to_f32(vc[0]).transpose(1, 0, 2).reshape(S, H * hd).copy()
    ctx = np.empty(H * hd, np.float32)
    L().xo_attend_one(np.ascontiguousarray(q.reshape(-1)), kf, vf, S, H, hd, ctx)
    assert np.allclose(out.reshape(-1), ctx, rtol=1e-6, atol=1e-7)
    for h in range(H):
        on = np.empty(hd, np.float32)
        L().xo_attn_online(np.ascontiguousarray(q[0, h]), np.ascontiguousarray(kc[0, h]),
                           np.ascontiguousarray(vc[0, h]), S, hd, 1.0 / math.sqrt(hd), on)
        assert np.allclose(on, out[0, h], rtol=1e-5, atol=1e-6)


def test_attn_decode_gqa_mapping_and_lengths():
    rng = np.random.default_rng(8)
    b, hq, hkv, hd, ctx = 3, 4, 1, 64, 50
    kc, vc = _rand_cache(rng, b, hkv, ctx, hd)
    q = rng.standard_normal((b, hq, hd)).astype(np.float32)
    lens = np.array([50, 7, 23], np.int32)
    out = O.attn_decode(q, kc, vc, lens, 0.125)
    for bi in range(b):
        for h in range(hq):  # each q head against the single kv head, own length
            o1 = O.attn_decode(q[bi:bi + 1, h:h + 1].copy(), kc[bi:bi + 1].copy(),
                               vc[bi:bi + 1].copy(), lens[bi:bi + 1], 0.125)
            assert np.array_equal(o1[0, 0], out[bi, h])
    # positions beyond the length are ignored
    kc2 = kc.copy()
    kc2[1, 0, 7:] = 0x7F80  # +inf keys past the length
    assert np.array_equal(O.attn_decode(q, kc2, vc, lens, 0.125)[1], out[1])


# ---------------------------------------------------------------- argmax --

def test_argmax_tie_rules():
    v = np.array([1.0, 3.0, 2.0, 3.0, 0.0], np.float32)
    assert L().xo_argmax_first(v, 5) == 1      # whisper.rs:749-757 (strict >)
    assert L().xo_argmax_last(v, 5) == 3       # Iterator::max_by: last of equal maxima


# ------------------------------------------------------------- synth ----

def test_synth_statistics_and_determinism():
    a = O.synth_fill(7, 1234, 0.0, 0.02, 400_000)
    b = O.synth_fill(7, 1234, 0.0, 0.02, 400_000)
    c = O.synth_fill(7, 1235, 0.0, 0.02, 400_000)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    assert abs(a.mean()) < 2e-4 and abs(a.std() - 0.02) < 2e-4
    one = O.synth_fill(3, 9, 1.0, 0.02, 200_000)
    assert abs(one.mean() - 1.0) < 2e-4
    # element i depends only on (seed, tensor, i)
    base = L().xo_synth_base(7, 1234)
    assert all(L().xo_synth_value(base, i, 0.0, 0.02) == a[i] for i in (0, 1, 99_999, 399_999))


# ---- int8 per-utterance cross K/V (whisper_decoder.rs:1186-1219,
# write_buf_i8 :1110-1134; kernel side gen_decode.py:263-282) ----

def test_cross_i8_quant_scale_rounding_and_layout():
    """Channel (h, d) scale = max_t |x| / 127; Rust round() is half away from
    zero (a half-even rint would give 2, -2, 0, -126 below); a zero channel
    gets scale 1 and zeros; NaN stores 0; output is head-major [H, T, hd]."""
    T, H, hd = 6, 2, 4
    rng = np.random.default_rng(3)
    x = rng.standard_normal((T, H * hd)).astype(np.float32)
    x[:, 0] = [2.5, -2.5, 0.5, -126.5, 127.0, 1.0]   # max 127: scale 1, inverse 1
    x[:, 1] = 0.0
    x[2, 5] = np.nan
    q, s = O.quant_cross_i8(x, H, hd)
    assert q.shape == (H, T, hd)
    assert s[0] == np.float32(1.0)
    assert list(q[0, :, 0]) == [3, -3, 1, -127, 127, 1]
    assert s[1] == 1.0 and not q[0, :, 1].any()
    assert q[1, 2, 1] == 0  # NaN
    for c in range(2, H * hd):
        h, d = divmod(c, hd)
        col = x[:, c].astype(np.float64)
        if c == 5:
            col = np.where(np.isnan(col), 0.0, col)
        amax = np.max(np.abs(col))
        assert s[c] == np.float32(np.float32(amax) / np.float32(127.0))
        qc = q[h, :, d].astype(np.float64)
        assert np.max(np.abs(qc)) == 127                      # the channel max maps to +-127
        ok = ~np.isnan(x[:, c])
        assert np.all(np.abs(qc[ok] * s[c] - col[ok]) <= s[c] * (0.5 + 1e-6))  # half a step


def test_cross_i8_attention_identities():
    """int8 K scores use q * s_k, int8 V outputs are scaled by s_v: against a
    float64 attention over the dequantised K / V, and the one-key closed form
    (the output is the key's value row)."""
    T, hd = 37, 64
    rng = np.random.default_rng(4)
    kf = rng.standard_normal((T, hd)).astype(np.float32)
    vf = rng.standard_normal((T, hd)).astype(np.float32) * 3
    k8, sk = O.quant_cross_i8(kf, 1, hd)
    v8, sv = O.quant_cross_i8(vf, 1, hd)
    k8, v8 = k8[0], v8[0]
    q = rng.standard_normal(hd).astype(np.float32)
    scale = 1.0 / 8.0
    kd = k8.astype(np.float64) * sk.astype(np.float64)
    vd = v8.astype(np.float64) * sv.astype(np.float64)
    sc = kd @ q.astype(np.float64) * scale
    p = np.exp(sc - sc.max())
    p /= p.sum()
    want = p @ vd
    got = O.head_attend_x8(q, scale, k8=k8, sk=sk, v8=v8, sv=sv)
    assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))
    one = O.head_attend_x8(q, scale, k8=k8[:1], sk=sk, v8=v8[:1], sv=sv)
    assert np.array_equal(one, (v8[0].astype(np.float32) * sv).astype(np.float32))
    # int8 K with bf16 V, and bf16 K with int8 V, equal the same algebra
    vb = O.bf16_bits(vf)
    got_k = O.head_attend_x8(q, scale, k8=k8, sk=sk, vb=vb)
    want_k = p @ O.bf16_to_f32(vb).astype(np.float64).reshape(T, hd)
    assert np.max(np.abs(got_k - want_k)) <= 1e-5 * np.max(np.abs(want_k))


def test_cross_i8_decoder_close_to_bf16_cross():
    """The oracle decoder with int8 cross K / V: logits within the
    quantisation's reach of the bf16-cross decoder (2 layers), and the flag
    acts at set_cross."""
    cfg = O.ModelConfig()
    vals = dict(family=1, n_layers=2, d_model=256, n_heads=4, n_kv_heads=4, head_dim=64, ffn=1024,
                vocab=1000, max_pos=448, max_ctx=64, wdtype=2, eps=1e-5, rope_theta=0.0, n_cross=100)
    for k, v in vals.items():
        setattr(cfg, k, v)
    a = O.OracleModel(cfg, 5, 1)
    b = O.OracleModel(cfg, 5, 1)
    a.set_cross(None)
    b.set_cross_i8(True, True)
    toks, pos = np.array([7], np.int32), np.array([0], np.int32)
    la0 = a.step(toks, pos)
    b.reset()
    b.set_cross(None)
    lb = b.step(toks, pos)
    rel = np.linalg.norm(lb - la0) / np.linalg.norm(la0)
    assert 0 < rel < 3e-2, rel
    a.close()
    b.close()
