"""GPU parity of the decode GEMV family against the CPU oracle.

BASELINE config 2 (isolated norm+GEMV): x bf16 ~N(0,1), LayerNorm gamma/beta
~N(1,0.1)/N(0,0.1), W int8 U[-127,127] with per-row scale U(0.001,0.02), a
bfp16 variant and a bf16 variant; shapes M x K in {3072x768, 768x3072,
6912x1152, 4096x4096, 14336x4096}; batch 1/4/8; int8-activation variant
bit-exact.  Tolerance (BASELINE): fp32-accumulated outputs within rel 1e-2 /
abs 1e-3; the GPU and the oracle share the same quantised weights, so the
observed difference is fp32 summation order only and the test also bounds
the relative L2 error at 1e-5.
"""
import numpy as np
import pytest

import oracle_lib as O

pytestmark = pytest.mark.gpu

SHAPES = [(3072, 768), (768, 3072), (6912, 1152), (4096, 4096), (14336, 4096)]


def close(got, want, rtol=1e-2, atol=1e-3, rel_l2=1e-5):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape
    err = np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30)
    assert np.allclose(got, want, rtol=rtol, atol=atol), "max abs diff %g" % np.max(np.abs(got - want))
    assert err <= rel_l2, "rel-L2 %g" % err


def config2_inputs(m, k, b, seed):
    rng = np.random.default_rng(seed)
    x = O.bf16_bits(rng.standard_normal((b, k)).astype(np.float32))
    gamma = rng.normal(1.0, 0.1, k).astype(np.float32)
    beta = rng.normal(0.0, 0.1, k).astype(np.float32)
    q = rng.integers(-127, 128, (m, k)).astype(np.int8)
    s = rng.uniform(0.001, 0.02, m).astype(np.float32)
    return x, gamma, beta, q, s


def oracle_ln(xbits, gamma, beta, eps=1e-5):
    return O.norm_rows(O.bf16_to_f32(xbits), 1, gamma, beta, eps)


@pytest.mark.parametrize("m,k", SHAPES)
@pytest.mark.parametrize("b", [1, 4, 8])
def test_norm_gemv_int8_config2(gpu, xe, m, k, b):
    dev, ctx = gpu
    print("[case] int8 LN+GEMV m=%d k=%d b=%d" % (m, k, b), flush=True)
    x, gamma, beta, q, s = config2_inputs(m, k, b, seed=m + k + b)
    w = ctx.register_weight_q8(q, s)
    ctx.set_norm(w, xe.Norm.Ln(gamma, beta, 1e-5))
    got = ctx.fused_norm_gemv(w, x)
    want = O.gemv_i8(oracle_ln(x, gamma, beta), q, s)
    w.free()
    close(got, want)


@pytest.mark.parametrize("m,k", SHAPES)
@pytest.mark.parametrize("b", [1, 4, 8])
def test_norm_gemv_bfp16_config2(gpu, xe, m, k, b):
    dev, ctx = gpu
    print("[case] bfp16 LN+GEMV m=%d k=%d b=%d" % (m, k, b), flush=True)
    rng = np.random.default_rng(m * 3 + k + b)
    x = O.bf16_bits(rng.standard_normal((b, k)).astype(np.float32))
    gamma = rng.normal(1.0, 0.1, k).astype(np.float32)
    beta = rng.normal(0.0, 0.1, k).astype(np.float32)
    wf = (rng.standard_normal((m, k)) * 0.02).astype(np.float32)
    mant, exps = O.bfp16_encode(wf)
    w = ctx.register_weight_bfp16(mant, exps)
    ctx.set_norm(w, xe.Norm.Ln(gamma, beta, 1e-5))
    got = ctx.fused_norm_gemv(w, x)
    want = O.gemv_bfp16(oracle_ln(x, gamma, beta), mant, exps)
    w.free()
    close(got, want)


@pytest.mark.parametrize("m,k", SHAPES)
@pytest.mark.parametrize("b", [1, 4, 8])
def test_norm_gemv_bf16_config2(gpu, xe, m, k, b):
    dev, ctx = gpu
    print("[case] bf16 LN+GEMV m=%d k=%d b=%d" % (m, k, b), flush=True)
    rng = np.random.default_rng(m * 5 + k + b)
    x = O.bf16_bits(rng.standard_normal((b, k)).astype(np.float32))
    gamma = rng.normal(1.0, 0.1, k).astype(np.float32)
    beta = rng.normal(0.0, 0.1, k).astype(np.float32)
    wbits = O.bf16_bits((rng.standard_normal((m, k)) * 0.02).astype(np.float32))
    w = ctx.register_weight_bf16(wbits)
    ctx.set_norm(w, xe.Norm.Ln(gamma, beta, 1e-5))
    got = ctx.fused_norm_gemv(w, x)
    want = O.gemv_bf16w(oracle_ln(x, gamma, beta), wbits)
    w.free()
    close(got, want)


def lcg_fill(n, seed):
    """ctx_decode.rs:722-730 lcg_fill: ((s >> 8) / u32::MAX) - 0.5."""
    out = np.empty(n, np.float32)
    s = seed
    for i in range(n):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = np.float32(np.float32(s >> 8) / np.float32(4294967295.0)) - np.float32(0.5)
    return out


@pytest.mark.parametrize("wdtype", ["i8", "bf16", "bfp16"])
def test_reference_gemv_parity_768x768(gpu, xe, wdtype):
    """gemv_parity_768x768 (ctx_decode.rs:735-776) with the reference's LCG
    inputs; W in the reference's [K, N] layout."""
    dev, ctx = gpu
    k = n = 768
    w_kn = lcg_fill(k * n, 0x12345678).reshape(k, n)
    x = lcg_fill(k, 0x9E3779B9)
    dt = {"i8": xe.XE_I8, "bf16": xe.XE_BF16, "bfp16": xe.XE_BFP16}[wdtype]
    w = ctx.register_weight(w_kn, dt, layout=xe.XE_LAYOUT_KN)
    got = ctx.gemv(w, x)
    w.free()
    w_mk = np.ascontiguousarray(w_kn.T)
    if wdtype == "i8":
        q, s = O.quant_rows_i8(w_mk)
        want = O.gemv_i8(x[None], q, s)[0]
    elif wdtype == "bf16":
        want = O.gemv_bf16w(x[None], O.bf16_bits(w_mk))[0]
    else:
        mant, exps = O.bfp16_encode(w_mk)
        want = O.gemv_bfp16(x[None], mant, exps)[0]
    close(got, want)
    # and the reference's own gate against the unquantised f64 product
    ref = x.astype(np.float64) @ w_kn.astype(np.float64)
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert rel <= 0.08


def test_reference_fused_ln_parity_768x768(gpu, xe):
    """fused_ln_parity_768x768 (ctx_decode.rs:782-830): LN(x; gamma, beta) @ W + bias."""
    dev, ctx = gpu
    k = n = 768
    w_kn = lcg_fill(k * n, 0x12345678).reshape(k, n)
    x = lcg_fill(k, 0x9E3779B9)
    gamma = lcg_fill(k, 0xABCD1234) + np.float32(1.0)
    beta = lcg_fill(k, 0x5555AAAA)
    bias = lcg_fill(n, 0x0F0FF0F0)
    w = ctx.register_fused(w_kn, xe.Norm.Ln(gamma, beta, 1e-5), xe.XE_I8,
                           layout=xe.XE_LAYOUT_KN, bias=bias)
    got = ctx.fused_norm_gemv(w, x)
    w.free()
    q, s = O.quant_rows_i8(np.ascontiguousarray(w_kn.T))
    want = O.gemv_i8(O.norm_rows(x[None], 1, gamma, beta, 1e-5), q, s, bias)[0]
    # lcg_fill's (s >> 8) / u32::MAX puts every value near -0.5, so y ~ 190 is
    # the residue of a large cancellation: fp32 order noise is ~5e-5 relative.
    close(got, want, rel_l2=1e-3)
    mean, var = x.astype(np.float64).mean(), x.astype(np.float64).var()
    xn = (x - mean) / np.sqrt(var + 1e-5) * gamma + beta
    ref = xn @ w_kn.astype(np.float64) + bias
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 0.08


@pytest.mark.parametrize("norm", ["rms", "rms1p", "none"])
def test_norm_variants(gpu, xe, norm):
    dev, ctx = gpu
    rng = np.random.default_rng(11)
    m, k, b = 1152, 1152, 2
    x = rng.standard_normal((b, k)).astype(np.float32) * 3
    g = rng.normal(0.0, 0.3, k).astype(np.float32)
    q = rng.integers(-127, 128, (m, k)).astype(np.int8)
    s = rng.uniform(0.001, 0.02, m).astype(np.float32)
    bias = rng.standard_normal(m).astype(np.float32)
    w = ctx.register_weight_q8(q, s, bias)
    kind = {"rms": xe.XE_NORM_RMS, "rms1p": xe.XE_NORM_RMS1P, "none": xe.XE_NORM_NONE}[norm]
    if kind != xe.XE_NORM_NONE:
        ctx.set_norm(w, xe.Norm(kind, g, None, 1e-6))
    got = ctx.fused_norm_gemv(w, x)
    w.free()
    h = O.norm_rows(x, kind, g if kind else None, None, 1e-6) if kind else x
    close(got, O.gemv_i8(h, q, s, bias))


@pytest.mark.parametrize("m,k", [(1, 16), (1000, 1152), (37, 4112), (513, 6912), (2048, 64)])
def test_ragged_shapes(gpu, xe, m, k):
    dev, ctx = gpu
    rng = np.random.default_rng(m + k)
    q = rng.integers(-127, 128, (m, k)).astype(np.int8)
    q[0] = 0                                   # an all-zero row
    s = rng.uniform(0.001, 0.02, m).astype(np.float32)
    x = rng.standard_normal((3, k)).astype(np.float32)
    w = ctx.register_weight_q8(q, s)
    got = ctx.gemv(w, x)
    w.free()
    close(got, O.gemv_i8(x, q, s))
    assert not got[:, 0].any()


def test_constant_input_layernorm(gpu, xe):
    """LN of a constant row is beta (variance 0 -> inv = 1/sqrt(eps))."""
    dev, ctx = gpu
    rng = np.random.default_rng(5)
    m, k = 256, 768
    q = rng.integers(-127, 128, (m, k)).astype(np.int8)
    s = rng.uniform(0.001, 0.02, m).astype(np.float32)
    gamma = rng.normal(1.0, 0.1, k).astype(np.float32)
    beta = rng.normal(0.0, 0.1, k).astype(np.float32)
    w = ctx.register_weight_q8(q, s)
    ctx.set_norm(w, xe.Norm.Ln(gamma, beta, 1e-5))
    got = ctx.fused_norm_gemv(w, np.full((1, k), 2.5, np.float32))
    w.free()
    close(got, O.gemv_i8(beta[None], q, s))


@pytest.mark.parametrize("b", [1, 3, 8, 9, 16, 40, 64, 200, 512])
def test_i8act_bit_exact(gpu, xe, b):
    """int8 x int8 -> i32, exact: the sdot4 GEMV up to 8 rows, the int8 MFMA
    GEMM beyond (ragged row and batch counts, K not a multiple of 64)."""
    dev, ctx = gpu
    rng = np.random.default_rng(b)
    for m, k in [(3072, 768), (768, 3072), (1000, 1152), (130, 1040)]:
        print("[case] i8act m=%d k=%d b=%d" % (m, k, b), flush=True)
        q = rng.integers(-127, 128, (m, k)).astype(np.int8)
        xq = rng.integers(-127, 128, (b, k)).astype(np.int8)
        w = ctx.register_weight_q8(q, np.ones(m, np.float32))
        got = ctx.gemv_i8act(w, xq)
        w.free()
        want = np.empty((b, m), np.int32)
        O.lib().xo_gemm_i8i8_i32(xq, b, k, q, m, want)
        assert np.array_equal(got, want)


@pytest.mark.parametrize("m,k", SHAPES)
@pytest.mark.parametrize("b", [1, 4, 8])
def test_i8act_config2_bit_exact(gpu, xe, m, k, b):
    """Config 2's int8-activation variant at every shape and batch: x and W
    int8 U[-127, 127], i32 outputs equal to the exact integer products."""
    dev, ctx = gpu
    print("[case] i8act config2 m=%d k=%d b=%d" % (m, k, b), flush=True)
    rng = np.random.default_rng(m + 3 * k + b)
    q = rng.integers(-127, 128, (m, k)).astype(np.int8)
    xq = rng.integers(-127, 128, (b, k)).astype(np.int8)
    w = ctx.register_weight_q8(q, rng.uniform(0.001, 0.02, m).astype(np.float32))
    got = ctx.gemv_i8act(w, xq)
    w.free()
    want = np.empty((b, m), np.int32)
    O.lib().xo_gemm_i8i8_i32(xq, b, k, q, m, want)
    assert np.array_equal(got, want)


def test_bfp16_encoder_half_even_ties(gpu, xe):
    """The product's bfp16 encoder rounds exact half-quantum ties to even
    (golden_ffn_gemm.py:47, numpy round): the block [64, 2.5, -2.5, 3.5,
    0 ...] has e = floor(log2 64) = 6, quantum 2^(e - 6) = 1, so it stores
    [64, 2, -2, 4, 0 ...] with exponent byte 6 + 127 = 133.  Read back through
    the GEMV with one-hot inputs (y = W[:, i])."""
    dev, ctx = gpu
    k = 16
    wf = np.zeros((2, k), np.float32)
    wf[0, :4] = [64.0, 2.5, -2.5, 3.5]
    wf[1, 8:12] = [-64.0, 0.5, 1.5, -0.5]  # quantum 1: 0, 2, -0
    w = ctx.register_weight(wf, xe.XE_BFP16)
    eye = np.eye(k, dtype=np.float32)
    got = np.vstack([ctx.gemv(w, eye[:8]), ctx.gemv(w, eye[8:])])  # row i: W[:, i]
    w.free()
    want = np.zeros((2, k), np.float32)
    want[0, :4] = [64, 2, -2, 4]
    want[1, 8:12] = [-64, 0, 2, 0]
    assert np.array_equal(np.asarray(got).T, want)


def test_w8a8_linear_bit_exact(gpu, xe):
    """forward_view_int8 (ctx2.rs:771-830): activation quant, i32 GEMM and the
    (acc * scale_a) * ws + bias dequant reproduce the oracle bit for bit."""
    dev, ctx = gpu
    rng = np.random.default_rng(21)
    m, k, b = 1536, 768, 4
    wf = (rng.standard_normal((m, k)) * 0.02).astype(np.float32)
    bias = rng.standard_normal(m).astype(np.float32)
    x = rng.standard_normal((b, k)).astype(np.float32)
    w = ctx.register_weight(wf, xe.XE_I8, bias=bias)
    got, sa = ctx.w8a8_linear(w, x)
    w.free()
    q, s = O.quant_rows_i8(wf)
    want = np.empty((b, m), np.float32)
    import ctypes as C
    osa = C.c_float()
    O.lib().xo_w8a8_linear(x, b, k, q, s, m, O.ptr(bias), want, C.byref(osa))
    assert sa == osa.value
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("b", [1, 8, 64, 512])
@pytest.mark.parametrize("epi", ["none", "bias", "silu_bias"])
def test_w8a8_device_epilogues_bit_exact(gpu, xe, b, epi):
    """xe_w8a8_linear_dev: amax, quant, product and the dequant epilogue
    (Epi::None / Bias / SiluBias, ctx2.rs:1386-1435) all on the device, equal
    to the oracle bit for bit (scale_a included), at the reference's
    Whisper-encoder shapes (K = 768, N in {768, 1536, 3072}, Mp <= 512)."""
    dev, ctx = gpu
    rng = np.random.default_rng(100 + b)
    m, k = {1: 3072, 8: 1536, 64: 768, 512: 1536}[b], 768
    print("[case] w8a8 dev m=%d k=%d b=%d epi=%s" % (m, k, b, epi), flush=True)
    wf = (rng.standard_normal((m, k)) * 0.02).astype(np.float32)
    bias = rng.standard_normal(m).astype(np.float32)
    x = (rng.standard_normal((b, k)) * 3.0).astype(np.float32)
    x[0, 5] = 0.0
    code = {"none": xe.XE_EPI_NONE, "bias": xe.XE_EPI_BIAS, "silu_bias": xe.XE_EPI_SILU_BIAS}[epi]
    w = ctx.register_weight(wf, xe.XE_I8, bias=bias)
    xb = xe.Buf.from_array(dev, x)
    yb = xe.Buf(dev, b * m * 4)
    sab = xe.Buf(dev, 4)
    ctx.w8a8_linear_dev(w, xb, b, code, yb, sab)
    ctx.synchronize()
    got = yb.read(np.float32, b * m).reshape(b, m)
    sa = sab.read(np.float32, 1)[0]
    for bb in (xb, yb, sab):
        bb.free()
    w.free()
    q, s = O.quant_rows_i8(wf)
    want, osa = O.w8a8_linear(x, q, s, bias, {"none": O.EPI_NONE, "bias": O.EPI_BIAS,
                                               "silu_bias": O.EPI_SILU_BIAS}[epi])
    assert sa == np.float32(osa)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_w8a8_all_zero_activations(gpu, xe):
    """quant_scale's guard: an all-zero tensor gives scale_a = 1.0 and the
    bias alone (ctx2.rs:1376)."""
    dev, ctx = gpu
    m, k, b = 256, 768, 16
    rng = np.random.default_rng(5)
    wf = (rng.standard_normal((m, k)) * 0.02).astype(np.float32)
    bias = rng.standard_normal(m).astype(np.float32)
    w = ctx.register_weight(wf, xe.XE_I8, bias=bias)
    got, sa = ctx.w8a8_linear(w, np.zeros((b, k), np.float32))
    w.free()
    assert sa == 1.0
    assert np.array_equal(got, np.broadcast_to(bias, (b, m)))


def test_registration_rejects_bad_k(gpu, xe):
    dev, ctx = gpu
    with pytest.raises(xe.XdnaError, match="multiple of 16"):
        ctx.register_weight_q8(np.zeros((4, 20), np.int8), np.ones(4, np.float32))


# ---- more than 8 rows: the MFMA GEMM behind the same op-layer entry ----

@pytest.mark.parametrize("m,k", [(6912, 1152), (1152, 6912), (3072, 768)])
@pytest.mark.parametrize("b", [16, 64, 200])
def test_norm_gemm_int8_batched(gpu, xe, m, k, b):
    """xe_fused_norm_gemv at 16..200 rows (MFMA GEMM, bf16 three-part split
    of the fp32 activations, fp32 accumulate) against the oracle GEMV."""
    dev, ctx = gpu
    print("[case] int8 LN+GEMM m=%d k=%d b=%d" % (m, k, b), flush=True)
    x, gamma, beta, q, s = config2_inputs(m, k, b, seed=m + k + b)
    w = ctx.register_weight_q8(q, s)
    ctx.set_norm(w, xe.Norm.Ln(gamma, beta, 1e-5))
    got = ctx.fused_norm_gemv(w, x)
    want = O.gemv_i8(oracle_ln(x, gamma, beta), q, s)
    w.free()
    err = np.linalg.norm(got - want) / np.linalg.norm(want)
    print("[gemm] m=%d k=%d b=%d rel-L2 %.3g max abs %.3g" % (m, k, b, err,
                                                            np.max(np.abs(got - want))), flush=True)
    close(got, want)


# The decoder's b = 64 projection shapes, every weight type: together they
# take each tile height of the K-sliced kernel (16, 32 and 64 rows), its
# split-K tail (QKV, O, down) and the unsplit path (gate/up), plus the
# wide-output kernel gemm_kernel: a 65536-row output (one row block a wave)
# and 262144 rows or more (the Gemma lm-head's width, here with a short K:
# four row blocks a wave), also ragged (rows past a 256-row tile, a last K
# step of 16).
GEMM_SHAPES = [(1536, 1152), (1152, 1024), (13824, 1152), (1152, 6912), (65536, 1152),
               (1000, 1040), (72, 48),  # ragged: K % 32 == 16, rows not a tile multiple
               (262144, 64), (262208, 80)]


@pytest.mark.parametrize("m,k", GEMM_SHAPES)
@pytest.mark.parametrize("wd", ["i8", "i4", "bf16", "bfp16"])
def test_gemm_b64_decoder_shapes(gpu, xe, m, k, wd):
    """64 streams through the MFMA GEMM against the oracle's GEMV of the same
    stored weights (fp32 activations, fp32 accumulation)."""
    dev, ctx = gpu
    b = 64
    print("[case] GEMM %s m=%d k=%d b=%d" % (wd, m, k, b), flush=True)
    rng = np.random.default_rng(m + 7 * k + len(wd))
    x = rng.standard_normal((b, k)).astype(np.float32)
    if wd == "i8":
        q = rng.integers(-127, 128, (m, k)).astype(np.int8)
        s = rng.uniform(0.001, 0.02, m).astype(np.float32)
        w = ctx.register_weight_q8(q, s)
        want = O.gemv_i8(x, q, s)
    elif wd == "i4":
        w_kn = (rng.standard_normal((k, m)) * 0.02).astype(np.float32)
        qk, s = O.quant_cols_i4(w_kn)
        w = ctx.register_weight_q4_kn(qk, s, None)
        want = O.lin_fwd_i4_kn(x, qk, s, None)
    elif wd == "bf16":
        wbits = O.bf16_bits((rng.standard_normal((m, k)) * 0.02).astype(np.float32))
        w = ctx.register_weight_bf16(wbits)
        want = O.gemv_bf16w(x, wbits)
    else:
        mant, exps = O.bfp16_encode((rng.standard_normal((m, k)) * 0.02).astype(np.float32))
        w = ctx.register_weight_bfp16(mant, exps)
        want = O.gemv_bfp16(x, mant, exps)
    got = ctx.gemv(w, x)
    w.free()
    close(got, want)


# ---- int4 weights (Lin int4 branch, opt125m_decode.rs:63-105) ----

@pytest.mark.parametrize("m,k", [(768, 768), (3072, 768), (768, 3072), (6912, 1152)])
@pytest.mark.parametrize("b", [1, 4, 8, 16])
def test_gemv_int4_against_reference_loop(gpu, xe, m, k, b):
    """OPT's int4 linear: weights quantised by the reference's Lin::load int4
    rule in its own [K, N/2] packing, registered as is, and the output
    compared with the reference's k-outer Lin::fwd int4 loop (bias added);
    b = 16 runs the MFMA GEMM path."""
    dev, ctx = gpu
    print("[case] int4 GEMV m=%d k=%d b=%d" % (m, k, b), flush=True)
    rng = np.random.default_rng(m + 3 * k + b)
    w_kn = (rng.standard_normal((k, m)) * 0.02).astype(np.float32)
    bias = rng.normal(0.0, 0.1, m).astype(np.float32)
    x = rng.standard_normal((b, k)).astype(np.float32)
    qk, s = O.quant_cols_i4(w_kn)
    w = ctx.register_weight_q4_kn(qk, s, bias)
    got = ctx.gemv(w, x)
    w.free()
    want = O.lin_fwd_i4_kn(x, qk, s, bias)
    close(got, want)


def test_gemv_int4_fp32_registration_and_fused_ln(gpu, xe):
    """xe_register_fused with XE_I4 quantises on the host like Lin::load int4
    (codes equal the oracle's [M, K] packing) and applies the LN prologue."""
    dev, ctx = gpu
    m, k, b = 1152, 1152, 2
    rng = np.random.default_rng(77)
    wf = (rng.standard_normal((m, k)) * 0.02).astype(np.float32)
    gamma = rng.normal(1.0, 0.1, k).astype(np.float32)
    beta = rng.normal(0.0, 0.1, k).astype(np.float32)
    x = rng.standard_normal((b, k)).astype(np.float32)
    w = ctx.register_fused(wf, xe.Norm.Ln(gamma, beta, 1e-5), xe.XE_I4)
    got = ctx.fused_norm_gemv(w, x)
    w.free()
    q, s = O.quant_rows_i4(wf)
    want = O.gemv_i4(O.norm_rows(x, 1, gamma, beta, 1e-5), q, s)
    close(got, want)


@pytest.mark.parametrize("rule", ["lin", "elf"])
def test_int8_quant_rules(gpu, xe, rule):
    """xe_register_weight_q8_rule: Lin::load's rule (half away, fp32 scale)
    or the fused ELF's qrow (half even, bf16 scale, gen_decode.py:158-165);
    the stored codes and scales are the oracle's, and the GEMV with bias
    matches the oracle's on them."""
    dev, ctx = gpu
    rng = np.random.default_rng(44)
    m, k = 2304, 768
    wf = (rng.standard_normal((m, k)) * 0.02).astype(np.float32)
    wf[7, :4] = [0.5, 1.5, 2.5, 127.0]  # exact ties at scale 1.0
    bias = rng.normal(0.0, 0.1, m).astype(np.float32)
    x = rng.standard_normal((2, k)).astype(np.float32)
    code = xe.XE_Q8_LIN if rule == "lin" else xe.XE_Q8_ELF
    w = ctx.register_weight_q8_rule(wf, code, bias=bias)
    got = ctx.gemv(w, x)
    w.free()
    q, s = O.quant_rows_i8(wf) if rule == "lin" else O.quant_rows_i8_elf(wf)
    close(got, O.gemv_i8(x, q, s, bias))
