"""GPU decode backends against the oracle decoder (configs 1, 4, 5).

Bars:
  * synthetic int8 weights produced on the GPU equal the oracle's bit for bit
    (q and per-row scale), including the fused QKV rows and the interleaved
    Gemma gate/up rows;
  * greedy token streams identical to the oracle on the same seeded weights
    and prompts; a stream may part only at an fp32 tie, and is then replayed
    by the oracle to its end (tests/parity_util.py greedy_identity);
  * logits within rel 1e-2 / abs 1e-3 of the oracle's (fp32 accumulate).
Tiny configs of every family and weight format run to many steps; the real
OPT-125m and Gemma-3-1B shapes run shorter streams the oracle finishes in
seconds.  The bench's own plans (max_ctx 4096, long prompts) are covered in
tests/test_long_gpu.py.
"""
import os

import numpy as np
import pytest

import oracle_lib as O
from parity_util import compare_logits, greedy_identity

pytestmark = pytest.mark.gpu


@pytest.fixture(params=["graph", "ll"])
def executor(request):
    """Run the test under each step executor (XE_STEP is read at every step)."""
    old = os.environ.get("XE_STEP")
    os.environ["XE_STEP"] = request.param
    yield request.param
    if old is None:
        os.environ.pop("XE_STEP", None)
    else:
        os.environ["XE_STEP"] = old


def tiny(xe, family, wdtype):
    if family == xe.XE_OPT:
        return xe.OPT_125M.replace(n_layers=2, d_model=256, n_heads=4, n_kv_heads=4, ffn=1024,
                                   vocab=1000, max_pos=256, max_ctx=256, wdtype=wdtype)
    if family == xe.XE_WHISPER:
        return xe.WHISPER_SMALL.replace(n_layers=2, d_model=256, n_heads=4, n_kv_heads=4,
                                        ffn=1024, vocab=1000, n_cross=100, wdtype=wdtype)
    return xe.GEMMA3_1B.replace(n_layers=2, d_model=256, ffn=1024, vocab=2048, max_ctx=512,
                                wdtype=wdtype)


def oracle_cfg(cfg):
    c = O.ModelConfig()
    for name, _ in O.ModelConfig._fields_:
        setattr(c, name, getattr(cfg, name))
    return c


def build(xe, gpu, cfg, seed, batch):
    dev, _ = gpu
    dec = xe.Decoder(dev, cfg, max_batch=batch)
    dec.init_synthetic(seed)
    om = O.OracleModel(oracle_cfg(cfg), seed, batch)
    if cfg.family == xe.XE_WHISPER:
        om.set_cross(None)
    return dec, om


def prompts(cfg, batch, n, seed):
    rng = np.random.default_rng(seed)
    return rng.integers(0, cfg.vocab, (batch, n)).astype(np.int32)


@pytest.mark.parametrize("family", ["opt", "whisper", "gemma"])
def test_synthetic_weights_bit_exact(gpu, xe, family):
    fam = {"opt": xe.XE_OPT, "whisper": xe.XE_WHISPER, "gemma": xe.XE_GEMMA3}[family]
    cfg = tiny(xe, fam, xe.XE_I8)
    dec, om = build(xe, gpu, cfg, seed=5, batch=1)
    kinds = [(O.XE_T_TOK_EMB, -1), (O.XE_T_Q_W, 0), (O.XE_T_K_W, 1), (O.XE_T_V_W, 0),
             (O.XE_T_O_W, 1), (O.XE_T_FC1_W, 0), (O.XE_T_FC2_W, 1)]
    if fam == xe.XE_GEMMA3:
        kinds.append((O.XE_T_UP_W, 1))
    if fam == xe.XE_WHISPER:
        kinds += [(O.XE_T_XQ_W, 0), (O.XE_T_XK_W, 1), (O.XE_T_XO_W, 1)]
    for kind, layer in kinds:
        want_q, want_s = om.tensor_q8(kind, layer)
        got_q, got_s = dec.get_tensor_q8(kind, layer, *want_q.shape)
        assert np.array_equal(got_q, want_q), (kind, layer)
        assert np.array_equal(got_s.view(np.uint32), want_s.view(np.uint32)), (kind, layer)
    dec.close()
    om.close()


CASES = [(f, w) for f in ("opt", "whisper", "gemma") for w in ("i8", "bf16", "bfp16")]


@pytest.mark.parametrize("family,wd", CASES)
def test_tiny_greedy_identity(gpu, xe, executor, family, wd):
    fam = {"opt": xe.XE_OPT, "whisper": xe.XE_WHISPER, "gemma": xe.XE_GEMMA3}[family]
    wdtype = {"i8": xe.XE_I8, "bf16": xe.XE_BF16, "bfp16": xe.XE_BFP16}[wd]
    cfg = tiny(xe, fam, wdtype)
    batch = 3
    print("[case] tiny %s %s batch %d %s" % (family, wd, batch, executor), flush=True)
    dec, om = build(xe, gpu, cfg, seed=11, batch=batch)
    pr = prompts(cfg, batch, 6, seed=1)
    got = dec.generate(pr, 40)
    greedy_identity(got, om, pr, "tiny-%s-%s" % (family, wd))
    dec.close()
    om.close()


@pytest.mark.parametrize("family", ["opt", "gemma"])
def test_tiny_greedy_four_streams(gpu, xe, executor, family):
    """Four streams: the widest low-latency step (its 4-stream instantiation
    with every stream live) and, on the graph executor, the smallest batch
    whose projections run on the MFMA GEMM (one 16-stream tile, 12 rows
    empty)."""
    fam = {"opt": xe.XE_OPT, "gemma": xe.XE_GEMMA3}[family]
    cfg = tiny(xe, fam, xe.XE_I8)
    batch = 4
    print("[case] tiny %s i8 batch %d %s" % (family, batch, executor), flush=True)
    dec, om = build(xe, gpu, cfg, seed=17, batch=batch)
    assert dec.executor(batch) == executor, dec.executor(batch)
    pr = prompts(cfg, batch, 5, seed=2)
    got = dec.generate(pr, 32)
    greedy_identity(got, om, pr, "tiny-%s-b4-%s" % (family, executor))
    dec.close()
    om.close()


@pytest.mark.parametrize("family", ["opt", "whisper", "gemma"])
def test_tiny_step_logits(gpu, xe, executor, family):
    """step() logits (per-stream positions) vs the oracle's, step by step."""
    fam = {"opt": xe.XE_OPT, "whisper": xe.XE_WHISPER, "gemma": xe.XE_GEMMA3}[family]
    cfg = tiny(xe, fam, xe.XE_I8)
    dec, om = build(xe, gpu, cfg, seed=3, batch=2)
    rng = np.random.default_rng(2)
    for p in range(12):
        toks = rng.integers(0, cfg.vocab, 2).astype(np.int32)
        pos = np.array([p, p], np.int32)
        got, nxt = dec.step(toks, pos)
        want = om.step(toks, pos)
        assert np.allclose(got, want, rtol=1e-2, atol=1e-3), np.max(np.abs(got - want))
        # fp32 order differences occasionally flip a bf16 K/V element by one
        # ulp (2^-9) at the cache write; that bounds the logits drift near 1e-4
        rel = np.linalg.norm(got - want) / np.linalg.norm(want)
        assert rel < 1e-3, rel
        for b in range(2):
            assert nxt[b] == om.argmax(want[b])
    dec.close()
    om.close()


def test_opt125m_config1(gpu, xe, executor):
    """Config 1: OPT-125m shape, int8, seed 0, 32-token prompt, 128 greedy steps."""
    cfg = xe.OPT_125M
    dec, om = build(xe, gpu, cfg, seed=0, batch=1)
    pr = prompts(cfg, 1, 32, seed=0)
    got = dec.generate(pr, 128)
    greedy_identity(got, om, pr, "opt125m", eps=5e-3)
    dec.close()
    om.close()


def test_gemma3_1b_short(gpu, xe, executor):
    """Config 5 shape (Gemma-3-1B, int8, seed 2): a short prompt and stream the
    oracle finishes in seconds, plus step logits."""
    cfg = xe.GEMMA3_1B.replace(max_ctx=512)
    dec, om = build(xe, gpu, cfg, seed=2, batch=1)
    pr = prompts(cfg, 1, 8, seed=2)
    got = dec.generate(pr, 8)
    greedy_identity(got, om, pr, "gemma3-1b", eps=1e-2)
    dec.close()
    om.close()


def test_whisper_small_short(gpu, xe, executor):
    """Config 4 shape (Whisper-small, int8, seed 1, 1500 encoder frames, 4-token
    start prompt)."""
    cfg = xe.WHISPER_SMALL
    dec, om = build(xe, gpu, cfg, seed=1, batch=1)
    pr = prompts(cfg, 1, 4, seed=1)
    got = dec.generate(pr, 12)
    greedy_identity(got, om, pr, "whisper-small", eps=5e-3)
    dec.close()
    om.close()


# ---- per-utterance int8 cross K / V (gen_decode.py:263-282) ----

@pytest.mark.parametrize("k8,v8,step", [(1, 0, None), (0, 1, None), (1, 1, None), (1, 1, "graph")])
def test_whisper_int8_cross_kv(gpu, xe, monkeypatch, k8, v8, step):
    """int8 cross K and/or V with per-channel scales, quantised on the GPU
    from the fp32 projections (whisper_decoder.rs:1186-1219): step logits and
    a greedy stream against the oracle with the same quantisation.  K and V
    both int8 run inside the low-latency step (int8 rows converted exactly
    for the matrix-core Q.K, the K scale on q, the V scale on the partial
    sums); K or V alone, or XE_STEP=graph, on the phase kernels."""
    if step:
        monkeypatch.setenv("XE_STEP", step)
    else:
        monkeypatch.delenv("XE_STEP", raising=False)
    dev, _ = gpu
    cfg = tiny(xe, xe.XE_WHISPER, xe.XE_I8)
    print("[case] tiny whisper int8 cross k=%d v=%d %s" % (k8, v8, step or "default"), flush=True)
    dec = xe.Decoder(dev, cfg, max_batch=2)
    dec.init_synthetic(9)
    dec.set_cross_int8(k8, v8)
    dec.precompute_cross(None)
    want_exec = "ll" if k8 and v8 and step is None else "graph"
    assert dec.executor(1) == want_exec and dec.executor(2) == want_exec
    om = O.OracleModel(oracle_cfg(cfg), 9, 2)
    om.set_cross_i8(k8, v8)
    om.set_cross(None)
    rng = np.random.default_rng(5)
    for p in range(8):
        toks = rng.integers(0, cfg.vocab, 2).astype(np.int32)
        pos = np.array([p, p + 3], np.int32)
        got, nxt = dec.step(toks, pos)
        want = om.step(toks, pos)
        compare_logits(got, want, "whisper-int8-cross-k%d-v%d-step%d" % (k8, v8, p))
    om.close()
    dec.reset()
    pr = prompts(cfg, 2, 4, seed=6)
    got = dec.generate(pr, 30)
    om = O.OracleModel(oracle_cfg(cfg), 9, 2)
    om.set_cross_i8(k8, v8)
    om.set_cross(None)
    greedy_identity(got, om, pr, "whisper-int8-cross-k%d-v%d" % (k8, v8))
    om.close()
    # back to bf16 cross K / V: the default executor again, oracle's stream
    dec.set_cross_int8(0, 0)
    dec.precompute_cross(None)
    assert dec.executor(1) == (step or "ll")
    dec.reset()
    got = dec.generate(pr[:1], 12)
    om = O.OracleModel(oracle_cfg(cfg), 9, 1)
    om.set_cross(None)
    greedy_identity(got, om, pr[:1], "whisper-bf16-cross-after-int8")
    om.close()
    dec.close()


def test_whisper_small_int8_cross(gpu, xe, monkeypatch):
    """Config 4 shape (Whisper-small, 1500 frames) with int8 cross K and V on
    the low-latency executor (two streams, one starting later): a greedy
    stream against the oracle, then step logits."""
    monkeypatch.delenv("XE_STEP", raising=False)
    dev, _ = gpu
    cfg = xe.WHISPER_SMALL
    dec = xe.Decoder(dev, cfg, max_batch=2)
    dec.init_synthetic(1)
    dec.set_cross_int8(1, 1)
    dec.precompute_cross(None)
    assert dec.executor(1) == "ll" and dec.executor(2) == "ll"
    om = O.OracleModel(oracle_cfg(cfg), 1, 2)
    om.set_cross_i8(1, 1)
    om.set_cross(None)
    pr = prompts(cfg, 2, 4, seed=1)
    got = dec.generate(pr, 40)
    greedy_identity(got, om, pr, "whisper-small-int8-cross", eps=5e-3)
    tok = got[:, -1].copy()
    pos = np.full(2, 4 + 40 - 1, np.int32)
    g, _ = dec.step(tok, pos)
    om.reset()
    for p in range(4):
        om.step(pr[:, p], np.full(2, p, np.int32))
    for i in range(39):
        om.step(got[:, i], np.full(2, 4 + i, np.int32))
    w = om.step(tok, pos)
    compare_logits(g, w, "whisper-small-int8-cross-step", atol=5e-3)
    dec.close()
    om.close()


# ---- batched projections on MFMA (gemm.hip): more than 8 streams ----

@pytest.mark.parametrize("family,wd", CASES)
def test_tiny_batched_gemm_identity(gpu, xe, family, wd):
    """20 streams (two MFMA column blocks, the second partial): every
    projection runs as the bf16x3 MFMA GEMM; greedy streams equal the
    oracle's fp32 ones."""
    fam = {"opt": xe.XE_OPT, "whisper": xe.XE_WHISPER, "gemma": xe.XE_GEMMA3}[family]
    wdtype = {"i8": xe.XE_I8, "bf16": xe.XE_BF16, "bfp16": xe.XE_BFP16}[wd]
    cfg = tiny(xe, fam, wdtype)
    batch = 20
    print("[case] tiny batched %s %s batch %d" % (family, wd, batch), flush=True)
    dec, om = build(xe, gpu, cfg, seed=13, batch=batch)
    pr = prompts(cfg, batch, 5, seed=4)
    got = dec.generate(pr, 24)
    greedy_identity(got, om, pr, "tiny-b%d-%s-%s" % (batch, family, wd))
    dec.close()
    om.close()


@pytest.mark.parametrize("family", ["opt", "gemma"])
def test_tiny_batched_step_logits(gpu, xe, family):
    """step() logits at 17 streams with per-stream positions vs the oracle."""
    fam = {"opt": xe.XE_OPT, "gemma": xe.XE_GEMMA3}[family]
    cfg = tiny(xe, fam, xe.XE_I8)
    batch = 17
    dec, om = build(xe, gpu, cfg, seed=3, batch=batch)
    rng = np.random.default_rng(7)
    for p in range(6):
        toks = rng.integers(0, cfg.vocab, batch).astype(np.int32)
        pos = (np.arange(batch, dtype=np.int32) % 3 + p).astype(np.int32)
        got, nxt = dec.step(toks, pos)
        want = om.step(toks, pos)
        assert np.allclose(got, want, rtol=1e-2, atol=1e-3), np.max(np.abs(got - want))
        rel = np.linalg.norm(got - want) / np.linalg.norm(want)
        assert rel < 1e-3, rel
        for b in range(batch):
            assert nxt[b] == om.argmax(want[b])
    dec.close()
    om.close()


@pytest.mark.parametrize("family", ["gemma", "opt"])
@pytest.mark.parametrize("batch", [1, 3, 20])
def test_argmax_tie_rule_on_planted_ties(gpu, xe, family, batch):
    """Exact ties among the largest logits: rows of the tied embedding /
    lm-head planted equal (+c e_0 at several vocab positions, -c e_0 at
    others), so their logits are bit-identical and, for most streams, the
    largest.  The token the device argmax picks is the family rule's on
    the same logits (the oracle's argmax: first max for Gemma, whisper.rs:
    749-757; last max for OPT, opt125m_decode.rs:303), with the tied rows
    spread over different argmax blocks, lanes and workgroups: 1 and 3
    streams (the low-latency kernel's argmax over its 256 workgroups), 20
    (the argmax partial and final kernels)."""
    dev, _ = gpu
    fam = {"opt": xe.XE_OPT, "gemma": xe.XE_GEMMA3}[family]
    cfg = tiny(xe, fam, xe.XE_I8)
    V, D = cfg.vocab, cfg.d_model
    print("[case] planted ties %s b=%d" % (family, batch), flush=True)
    dec = xe.Decoder(dev, cfg, max_batch=batch)
    dec.init_synthetic(3)
    om = O.OracleModel(oracle_cfg(cfg), 3, 1)
    rows, cols = xe.tensor_shape(cfg, O.XE_T_TOK_EMB, -1)
    q, sc = dec.get_tensor_q8(O.XE_T_TOK_EMB, -1, rows, cols)
    emb = q.astype(np.float32) * sc[:, None]
    plus = [3, 4, 130, V // 2 + 7, V - 1]
    minus = [5, 131, V // 2 + 8, V - 2]
    for r in plus:
        emb[r] = 0.0
        emb[r, 0] = 4.0
    for r in minus:
        emb[r] = 0.0
        emb[r, 0] = -4.0
    dec.set_tensor(O.XE_T_TOK_EMB, -1, emb)
    planted = set(plus) | set(minus)
    rng = np.random.default_rng(5)
    hits = 0
    for step in range(4):
        toks = rng.integers(0, V, batch).astype(np.int32)
        toks = np.array([t if t not in planted else (t + 11) % V for t in toks], np.int32)
        pos = np.full(batch, step, np.int32)
        logits, nxt = dec.step(toks, pos)
        for b in range(batch):
            want = om.argmax(logits[b])
            assert nxt[b] == want, (step, b, int(nxt[b]), int(want))
            if want in planted:
                group = plus if want in plus else minus
                vals = logits[b][group].view(np.uint32)
                assert np.all(vals == vals[0]), (step, b)
                assert want == (max(group) if family == "opt" else min(group)), (step, b, want)
                hits += 1
    dec.close()
    om.close()
    assert hits >= 2 * batch, hits


PARTS_CASES = [("gemma", 64, "gemv_gateup_pro"), ("whisper", 32, "gemv_fc1_pro"), ("opt", 16, "gemv_fc1_pro")]


@pytest.mark.parametrize("family,batch,pro", PARTS_CASES)
def test_gemm_split_partials_in_prologue(gpu, xe, monkeypatch, family, batch, pro):
    """A GEMM that splits K hands its split partials to the next phase's
    prologue, which adds them in split order and applies the GEMM's epilogue
    (GemvParams::sub_part), instead of the GEMM's own arrival counter and
    finishing workgroup: forced steps on the real shapes give logits bit for
    bit equal to XE_GEMM_DEFER=0 (the GEMM's own finish), and the prologue
    does read the partials (its profiled bytes grow by the extra splits)."""
    dev, _ = gpu
    cfg = {"gemma": xe.GEMMA3_1B.replace(n_layers=2, max_ctx=64),
           "whisper": xe.WHISPER_SMALL.replace(n_layers=2),
           "opt": xe.OPT_125M.replace(n_layers=2)}[family]
    print("[case] split partials %s b=%d" % (family, batch), flush=True)
    rng = np.random.default_rng(3)
    toks = rng.integers(0, cfg.vocab, (4, batch)).astype(np.int32)
    outs, pro_bytes = [], []
    for defer in ("0", "1"):
        monkeypatch.setenv("XE_GEMM_DEFER", defer)
        dec = xe.Decoder(dev, cfg, max_batch=batch)
        dec.init_synthetic(5)
        if family == "whisper":
            dec.precompute_cross(None)
        assert dec.executor(batch) == "graph"
        logits = []
        for i in range(4):
            g, _ = dec.step(toks[i], np.full(batch, i, np.int32))
            logits.append(g.copy())
        pro_bytes.append(sum(by for lab, _, by in dec.profile_step(batch) if lab == pro))
        outs.append(np.stack(logits))
        dec.close()
    monkeypatch.delenv("XE_GEMM_DEFER", raising=False)
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    assert pro_bytes[1] > pro_bytes[0] > 0, pro_bytes


def test_gemma_lmhead_int8_digits(gpu, xe, monkeypatch):
    """XE_GEMM_I8=1: the 262144-row lm-head at 64 streams on the int8 matrix
    cores (gemm_i8_kernel): the final norm writes each stream's row as four
    int8 digit planes of rint(x 2^(30 - E)), the weights are the int8 MFMA
    operand as stored, the four int32 sums combine exactly in fp64.  Forced
    steps on the real Gemma-3-1B shape (2 layers): logits within the oracle's
    bar, and not bit-equal to the bf16-plane path (the digit path ran)."""
    dev, _ = gpu
    cfg = xe.GEMMA3_1B.replace(n_layers=2, max_ctx=64)
    batch = 64
    print("[case] gemma lm-head int8 digits b=%d" % batch, flush=True)
    om = O.OracleModel(oracle_cfg(cfg), 6, batch)
    rng = np.random.default_rng(8)
    toks = rng.integers(0, cfg.vocab, (3, batch)).astype(np.int32)
    outs = []
    for flag in ("1", "0"):
        monkeypatch.setenv("XE_GEMM_I8", flag)
        dec = xe.Decoder(dev, cfg, max_batch=batch)
        dec.init_synthetic(6)
        outs.append(np.stack([dec.step(toks[i], np.full(batch, i, np.int32))[0].copy() for i in range(3)]))
        dec.close()
    monkeypatch.delenv("XE_GEMM_I8", raising=False)
    om.reset()
    for i in range(3):
        want = om.step(toks[i], np.full(batch, i, np.int32))
        # the bars of the bf16 path at this depth and batch (test_long_gpu.py B64_DEPTHS)
        compare_logits(outs[0][i], want, "gemma-lmhead-i8-pos%d" % i, rel_l2=5e-4, atol=5e-3)
    assert not np.array_equal(outs[0], outs[1])
    assert np.abs(outs[0] - outs[1]).max() < 1e-4
    om.close()


def test_tiny_gemma_b64(gpu, xe):
    """64 streams (the config-5 batch) on the tiny Gemma shape."""
    cfg = tiny(xe, xe.XE_GEMMA3, xe.XE_I8)
    dec, om = build(xe, gpu, cfg, seed=2, batch=64)
    pr = prompts(cfg, 64, 4, seed=9)
    got = dec.generate(pr, 16)
    greedy_identity(got, om, pr, "tiny-gemma-b64")
    dec.close()
    om.close()


def test_gemma3_1b_batched_short(gpu, xe):
    """Config 5 shape at 16 streams: the MFMA GEMM path on the real sizes
    (K = 1152 and 6912, GeGLU pairs, the 262144-row lm-head)."""
    cfg = xe.GEMMA3_1B.replace(max_ctx=64)
    batch = 16
    dec, om = build(xe, gpu, cfg, seed=2, batch=batch)
    pr = prompts(cfg, batch, 3, seed=5)
    got = dec.generate(pr, 3)
    greedy_identity(got, om, pr, "gemma3-1b-b16", eps=1e-2)
    dec.close()
    om.close()


def test_gemma3_1b_bf16_b64_short(gpu, xe):
    """Config 5's bf16 baseline at its second batch: the real Gemma-3-1B
    shapes with bf16 weights at 64 streams (the MFMA GEMM's bf16 weight path,
    64-stream tiles, the 262144-row lm-head), greedy streams against the
    oracle."""
    cfg = xe.GEMMA3_1B.replace(wdtype=xe.XE_BF16, max_ctx=64)
    batch = 64
    print("[case] gemma3-1b bf16 b=%d" % batch, flush=True)
    dec, om = build(xe, gpu, cfg, seed=2, batch=batch)
    assert dec.executor(batch) == "graph"
    pr = prompts(cfg, batch, 2, seed=6)
    got = dec.generate(pr, 2)
    greedy_identity(got, om, pr, "gemma3-1b-bf16-b64", eps=1e-2)
    dec.close()
    om.close()


def test_decode_bounds_follow_step_positions(gpu, xe):
    """decode() bounds every stream by its own position, as step() left it:
    feed 4 tokens, step one stream at max_ctx - 1, then decode must refuse
    (its K/V row would land past the cache), and so must a decode of more
    streams than were fed."""
    cfg = xe.GEMMA3_1B.replace(n_layers=2, d_model=256, ffn=1024, vocab=2048, max_ctx=64)
    dev, _ = gpu
    dec = xe.Decoder(dev, cfg, max_batch=2)
    dec.init_synthetic(5)
    with pytest.raises(xe.XdnaError, match="feed a prompt first"):
        dec.decode(1, batch=1)
    dec.feed(np.arange(4, dtype=np.int32)[None])
    with pytest.raises(xe.XdnaError, match="exceeds the streams fed"):
        dec.decode(1, batch=2)
    dec.decode(2, batch=1)                       # positions 4, 5: fine
    dec.step(np.array([7], np.int32), np.array([cfg.max_ctx - 1], np.int32))
    with pytest.raises(xe.XdnaError, match="past max_ctx"):
        dec.decode(1, batch=1)
    with pytest.raises(xe.XdnaError, match="position out of range"):
        dec.step(np.array([7], np.int32), np.array([cfg.max_ctx], np.int32))
    # a new prompt restarts the positions
    dec.feed(np.arange(4, dtype=np.int32)[None])
    toks, _ = dec.decode(cfg.max_ctx - 4, batch=1)
    assert toks.shape == (1, cfg.max_ctx - 4)
    with pytest.raises(xe.XdnaError, match="past max_ctx"):
        dec.decode(1, batch=1)
    dec.close()


# ---- the stop rule (EOT; whisper.rs:371-380 single stream, :618-668 batched) ----
# (family, executor, streams, step of stream 0 whose token is the stop id)
STOP_CASES = [("gemma", "ll", 2, 20), ("gemma", "graph", 2, 20), ("gemma", "graph", 12, 20),
              ("whisper", "ll", 1, 14), ("opt", "graph", 3, 0), ("gemma", "ll", 1, 0)]


@pytest.mark.parametrize("family,step,batch,at", STOP_CASES)
def test_stop_token(gpu, xe, monkeypatch, family, step, batch, at):
    """generate_until against the oracle's: each stream ends at its first
    emitted stop token (tokens before it identical, n_out equal, the stop id
    after), streams that never emit it run to max_new; stopped streams are
    fed the stop id while the others continue.  Then a single stream stopped
    mid-run: the device loop ends at once (low-latency: the launch stops at
    that step) or at the next check (phase kernels: every 8 steps)."""
    monkeypatch.setenv("XE_STEP", step)
    fam = {"opt": xe.XE_OPT, "whisper": xe.XE_WHISPER, "gemma": xe.XE_GEMMA3}[family]
    cfg = tiny(xe, fam, xe.XE_I8)
    max_new = 48
    print("[case] stop %s %s batch %d at %d" % (family, step, batch, at), flush=True)
    dec, om = build(xe, gpu, cfg, seed=13, batch=batch)
    if fam == xe.XE_WHISPER:
        dec.precompute_cross(None)
    pr = prompts(cfg, batch, 5, seed=3)
    free, _ = om.generate(pr, max_new)
    stop = int(free[0, at])
    om.reset()
    want, want_n, _ = om.generate_until(pr, max_new, stop)
    assert want_n[0] <= at
    got, got_n = dec.generate_until(pr, max_new, stop)
    assert dec.executor(batch) == step
    assert np.array_equal(got_n, want_n), (got_n, want_n)
    assert np.array_equal(got, want)
    # the decoder's own stop setting is back to none: a plain generate runs on
    g2 = dec.generate(pr, max_new)
    assert np.array_equal(g2, free)
    # one stream through set_stop / feed / decode: the run ends early
    dec.set_stop(stop)
    dec.feed(pr[:1])
    toks, _ = dec.decode(max_new - 1, batch=1)
    k = int(want_n[0])  # decode step k - 1 emits the stop (step j emits token j + 1)
    ran = dec.steps_run
    if step == "ll":
        assert ran == k, (ran, k)
    else:
        assert ran == min(max_new - 1, -(-k // 8) * 8), (ran, k)
    assert np.array_equal(toks[0, :max(k - 1, 0)], want[0, 1:k])
    assert np.all(toks[0, max(k - 1, 0):] == stop)
    dec.set_stop(-1)
    dec.close()
    om.close()
