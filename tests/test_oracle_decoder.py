"""The oracle's decoder composition (xo_step_one, oracle/xe_oracle.c) against
Hugging Face's OPT, Whisper-decoder and Gemma-3 implementations.

tests/golden/hf_decoder_*.npz hold HF's fp32 logits at every position of a
prompt + greedy stream, computed on the oracle's own weights (int8 q * scale,
fp32 vectors) by tests/golden/gen_hf_decoder_vectors.py; the reference builds
its goldens with the same library (scripts/opt125m_reference.py:7-9,
scripts/gemma_ref_generate.py:42-47).  The oracle keeps its K/V in fp32 here,
as the reference CPU decoders do (opt125m_decode.rs:263-268,
whisper_decoder.rs:458, 472); the product and its default oracle round K/V
to bf16, checked below as a bounded deviation.

What this pins: OPT's position offset (+2) and q scaling, pre-LN order and
ReLU; Whisper's cross attention (no k bias), three pre-norms and exact GELU;
Gemma-3's sandwich norms, (1 + w) RMSNorm, per-head q/k norms, RoPE
(rotate-half, theta from the config), sqrt(d) embedding scale, GeGLU-tanh
and the 1/sqrt(query_pre_attn_scalar) score scale; the tied head.  Each
planted mistake (oracle XO_MUT_*) must break the match.
"""
import os

import numpy as np
import pytest

import oracle_lib as O

HERE = os.path.dirname(os.path.abspath(__file__))
FAMILIES = ["opt", "whisper", "gemma3"]


def fixture(name):
    return np.load(os.path.join(HERE, "golden", "hf_decoder_%s.npz" % name), allow_pickle=False)


def oracle_model(fx, kv_f32=True):
    c = O.ModelConfig()
    for k, v in zip(fx["cfg_names"], fx["cfg_values"]):
        k = str(k)
        setattr(c, k, float(v) if k in ("eps", "rope_theta") else int(round(float(v))))
    om = O.OracleModel(c, int(fx["seed"]), 1)
    if kv_f32:
        om.set_kv_f32(True)
    if c.family == 1:
        om.set_cross(None)
    return om


def oracle_logits(om, tokens, n):
    return np.stack([om.step(np.array([tokens[p]], np.int32), np.array([p], np.int32))[0]
                     for p in range(n)])


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return np.linalg.norm(a - b, axis=-1) / np.linalg.norm(b, axis=-1)


@pytest.mark.parametrize("name", FAMILIES)
def test_oracle_decoder_matches_hf(name):
    fx = fixture(name)
    want = fx["logits"]
    toks = fx["tokens"]
    om = oracle_model(fx)
    got = oracle_logits(om, toks, want.shape[0])
    err = rel_l2(got, want)
    # fp32 on both sides; only summation order and libm differ (measured
    # <= 9.3e-7 rel-L2, 5.1e-7 max abs; every planted mistake >= 1.6e-2)
    assert err.max() <= 5e-6, err
    assert np.max(np.abs(got - want)) <= 5e-6
    # the greedy continuation: the oracle's argmax (its family tie rule) is
    # HF's token at every generated position
    n_prompt = int(fx["n_prompt"])
    for p in range(n_prompt - 1, want.shape[0]):
        assert om.argmax(got[p]) == toks[p + 1], p
    om.close()


CASES = [("opt", 1), ("opt", 6), ("whisper", 5), ("gemma3", 2), ("gemma3", 3), ("gemma3", 4)]
NAMES = {1: "OPT position offset +1", 2: "Gemma post-norms swapped", 3: "no sqrt(d) embedding scale",
         4: "RoPE theta 1e4", 5: "Whisper cross scores without 1/sqrt(hd)",
         6: "OPT q without hd^-0.5"}


@pytest.mark.parametrize("name,mutation", CASES)
def test_planted_composition_mistake_is_caught(name, mutation):
    """The fixtures pin the composition: each planted mistake moves the
    logits far outside the tolerance above."""
    fx = fixture(name)
    want = fx["logits"]
    om = oracle_model(fx)
    om.set_mutation(mutation)
    got = oracle_logits(om, fx["tokens"], want.shape[0])
    om.close()
    assert rel_l2(got, want).max() > 1e-2, NAMES[mutation]


@pytest.mark.parametrize("name", FAMILIES)
def test_bf16_kv_oracle_deviation_is_bounded(name):
    """The default oracle (bf16 K/V cache, the product's numerics) stays
    within bf16 rounding of HF's fp32-cache logits on these tiny models."""
    fx = fixture(name)
    want = fx["logits"]
    om = oracle_model(fx, kv_f32=False)
    got = oracle_logits(om, fx["tokens"], want.shape[0])
    om.close()
    err = rel_l2(got, want)
    assert err.max() <= 1e-2, err   # measured 1.3e-3 (OPT, Whisper), 4.1e-3 (Gemma-3)


def test_kouter_mode_is_bit_identical():
    """The reference-shaped k-outer linears ([K, N], opt125m_decode.rs:106-125)
    used for the CPU timing compute exactly the default form's values."""
    fx = fixture("gemma3")
    a = oracle_model(fx, kv_f32=False)
    b = oracle_model(fx, kv_f32=False)
    b.set_kouter(True)
    toks = fx["tokens"]
    la = oracle_logits(a, toks, 12)
    lb = oracle_logits(b, toks, 12)
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    a.close()
    b.close()


def test_oracle_stop_rule_truncates_the_free_stream():
    """xo_model_generate_until (the EOT rule of whisper.rs:371-380, 618-668):
    each stream is the plain greedy stream up to its first emitted stop
    token, n_out counts the tokens before it and the stop token fills the
    rest; a stream that never emits it is the plain stream.  Three streams of
    a tiny OPT model; the stop token is one the first stream emits at step 9
    (and a second case: the first token it emits, so n_out = 0)."""
    c = O.ModelConfig()
    for k, v in dict(family=0, n_layers=2, d_model=64, n_heads=2, n_kv_heads=2, head_dim=32, ffn=128,
                     vocab=50, max_pos=64, max_ctx=64, wdtype=2, eps=1e-5, rope_theta=0.0,
                     n_cross=0).items():
        setattr(c, k, v)
    om = O.OracleModel(c, 3, 3)
    prompt = np.random.default_rng(0).integers(0, 50, (3, 4)).astype(np.int32)
    free, _ = om.generate(prompt, 24)
    for at in (9, 0):
        om.reset()
        stop = int(free[0, at])
        out, n_out, _ = om.generate_until(prompt, 24, stop)
        for b in range(3):
            hits = np.nonzero(free[b] == stop)[0]
            k = int(hits[0]) if hits.size else 24
            assert n_out[b] == k, (b, n_out[b], k)
            assert np.array_equal(out[b, :k], free[b, :k])
            assert np.all(out[b, k:] == stop)
        assert n_out[0] <= at
    om.close()
