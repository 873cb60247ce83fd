"""The weight-file loader (xe_decoder_load_safetensors; the reference's arena
loader rust/npu-weights/src/arena.rs:14-99 and its OPT arch map
arch/opt.rs:1-123).

Host-only checks (no GPU) run the loader's dry run, xe_safetensors_plan, on
files written here with the safetensors package:
  * Hugging Face checkpoints of the three decoders built from the oracle's
    weights by tests/golden/gen_hf_decoder_vectors.py:checkpoint() -- the
    name tables there load into HF's own modules (every parameter present,
    every shape equal) and give the logits the oracle is pinned against.
    Each tensor of the file must map to the (kind, layer) whose oracle data
    it holds, so a swapped or wrong mapping fails;
  * a baked OPT arena in the reference's layout (names of arch/opt.rs,
    linears transposed [in, out] bf16, vectors f32, metadata arch "opt" and
    format_version "1");
  * files the loader must refuse (a tensor missing, another arch, another
    format version, a truncated header).
GPU checks load those files into a decoder and compare it with decoders
given the same weights through init_synthetic / xe_decoder_set_tensor.
"""
import os
import sys

import numpy as np
import pytest

import oracle_lib as O

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import gen_hf_decoder_vectors as G  # noqa: E402

st = pytest.importorskip("safetensors.numpy")

FAMILIES = ["opt", "whisper", "gemma3"]


def model_cfg(xe, cfgd):
    c = xe.ModelConfig()
    for k, v in cfgd.items():
        setattr(c, k, v)
    return c


def oracle(cfgd, seed):
    om = G.oracle_model(cfgd, seed)
    return om


def expected_data(om, kind, layer):
    """The oracle's tensor (kind, layer) as the checkpoint stores it."""
    try:
        q, s = om.tensor_q8(kind, layer)
        return (q.astype(np.float32) * s[:, None]).astype(np.float32)
    except Exception:
        return om.tensor_f32(kind, layer)


def hf_file(tmp_path, name, extras=True):
    cfgd, seed, _, _ = G.CASES[name]
    om = oracle(cfgd, seed)
    sd = G.checkpoint(name, cfgd, om)
    if extras:  # tensors a full checkpoint carries that the decoder does not use
        if name == "whisper":
            sd["proj_out.weight"] = sd["model.decoder.embed_tokens.weight"].copy()
            sd["model.encoder.layers.0.fc1.weight"] = np.zeros((8, 8), np.float32)
        else:
            key = "model.decoder.embed_tokens.weight" if name == "opt" else "model.embed_tokens.weight"
            sd["lm_head.weight"] = sd[key].copy()
    path = str(tmp_path / ("%s.safetensors" % name))
    st.save_file({k: np.ascontiguousarray(v, np.float32) for k, v in sd.items()}, path)
    return path, cfgd, seed, om, sd


@pytest.mark.parametrize("name", FAMILIES)
def test_plan_maps_every_hf_parameter_to_its_tensor(tmp_path, xe, name):
    path, cfgd, seed, om, sd = hf_file(tmp_path, name)
    naming, plan = xe.safetensors_plan(path, model_cfg(xe, cfgd))
    assert naming == "hf"
    assert set(plan) == set(sd)
    for k, tgt in plan.items():
        if k in ("lm_head.weight", "proj_out.weight") or k.startswith("model.encoder."):
            assert tgt is None, k
            continue
        assert tgt is not None, k
        kind, layer, transposed = tgt
        assert not transposed
        got = np.asarray(sd[k], np.float32).reshape(-1)
        want = expected_data(om, kind, layer).reshape(-1)
        assert got.shape == want.shape and np.array_equal(got, want), (k, kind, layer)
    om.close()


def test_plan_uses_tied_head_for_missing_embedding(tmp_path, xe):
    """arch/opt.rs:18-20: a checkpoint without embed_tokens gets it from the
    tied lm_head."""
    cfgd, seed, _, _ = G.CASES["opt"]
    om = oracle(cfgd, seed)
    sd = G.checkpoint("opt", cfgd, om)
    sd["lm_head.weight"] = sd.pop("model.decoder.embed_tokens.weight")
    path = str(tmp_path / "tied.safetensors")
    st.save_file(sd, path)
    _, plan = xe.safetensors_plan(path, model_cfg(xe, cfgd))
    assert plan["lm_head.weight"] == (O.XE_T_TOK_EMB, -1, False)
    om.close()


def arena_opt(sd, cfgd):
    """The reference's baked OPT arena (arch/opt.rs:1-20, arena.rs:14-40):
    linears transposed [in, out] in bf16, vectors f32, embed_tokens and
    embed_positions verbatim bf16, lm_head transposed."""
    bf = lambda a: O.bf16_bits(np.ascontiguousarray(a, np.float32))  # noqa: E731
    out = {"embed_tokens": bf(sd["model.decoder.embed_tokens.weight"]),
           "embed_positions": bf(sd["model.decoder.embed_positions.weight"]),
           "ln_final.weight": sd["model.decoder.final_layer_norm.weight"],
           "ln_final.bias": sd["model.decoder.final_layer_norm.bias"],
           "lm_head.weight": bf(sd["model.decoder.embed_tokens.weight"].T)}
    for l in range(cfgd["n_layers"]):
        p = "model.decoder.layers.%d." % l
        for dst, src in (("q", "self_attn.q_proj"), ("k", "self_attn.k_proj"), ("v", "self_attn.v_proj"),
                         ("out", "self_attn.out_proj"), ("fc1", "fc1"), ("fc2", "fc2")):
            out["L%d/%s.weight" % (l, dst)] = bf(sd[p + src + ".weight"].T)
            out["L%d/%s.bias" % (l, dst)] = sd[p + src + ".bias"]
        for dst, src in (("ln_self", "self_attn_layer_norm"), ("ln_ffn", "final_layer_norm")):
            out["L%d/%s.weight" % (l, dst)] = sd[p + src + ".weight"]
            out["L%d/%s.bias" % (l, dst)] = sd[p + src + ".bias"]
    return out


def write_bf16_safetensors(path, tensors, metadata):
    """safetensors.numpy has no bfloat16: uint16 arrays are written, then the
    header is rewritten with dtype BF16 for them (same width: the data
    offsets, relative to the end of the header, do not move)."""
    import json
    st.save_file({k: np.ascontiguousarray(v) for k, v in tensors.items()}, path, metadata=metadata)
    raw = open(path, "rb").read()
    n = int.from_bytes(raw[:8], "little")
    hdr = json.loads(raw[8:8 + n])
    for k, v in hdr.items():
        if k != "__metadata__" and v["dtype"] == "U16":
            v["dtype"] = "BF16"
    h = json.dumps(hdr).encode()
    h += b" " * (-len(h) % 8)
    open(path, "wb").write(len(h).to_bytes(8, "little") + h + raw[8 + n:])


def arena_file(tmp_path, meta=None, cfgd=None):
    cfgd = cfgd or G.CASES["opt"][0]
    seed = G.CASES["opt"][1]
    om = oracle(cfgd, seed)
    sd = G.checkpoint("opt", cfgd, om)
    ar = arena_opt(sd, cfgd)
    path = str(tmp_path / "opt_arena.safetensors")
    write_bf16_safetensors(path, ar, meta or {"format_version": "1", "arch": "opt",
                                              "source_ref": "test", "source_fingerprint": "0"})
    return path, cfgd, om, ar


def test_plan_reference_arena_layout(tmp_path, xe):
    path, cfgd, om, ar = arena_file(tmp_path)
    naming, plan = xe.safetensors_plan(path, model_cfg(xe, cfgd))
    assert naming == "arena"
    assert plan["lm_head.weight"] is None  # tied with embed_tokens
    for k, tgt in plan.items():
        if k == "lm_head.weight":
            continue
        kind, layer, transposed = tgt
        assert transposed == (k.endswith(".weight") and k.startswith("L") and "/ln_" not in k), k
        a = ar[k]
        got = O.bf16_to_f32(a) if a.dtype == np.uint16 else a
        if transposed:
            got = got.T
        want = expected_data(om, kind, layer).reshape(got.shape)
        if a.dtype == np.uint16:
            want = O.bf16_to_f32(O.bf16_bits(want))
        assert np.array_equal(got, want), (k, kind, layer)
    om.close()


@pytest.mark.parametrize("meta,msg", [
    ({"format_version": "1", "arch": "bert"}, "arch"),
    ({"format_version": "2", "arch": "opt"}, "format_version"),
])
def test_plan_refuses_other_arenas(tmp_path, xe, meta, msg):
    path, cfgd, om, _ = arena_file(tmp_path, meta)
    with pytest.raises(xe.XdnaError, match=msg):
        xe.safetensors_plan(path, model_cfg(xe, cfgd))
    om.close()


def test_plan_refuses_missing_tensor_and_bad_files(tmp_path, xe):
    path, cfgd, seed, om, sd = hf_file(tmp_path, "gemma3", extras=False)
    del sd["model.layers.1.post_feedforward_layernorm.weight"]
    p2 = str(tmp_path / "missing.safetensors")
    st.save_file(sd, p2)
    with pytest.raises(xe.XdnaError, match="lacks tensors"):
        xe.safetensors_plan(p2, model_cfg(xe, cfgd))
    raw = open(path, "rb").read()
    p3 = str(tmp_path / "trunc.safetensors")
    open(p3, "wb").write(raw[:100])
    with pytest.raises(xe.XdnaError):
        xe.safetensors_plan(p3, model_cfg(xe, cfgd))
    with pytest.raises(xe.XdnaError, match="cannot open"):
        xe.safetensors_plan(str(tmp_path / "absent.safetensors"), model_cfg(xe, cfgd))
    om.close()


# ---------------------------------------------------------------- GPU ----

def forced_logits(dec, toks, n):
    out = []
    for p in range(n):
        lg, _ = dec.step(np.array([toks[p]], np.int32), np.array([p], np.int32))
        out.append(lg[0])
    return np.stack(out)


# GPU shapes: the decoder's heads are 64 / 128 / 256 wide (the HF fixture
# configurations above use 16 / 32)
GPU_CASES = {
    "opt": dict(G.CASES["opt"][0], d_model=256, head_dim=64, ffn=512, vocab=512),
    "whisper": dict(G.CASES["whisper"][0], d_model=256, head_dim=64, ffn=512, vocab=512),
    "gemma3": dict(G.CASES["gemma3"][0], d_model=256, head_dim=256, ffn=512, vocab=512),
}


@pytest.mark.gpu
@pytest.mark.parametrize("name", FAMILIES)
def test_gpu_hf_checkpoint_equals_synthetic_init(tmp_path, gpu, xe, name):
    """A decoder loaded from the HF checkpoint of the oracle's weights runs
    like the decoder that generated them (init_synthetic): the checkpoint
    holds q * scale, which requantises to the same int8 codes (a scale may
    move by one ulp), so teacher-forced logits agree to ~1e-6 and so does
    the argmax wherever the top-2 margin is not a tie."""
    dev, _ = gpu
    cfgd, seed = GPU_CASES[name], G.CASES[name][1]
    om = oracle(cfgd, seed)
    sd = G.checkpoint(name, cfgd, om)
    path = str(tmp_path / ("%s.safetensors" % name))
    st.save_file({k: np.ascontiguousarray(v, np.float32) for k, v in sd.items()}, path)
    cfg = model_cfg(xe, cfgd)
    a = xe.Decoder(dev, cfg, max_batch=1)
    b = xe.Decoder(dev, cfg, max_batch=1)
    print("[case] loader %s: %d tensors" % (name, a.load_safetensors(path)), flush=True)
    b.init_synthetic(seed)
    if name == "whisper":
        a.set_tensor(O.XE_T_ENC_OUT, -1, om.tensor_f32(O.XE_T_ENC_OUT, -1))
        a.precompute_cross(None)
        b.precompute_cross(None)
    rng = np.random.default_rng(seed)
    toks = rng.integers(0, cfgd["vocab"], 16).astype(np.int32)
    la, lb = forced_logits(a, toks, 16), forced_logits(b, toks, 16)
    err = np.linalg.norm(la - lb, axis=1) / np.linalg.norm(lb, axis=1)
    assert err.max() <= 1e-5, err
    for p in range(16):
        if np.argmax(la[p]) != np.argmax(lb[p]):
            top = np.sort(lb[p])[-2:]
            assert top[1] - top[0] <= 1e-4, p
    a.close()
    b.close()
    om.close()


@pytest.mark.gpu
def test_gpu_reference_arena_equals_set_tensor(tmp_path, gpu, xe):
    """The baked OPT arena (bf16 [in, out] linears) loads into exactly the
    decoder that xe_decoder_set_tensor builds from the same values
    ([out, in] fp32): identical int8 codes, scales and logits."""
    dev, _ = gpu
    path, cfgd, om, ar = arena_file(tmp_path, cfgd=GPU_CASES["opt"])
    cfg = model_cfg(xe, cfgd)
    a = xe.Decoder(dev, cfg, max_batch=1)
    b = xe.Decoder(dev, cfg, max_batch=1)
    assert a.load_safetensors(path) == len(ar) - 1
    _, plan = xe.safetensors_plan(path, cfg)
    for k, tgt in plan.items():
        if tgt is None:
            continue
        kind, layer, transposed = tgt
        v = ar[k]
        v = O.bf16_to_f32(v) if v.dtype == np.uint16 else np.asarray(v, np.float32)
        b.set_tensor(kind, layer, v.T.copy() if transposed else v)
    for kind in (O.XE_T_TOK_EMB, O.XE_T_Q_W, O.XE_T_O_W, O.XE_T_FC1_W, O.XE_T_FC2_W):
        for layer in ([-1] if kind == O.XE_T_TOK_EMB else range(cfgd["n_layers"])):
            rows, cols = xe.tensor_shape(cfg, kind, layer)
            qa, sa = a.get_tensor_q8(kind, layer, rows, cols)
            qb, sb = b.get_tensor_q8(kind, layer, rows, cols)
            assert np.array_equal(qa, qb) and np.array_equal(sa.view(np.uint32), sb.view(np.uint32))
    rng = np.random.default_rng(3)
    toks = rng.integers(0, cfgd["vocab"], 12).astype(np.int32)
    la, lb = forced_logits(a, toks, 12), forced_logits(b, toks, 12)
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    a.close()
    b.close()
    om.close()


def _raw_safetensors(path, header, data=b""):
    h = header.encode()
    with open(path, "wb") as f:
        f.write(len(h).to_bytes(8, "little") + h + data)
    return str(path)


@pytest.mark.parametrize("header,msg", [
    ('{"a":{"dtype":"F32","shape":[2],"data_offsets":[-8,0]}}', "non-negative integer"),
    ('{"a":{"dtype":"F32","shape":[2],"data_offsets":[0,7.5]}}', "non-negative integer"),
    ('{"a":{"dtype":"F32","shape":[2],"data_offsets":[0,"8"]}}', "non-negative integer"),
    ('{"a":{"dtype":"F32","shape":[-2],"data_offsets":[0,8]}}', "non-negative integer"),
    ('{"a":{"dtype":"F32","shape":[1e300],"data_offsets":[0,8]}}', "non-negative integer"),
    ('{"a":{"dtype":"F32","shape":[4294967296,4294967296,16],"data_offsets":[0,8]}}', "overflows"),
    ('{"a":{"dtype":"F32","shape":[3],"data_offsets":[0,8]}}', "does not match its shape"),
    ('1234567', "object expected"),
])
def test_plan_refuses_malformed_headers(tmp_path, xe, header, msg):
    """Header fields are checked before use: offsets and shape entries must
    be non-negative integers below 2^53, a shape's element count must not
    overflow, and a header that is a bare number at the end of the file is
    parsed from a terminated copy (nothing is read past it)."""
    p = _raw_safetensors(tmp_path / "bad.safetensors", header, b"\0" * 8)
    if header == "1234567":  # the header ends the file
        p = _raw_safetensors(tmp_path / "bare.safetensors", header)
    cfg = xe.OPT_125M.replace(n_layers=1)
    with pytest.raises(xe.XdnaError, match=msg):
        xe.safetensors_plan(p, cfg)
