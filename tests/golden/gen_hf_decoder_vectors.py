"""Write tests/golden/hf_decoder_{opt,whisper,gemma3}.npz: logits of Hugging
Face's own decoder implementations on the oracle's weights, the independent
check of the oracle's decoder composition (xo_step_one in
oracle/xe_oracle.c).

The reference builds its goldens with the same library: OPT in
scripts/opt125m_reference.py:7-9 (OPTForCausalLM) and Gemma in
scripts/gemma_ref_generate.py:42-47 (AutoModelForCausalLM); its Whisper host
decoder mirrors the HF/ONNX Whisper decoder (whisper_decoder.rs:388-535).
Nothing is downloaded: each model is built from a config object (tiny
shapes) and loaded with the oracle's synthetic int8 weights, dequantised
(q * scale) to fp32, and the fp32 vectors (norms, biases, positions).

Run in the build container only (torch + transformers; recorded in each
fixture); the GPU box only reads the .npz files:
    python tests/golden/gen_hf_decoder_vectors.py
Per family: a random prompt, then greedy tokens chosen by HF's argmax; the
fixture holds every position's token and HF's fp32 logits, computed without
a KV cache (the full prefix each step), so HF's cache code is not involved.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

import oracle_lib as O  # noqa: E402

XE_OPT, XE_WHISPER, XE_GEMMA3 = 0, 1, 2
XE_I8 = 2

# tiny configurations: (family, n_layers, d, heads, kv heads, head_dim, ffn,
# vocab, max_pos, max_ctx, eps, rope_theta, n_cross), seed, prompt, new tokens
CASES = {
    "opt": (dict(family=XE_OPT, n_layers=2, d_model=64, n_heads=4, n_kv_heads=4, head_dim=16,
                 ffn=256, vocab=384, max_pos=64, max_ctx=64, wdtype=XE_I8, eps=1e-5,
                 rope_theta=0.0, n_cross=0), 7, 6, 18),
    "whisper": (dict(family=XE_WHISPER, n_layers=2, d_model=64, n_heads=4, n_kv_heads=4,
                     head_dim=16, ffn=256, vocab=384, max_pos=64, max_ctx=64, wdtype=XE_I8,
                     eps=1e-5, rope_theta=0.0, n_cross=24), 8, 4, 18),
    "gemma3": (dict(family=XE_GEMMA3, n_layers=2, d_model=64, n_heads=4, n_kv_heads=1,
                    head_dim=32, ffn=128, vocab=384, max_pos=64, max_ctx=64, wdtype=XE_I8,
                    eps=1e-6, rope_theta=1e6, n_cross=0), 9, 6, 18),
}


def oracle_model(cfgd, seed):
    c = O.ModelConfig()
    for k, v in cfgd.items():
        setattr(c, k, v)
    return O.OracleModel(c, seed, 1)


def weight(om, kind, layer):
    """The oracle's stored linear as fp32: int8 q * per-row scale."""
    q, s = om.tensor_q8(kind, layer)
    return (q.astype(np.float32) * s[:, None]).astype(np.float32)


def vec(om, kind, layer=-1):
    return om.tensor_f32(kind, layer)


def checkpoint(name, cfgd, om):
    """The oracle's weights as a Hugging Face checkpoint of the family:
    {parameter name: fp32 array}, linears [out, in] dequantised (q * scale).
    The names are the ones HF's modules own (load() checks that none is
    missing and every shape matches); Whisper's are those of
    WhisperForConditionalGeneration (model.decoder.*)."""
    L = cfgd["n_layers"]
    d = cfgd["d_model"]
    if name == "opt":
        sd = {"model.decoder.embed_tokens.weight": weight(om, O.XE_T_TOK_EMB, -1),
              "model.decoder.embed_positions.weight": vec(om, O.XE_T_POS_EMB).reshape(cfgd["max_pos"] + 2, -1),
              "model.decoder.final_layer_norm.weight": vec(om, O.XE_T_LNF_W),
              "model.decoder.final_layer_norm.bias": vec(om, O.XE_T_LNF_B)}
        for l in range(cfgd["n_layers"]):
            p = "model.decoder.layers.%d." % l
            for hf, kind, bkind in (("self_attn.q_proj", O.XE_T_Q_W, O.XE_T_Q_B),
                                    ("self_attn.k_proj", O.XE_T_K_W, O.XE_T_K_B),
                                    ("self_attn.v_proj", O.XE_T_V_W, O.XE_T_V_B),
                                    ("self_attn.out_proj", O.XE_T_O_W, O.XE_T_O_B),
                                    ("fc1", O.XE_T_FC1_W, O.XE_T_FC1_B),
                                    ("fc2", O.XE_T_FC2_W, O.XE_T_FC2_B)):
                sd[p + hf + ".weight"] = weight(om, kind, l)
                sd[p + hf + ".bias"] = vec(om, bkind, l)
            sd[p + "self_attn_layer_norm.weight"] = vec(om, O.XE_T_LN1_W, l)
            sd[p + "self_attn_layer_norm.bias"] = vec(om, O.XE_T_LN1_B, l)
            sd[p + "final_layer_norm.weight"] = vec(om, O.XE_T_LN2_W, l)
            sd[p + "final_layer_norm.bias"] = vec(om, O.XE_T_LN2_B, l)
        return sd
    if name == "whisper":
        sd = {"model.decoder.embed_tokens.weight": weight(om, O.XE_T_TOK_EMB, -1),
              "model.decoder.embed_positions.weight": vec(om, O.XE_T_POS_EMB).reshape(cfgd["max_pos"], d),
              "model.decoder.layer_norm.weight": vec(om, O.XE_T_LNF_W), "model.decoder.layer_norm.bias": vec(om, O.XE_T_LNF_B)}
        for l in range(cfgd["n_layers"]):
            p = "model.decoder.layers.%d." % l
            for hf, kind, bkind in (("self_attn.q_proj", O.XE_T_Q_W, O.XE_T_Q_B),
                                    ("self_attn.k_proj", O.XE_T_K_W, None),
                                    ("self_attn.v_proj", O.XE_T_V_W, O.XE_T_V_B),
                                    ("self_attn.out_proj", O.XE_T_O_W, O.XE_T_O_B),
                                    ("encoder_attn.q_proj", O.XE_T_XQ_W, O.XE_T_XQ_B),
                                    ("encoder_attn.k_proj", O.XE_T_XK_W, None),
                                    ("encoder_attn.v_proj", O.XE_T_XV_W, O.XE_T_XV_B),
                                    ("encoder_attn.out_proj", O.XE_T_XO_W, O.XE_T_XO_B),
                                    ("fc1", O.XE_T_FC1_W, O.XE_T_FC1_B),
                                    ("fc2", O.XE_T_FC2_W, O.XE_T_FC2_B)):
                sd[p + hf + ".weight"] = weight(om, kind, l)
                if bkind is not None:
                    sd[p + hf + ".bias"] = vec(om, bkind, l)
            for hf, wk, bk in (("self_attn_layer_norm", O.XE_T_LN1_W, O.XE_T_LN1_B),
                               ("encoder_attn_layer_norm", O.XE_T_LNX_W, O.XE_T_LNX_B),
                               ("final_layer_norm", O.XE_T_LN2_W, O.XE_T_LN2_B)):
                sd[p + hf + ".weight"] = vec(om, wk, l)
                sd[p + hf + ".bias"] = vec(om, bk, l)
        return sd
    sd = {"model.embed_tokens.weight": weight(om, O.XE_T_TOK_EMB, -1),
          "model.norm.weight": vec(om, O.XE_T_LNF_W)}
    for l in range(L):
        p = "model.layers.%d." % l
        for hf, kind in (("self_attn.q_proj", O.XE_T_Q_W), ("self_attn.k_proj", O.XE_T_K_W),
                         ("self_attn.v_proj", O.XE_T_V_W), ("self_attn.o_proj", O.XE_T_O_W),
                         ("mlp.gate_proj", O.XE_T_FC1_W), ("mlp.up_proj", O.XE_T_UP_W),
                         ("mlp.down_proj", O.XE_T_FC2_W)):
            sd[p + hf + ".weight"] = weight(om, kind, l)
        for hf, kind in (("self_attn.q_norm", O.XE_T_QNORM_W), ("self_attn.k_norm", O.XE_T_KNORM_W),
                         ("input_layernorm", O.XE_T_LN1_W),
                         ("post_attention_layernorm", O.XE_T_POST_ATTN_W),
                         ("pre_feedforward_layernorm", O.XE_T_LN2_W),
                         ("post_feedforward_layernorm", O.XE_T_POST_FFN_W)):
            sd[p + hf + ".weight"] = vec(om, kind, l)
    return sd


def build_opt(cfgd, om):
    import torch
    from transformers import OPTConfig, OPTForCausalLM
    hc = OPTConfig(vocab_size=cfgd["vocab"], hidden_size=cfgd["d_model"],
                   num_hidden_layers=cfgd["n_layers"], ffn_dim=cfgd["ffn"],
                   num_attention_heads=cfgd["n_heads"], max_position_embeddings=cfgd["max_pos"],
                   word_embed_proj_dim=cfgd["d_model"], do_layer_norm_before=True,
                   activation_function="relu", enable_bias=True, tie_word_embeddings=True,
                   pad_token_id=1, bos_token_id=2, eos_token_id=2)
    m = OPTForCausalLM(hc)
    sd = checkpoint("opt", cfgd, om)
    load(m, sd)

    def logits(prefix):
        with torch.no_grad():
            out = m(input_ids=torch.tensor([prefix]), use_cache=False)
        return out.logits[0, -1].float().numpy()
    return logits


def build_whisper(cfgd, om):
    import torch
    from transformers import WhisperConfig
    from transformers.models.whisper.modeling_whisper import WhisperDecoder
    d = cfgd["d_model"]
    hc = WhisperConfig(vocab_size=cfgd["vocab"], d_model=d, decoder_layers=cfgd["n_layers"],
                       decoder_attention_heads=cfgd["n_heads"], decoder_ffn_dim=cfgd["ffn"],
                       max_target_positions=cfgd["max_pos"], encoder_layers=1,
                       encoder_attention_heads=cfgd["n_heads"], encoder_ffn_dim=cfgd["ffn"],
                       activation_function="gelu", scale_embedding=False, pad_token_id=0,
                       bos_token_id=1, eos_token_id=2, decoder_start_token_id=1)
    m = WhisperDecoder(hc)
    pre = "model.decoder."
    sd = {k[len(pre):]: v for k, v in checkpoint("whisper", cfgd, om).items()}
    load(m, sd)
    # the encoder output as the decoder sees it: synthetic N(0,1) rounded to bf16
    enc = vec(om, O.XE_T_ENC_OUT).reshape(cfgd["n_cross"], d)
    enc = O.bf16_to_f32(O.bf16_bits(enc))
    emb = torch.from_numpy(sd["embed_tokens.weight"])

    def logits(prefix):
        with torch.no_grad():
            h = m(input_ids=torch.tensor([prefix]),
                  encoder_hidden_states=torch.from_numpy(enc)[None], use_cache=False)
            h = h.last_hidden_state[0, -1]
        return (h @ emb.T).float().numpy()   # proj_out tied to embed_tokens
    return logits


def build_gemma3(cfgd, om):
    import torch
    from transformers import Gemma3ForCausalLM, Gemma3TextConfig
    L = cfgd["n_layers"]
    hc = Gemma3TextConfig(vocab_size=cfgd["vocab"], hidden_size=cfgd["d_model"],
                          intermediate_size=cfgd["ffn"], num_hidden_layers=L,
                          num_attention_heads=cfgd["n_heads"],
                          num_key_value_heads=cfgd["n_kv_heads"], head_dim=cfgd["head_dim"],
                          query_pre_attn_scalar=cfgd["head_dim"], rms_norm_eps=cfgd["eps"],
                          layer_types=["full_attention"] * L, max_position_embeddings=4096,
                          rope_parameters={"full_attention": {"rope_type": "default",
                                                              "rope_theta": cfgd["rope_theta"]},
                                           "sliding_attention": {"rope_type": "default",
                                                                 "rope_theta": 10000.0}},
                          hidden_activation="gelu_pytorch_tanh", tie_word_embeddings=True,
                          attention_bias=False, pad_token_id=0, bos_token_id=2, eos_token_id=1)
    m = Gemma3ForCausalLM(hc)
    sd = checkpoint("gemma3", cfgd, om)
    load(m, sd)

    def logits(prefix):
        with torch.no_grad():
            out = m(input_ids=torch.tensor([prefix]), use_cache=False)
        return out.logits[0, -1].float().numpy()
    return logits


def load(m, sd):
    import torch
    own = dict(m.named_parameters())
    missing = sorted(set(own) - set(sd))
    assert not missing, missing
    with torch.no_grad():
        for k, v in sd.items():
            assert tuple(own[k].shape) == v.shape, (k, own[k].shape, v.shape)
            own[k].copy_(torch.from_numpy(np.ascontiguousarray(v, np.float32)))
    m.eval()


def main():
    import torch
    import transformers
    torch.set_num_threads(max(1, min(8, os.cpu_count() or 1)))
    torch.manual_seed(0)
    for name, (cfgd, seed, n_prompt, n_new) in CASES.items():
        om = oracle_model(cfgd, seed)
        fn = {"opt": build_opt, "whisper": build_whisper, "gemma3": build_gemma3}[name](cfgd, om)
        rng = np.random.default_rng(seed)
        toks = [int(t) for t in rng.integers(0, cfgd["vocab"], n_prompt)]
        logits = []
        for i in range(n_prompt + n_new - 1):
            lg = fn(toks[:i + 1])
            logits.append(lg)
            if i + 1 >= n_prompt:
                toks.append(int(np.argmax(lg)))
        out = os.path.join(HERE, "hf_decoder_%s.npz" % name)
        np.savez(out, tokens=np.array(toks, np.int32), logits=np.stack(logits).astype(np.float32),
                 n_prompt=np.int32(n_prompt), seed=np.int64(seed),
                 cfg_names=np.array(sorted(cfgd)), cfg_values=np.array([float(cfgd[k]) for k in sorted(cfgd)]),
                 versions=np.array(["torch " + torch.__version__,
                                    "transformers " + transformers.__version__]))
        om.close()
        print("wrote", out, "tokens", toks)


if __name__ == "__main__":
    main()
