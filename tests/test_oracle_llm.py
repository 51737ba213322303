"""Pins the LLM oracle (oracle/llm.py) on the CPU against an independent
implementation of the same published architectures: Hugging Face
transformers' Qwen3ForCausalLM and GPT2LMHeadModel (5.x, installed offline),
random-initialised from small configs, fp32. The reference (Strict) has no
LLM code, so this library cross-check is what fixes the oracle's model
definition (norm placement, q/k head norms, RoPE convention, GQA head
mapping, SwiGLU / GELU-tanh, biases, tied heads, causal KV-cache decoding).

The oracle rounds activations to fp16 where the GPU path does; transformers
runs in fp32 throughout, so logits agree to ~1e-3 relative. Tolerance stated:
max |logit_oracle - logit_hf| <= 1e-2 * max |logit_hf|. A wrong rotation
direction, a missing q/k norm, a transposed projection or a misplaced
residual moves logits by O(1) relative and fails it (see
test_oracle_catches_planted_rope_mistake).
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
transformers = pytest.importorskip("transformers")

import oracle.llm as ollm  # noqa: E402
from strict_amd import llm  # noqa: E402


def _qwen3_pair(seed=0):
    torch.manual_seed(seed)
    hf_cfg = transformers.Qwen3Config(
        vocab_size=1000, hidden_size=256, intermediate_size=768, num_hidden_layers=2,
        num_attention_heads=4, num_key_value_heads=2, head_dim=128, rope_theta=1e6,
        rms_norm_eps=1e-6, tie_word_embeddings=True, max_position_embeddings=512,
        attention_bias=False)
    hf_cfg._attn_implementation = "eager"
    model = transformers.Qwen3ForCausalLM(hf_cfg).eval()
    with torch.no_grad():  # non-trivial norm gains
        for name, p in model.named_parameters():
            if "norm" in name:
                p.add_(0.1 * torch.randn_like(p))
    cfg = llm.Config(llm.QWEN3, layers=2, hidden=256, heads=4, kv_heads=2, head_dim=128,
                     intermediate=768, vocab=1000, max_positions=512)
    sd = {k: v.detach().numpy().astype(np.float32) for k, v in model.state_dict().items()}
    layers = []
    for i in range(cfg.layers):
        p = f"model.layers.{i}."
        L = {
            "qkv": np.concatenate([sd[p + "self_attn.q_proj.weight"], sd[p + "self_attn.k_proj.weight"],
                                   sd[p + "self_attn.v_proj.weight"]]),
            "o": sd[p + "self_attn.o_proj.weight"],
            "gate_up": np.concatenate([sd[p + "mlp.gate_proj.weight"], sd[p + "mlp.up_proj.weight"]]),
            "down": sd[p + "mlp.down_proj.weight"],
            "norm1.g": sd[p + "input_layernorm.weight"],
            "norm2.g": sd[p + "post_attention_layernorm.weight"],
            "q_norm": sd[p + "self_attn.q_norm.weight"],
            "k_norm": sd[p + "self_attn.k_norm.weight"],
        }
        for name in ("qkv", "o", "gate_up", "down"):
            L[name + ".scale"] = np.ones(L[name].shape[0], np.float32)
        layers.append(L)
    emb = sd["model.embed_tokens.weight"]
    w = ollm.Weights(cfg, layers, emb, np.ones(emb.shape[0], np.float32), sd["model.norm.weight"],
                     inv_freq=ollm.inv_freq(cfg.rope_theta, cfg.head_dim))
    return model, w


def _gpt2_pair(seed=0):
    torch.manual_seed(seed)
    hf_cfg = transformers.GPT2Config(vocab_size=997, n_positions=512, n_embd=256, n_layer=2,
                                     n_head=4, n_inner=512, activation_function="gelu_new",
                                     layer_norm_epsilon=1e-5, resid_pdrop=0.0, embd_pdrop=0.0,
                                     attn_pdrop=0.0)
    hf_cfg._attn_implementation = "eager"
    model = transformers.GPT2LMHeadModel(hf_cfg).eval()
    with torch.no_grad():  # non-trivial LayerNorm parameters and biases
        for name, p in model.named_parameters():
            if "ln" in name or "bias" in name:
                p.add_(0.05 * torch.randn_like(p))
    cfg = llm.Config(llm.GPT2, layers=2, hidden=256, heads=4, kv_heads=4, head_dim=64,
                     intermediate=512, vocab=997, max_positions=512, norm_eps=1e-5)
    sd = {k: v.detach().numpy().astype(np.float32) for k, v in model.state_dict().items()}
    layers = []
    for i in range(cfg.layers):
        p = f"transformer.h.{i}."
        L = {  # Conv1D weights are [in, out]; the oracle takes [out, in]
            "qkv": sd[p + "attn.c_attn.weight"].T.copy(), "qkv.bias": sd[p + "attn.c_attn.bias"],
            "o": sd[p + "attn.c_proj.weight"].T.copy(), "o.bias": sd[p + "attn.c_proj.bias"],
            "fc": sd[p + "mlp.c_fc.weight"].T.copy(), "fc.bias": sd[p + "mlp.c_fc.bias"],
            "proj": sd[p + "mlp.c_proj.weight"].T.copy(), "proj.bias": sd[p + "mlp.c_proj.bias"],
            "norm1.g": sd[p + "ln_1.weight"], "norm1.b": sd[p + "ln_1.bias"],
            "norm2.g": sd[p + "ln_2.weight"], "norm2.b": sd[p + "ln_2.bias"],
        }
        for name in ("qkv", "o", "fc", "proj"):
            L[name + ".scale"] = np.ones(L[name].shape[0], np.float32)
        layers.append(L)
    wte = sd["transformer.wte.weight"]
    w = ollm.Weights(cfg, layers, wte, np.ones(wte.shape[0], np.float32),
                     sd["transformer.ln_f.weight"], sd["transformer.ln_f.bias"],
                     wpe=sd["transformer.wpe.weight"])
    return model, w


def _hf_logits(model, tokens):
    with torch.no_grad():
        return model(torch.tensor(tokens)[None, :]).logits[0].numpy()


def _assert_close(ours, ref):
    err = float(np.max(np.abs(ours - ref)))
    scale = float(np.max(np.abs(ref)))
    assert err <= 1e-2 * scale, (err, scale)
    return err / scale


@pytest.mark.parametrize("acc", [np.float32, np.float64], ids=["fp32-sums", "fp64-sums"])
@pytest.mark.parametrize("pair", [_qwen3_pair, _gpt2_pair])
def test_oracle_prefill_matches_transformers(pair, acc):
    # both summation orders of the linears (the second-opinion decoder the
    # GPU tests consult at near-ties sums in fp64)
    model, w = pair()
    tokens = np.random.default_rng(1).integers(0, w.cfg.vocab, 24)
    _assert_close(ollm.Decoder(w, accumulate=acc).forward(tokens), _hf_logits(model, tokens))


def test_linear_fp64_sums_match_double_precision_sums():
    rng = np.random.default_rng(4)
    h = rng.normal(0, 1, (3, 64)).astype(np.float16).astype(np.float32)
    w = rng.normal(0, 0.02, (5, 64)).astype(np.float32)
    exact = np.array([[sum(float(a) * float(b) for a, b in zip(hr, wr)) for wr in w] for hr in h])
    got = ollm.linear(h, w, np.ones(5, np.float32), accumulate=np.float64)
    assert np.array_equal(got, exact.astype(np.float32))


@pytest.mark.parametrize("pair", [_qwen3_pair, _gpt2_pair])
def test_oracle_kv_cache_decode_matches_full_sequence(pair):
    # token-by-token decoding with the oracle's KV cache == one causal pass
    model, w = pair(seed=3)
    tokens = np.random.default_rng(2).integers(0, w.cfg.vocab, 20)
    dec = ollm.Decoder(w)
    step_logits = [dec.forward(tokens[:8])[-1]]
    for t in tokens[8:]:
        step_logits.append(dec.forward([int(t)])[-1])
    full = _hf_logits(model, tokens)
    _assert_close(np.stack(step_logits[:-1]), full[7:-1])


def test_oracle_catches_planted_rope_mistake():
    # planting a wrong rotation direction in the oracle must fail the check
    model, w = _qwen3_pair()
    tokens = np.random.default_rng(1).integers(0, w.cfg.vocab, 24)
    ref = _hf_logits(model, tokens)
    good = ollm.rope
    try:
        ollm.rope = lambda x, c, s: good(x, c, -s)
        with pytest.raises(AssertionError):
            _assert_close(ollm.Decoder(w).forward(tokens), ref)
    finally:
        ollm.rope = good


def test_inv_freq_matches_transformers_rope_init():
    cfg = transformers.Qwen3Config(head_dim=128, rope_theta=1e6, hidden_size=256,
                                   num_attention_heads=4, num_key_value_heads=2)
    rope = transformers.models.qwen3.modeling_qwen3.Qwen3RotaryEmbedding(cfg)
    ref = rope.inv_freq.numpy().astype(np.float64)
    ours = ollm.inv_freq(1e6, 128).astype(np.float64)
    assert np.allclose(ours, ref, rtol=1e-6)


def test_decode_step_bytes_config4():
    # 598,099,456 B of weights + 469,762,048 B of KV at b = 1, 4096
    # positions; this build also counts norm gains of the q/k head norms and
    # the embedding row, so the weights figure is within 0.1 %
    b = llm.decode_step_bytes(llm.QWEN3_0_6B, 1, 4096)
    assert b["kv"] == 469_762_048
    assert abs(b["weights"] - 598_099_456) / 598_099_456 < 1e-3


# ---- the decoder building blocks, one at a time (torch CPU as an independent check) ----

def test_norms_and_activations_match_torch():
    F = torch.nn.functional
    rng = np.random.default_rng(3)
    x = rng.normal(0, 2, (9, 1024)).astype(np.float32)
    g = (1 + rng.normal(0, 0.1, 1024)).astype(np.float32)
    b = rng.normal(0, 0.1, 1024).astype(np.float32)
    xt = torch.from_numpy(x).double()
    ref = F.rms_norm(xt, (1024,), torch.from_numpy(g).double(), eps=1e-6).numpy()
    assert np.max(np.abs(ollm.rms_norm(x, g, 1e-6) - ref)) <= 1e-6 * np.max(np.abs(ref))
    ref = F.layer_norm(xt, (1024,), torch.from_numpy(g).double(), torch.from_numpy(b).double(),
                       eps=1e-5).numpy()
    assert np.max(np.abs(ollm.layer_norm(x, g, b, 1e-5) - ref)) <= 1e-6 * np.max(np.abs(ref))
    z = np.linspace(-12, 12, 100_001).astype(np.float32)
    zt = torch.from_numpy(z).double()
    assert np.max(np.abs(ollm.silu(z) - F.silu(zt).numpy())) <= 4e-6
    assert np.max(np.abs(ollm.gelu_tanh(z) - F.gelu(zt, approximate="tanh").numpy())) <= 4e-6


def test_attn_decode_matches_torch_sdpa_gqa():
    # grouped-query decode attention with ragged lengths against torch's
    # scaled_dot_product_attention (fp64, K / V repeated per query group)
    F = torch.nn.functional
    rng = np.random.default_rng(4)
    B, H, KVH, P, d = 3, 8, 2, 50, 64
    q = rng.normal(0, 1, (B, H, d)).astype(np.float32)
    k = rng.normal(0, 1, (B, KVH, P, d)).astype(np.float32)
    v = rng.normal(0, 1, (B, KVH, P, d)).astype(np.float32)
    lengths = [50, 1, 17]
    scale = 1 / np.sqrt(d)
    got = ollm.attn_decode(q, k, v, lengths, scale)
    for b, L in enumerate(lengths):
        qt = torch.from_numpy((q[b] * np.float32(scale)).astype(np.float32)).double()[:, None, :]
        kt = torch.from_numpy(np.repeat(k[b, :, :L], H // KVH, axis=0)).double()
        vt = torch.from_numpy(np.repeat(v[b, :, :L], H // KVH, axis=0)).double()
        ref = F.scaled_dot_product_attention(qt, kt, vt, scale=1.0)[:, 0].numpy()
        assert np.max(np.abs(got[b] - ref)) <= 1e-6


def test_attn_decode_closed_forms():
    rng = np.random.default_rng(5)
    B, H, KVH, P, d = 3, 4, 4, 9, 64
    q = rng.normal(0, 1, (B, H, d)).astype(np.float32)
    v = rng.normal(0, 1, (B, KVH, P, d)).astype(np.float32)
    k = np.broadcast_to(rng.normal(0, 1, d).astype(np.float32), (B, KVH, P, d)).copy()
    out = ollm.attn_decode(q, k, v, [9, 1, 0], 0.125)
    # identical keys: uniform weights, the mean of V
    assert np.allclose(out[0], v[0].mean(axis=1), atol=1e-6)
    # one position: that position's V
    assert np.array_equal(out[1], v[1, :, 0])
    # no positions: zeros
    assert not out[2].any()
