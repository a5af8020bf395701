"""The CPU restatement of the decoder-step operations (oracle/model.py), pinned by
properties the mathematics fixes rather than by retyping its formulas."""
import numpy as np
import pytest

from oracle import model as M


def test_rope_properties():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 3, 8))
    np.testing.assert_allclose(M.rope(x, np.zeros(5), 8, 1e6), x, atol=0)          # position 0: identity
    y = M.rope(x, np.arange(5) * 7.0, 8, 1e6)
    n = lambda a: a[..., :4] ** 2 + a[..., 4:] ** 2                                  # each pair keeps its norm
    np.testing.assert_allclose(n(y), n(x), rtol=1e-12)
    a, b = np.arange(5) * 3.0, np.arange(5) * 11.0                                   # rotations compose additively
    np.testing.assert_allclose(M.rope(M.rope(x, a, 8, 1e4), b, 8, 1e4), M.rope(x, a + b, 8, 1e4), atol=1e-12)
    # pair 0 turns by exactly the position (frequency theta^0 = 1)
    e = np.zeros((1, 1, 8)); e[0, 0, 0] = 1.0
    r = M.rope(e, np.array([0.5]), 8, 1e6)
    np.testing.assert_allclose([r[0, 0, 0], r[0, 0, 4]], [np.cos(0.5), np.sin(0.5)], atol=1e-15)


def test_rmsnorm_silu_argmax_properties():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((4, 16)) * 5
    y = M.rmsnorm(x, np.ones(16), 0.0)
    np.testing.assert_allclose(np.sqrt(np.mean(y * y, axis=1)), 1.0, rtol=1e-12)   # unit RMS
    np.testing.assert_allclose(M.rmsnorm(2 * x, np.ones(16), 0.0), y, rtol=1e-12)   # scale invariant
    assert M.silu_mul(np.array([0.0]), np.array([3.0]))[0] == 0.0
    np.testing.assert_allclose(M.silu_mul(np.array([40.0]), np.array([1.0])), [40.0], rtol=1e-15)
    assert M.argmax(np.array([[1.0, 3.0, 3.0, 2.0]]))[0] == 1                     # first of tied maxima
    assert (M.embed_gather(np.eye(3), [2, -1, 5]) == np.array([[0, 0, 1], [0, 0, 0], [0, 0, 0]])).all()


def _tiny(layers=2, Hq=4, Hkv=2, D=8, H=16, I=24, V=50, seed=3, zero=False):
    from types import SimpleNamespace
    cfg = SimpleNamespace(layers=layers, hidden=H, n_heads=Hq, n_kv_heads=Hkv, head_dim=D, inter=I, vocab=V,
                          eps=1e-6, theta=1e4)
    rng = np.random.default_rng(seed)
    f = lambda *s: (0.0 if zero else 0.3) * rng.standard_normal(s).astype(np.float16)
    W = {"embed": rng.standard_normal((V, H)).astype(np.float16).ravel(),
         "norm": (1 + 0.1 * rng.standard_normal(H)).astype(np.float16)}
    for l in range(layers):
        W.update({f"ln1.{l}": np.ones(H, np.float16), f"ln2.{l}": np.ones(H, np.float16),
                  f"wq.{l}": f(Hq * D, H), f"bq.{l}": f(Hq * D), f"wk.{l}": f(Hkv * D, H), f"bk.{l}": f(Hkv * D),
                  f"wv.{l}": f(Hkv * D, H), f"bv.{l}": f(Hkv * D), f"wo.{l}": f(H, Hq * D),
                  f"wg.{l}": f(I, H), f"wu.{l}": f(I, H), f"wd.{l}": f(H, I)})
    return cfg, W


def test_decoder_zero_layers_is_norm_and_tied_head():
    """Zero projections leave the residual stream at the embedding: logits are the
    final RMSNorm of the token's embedding against the tied embedding matrix."""
    cfg, W = _tiny(zero=True)
    tok = np.array([3, 7, 7, 41])
    got = M.decoder_logits(W, cfg, tok)
    E = W["embed"].reshape(cfg.vocab, cfg.hidden).astype(np.float64)
    x = E[tok]
    n = x / np.sqrt(np.mean(x * x, axis=1, keepdims=True) + cfg.eps) * W["norm"].astype(np.float64)
    np.testing.assert_allclose(got, n.astype(np.float16).astype(np.float64) @ E.T, rtol=2e-3, atol=2e-3)


def test_decoder_is_causal():
    """Logits at position i depend on tokens 0..i only (the causal mask)."""
    cfg, W = _tiny()
    a = np.array([5, 9, 13, 2, 30, 11])
    b = a.copy(); b[4:] = [44, 1]
    la, lb = M.decoder_logits(W, cfg, a), M.decoder_logits(W, cfg, b)
    np.testing.assert_array_equal(la[:4], lb[:4])
    assert np.abs(la[4:] - lb[4:]).max() > 1e-3


def test_decoder_grouped_query_equals_repeated_heads():
    """Hq/Hkv = 2 query heads per KV head gives the same logits as MHA whose K/V
    projections repeat each KV head for its query heads (head h uses KV head h // g)."""
    cfg, W = _tiny(Hq=4, Hkv=2)
    cfg_m, Wm = _tiny(Hq=4, Hkv=4)
    Wm = dict(W)
    D, H = cfg.head_dim, cfg.hidden
    for l in range(cfg.layers):
        for n, shape in (("wk", (2, D, H)), ("wv", (2, D, H)), ("bk", (2, D)), ("bv", (2, D))):
            Wm[f"{n}.{l}"] = np.repeat(W[f"{n}.{l}"].reshape(shape), 2, axis=0).reshape(-1, *shape[2:]) \
                if len(shape) == 3 else np.repeat(W[f"{n}.{l}"].reshape(shape), 2, axis=0).ravel()
    tok = np.array([1, 2, 3, 4, 5])
    np.testing.assert_allclose(M.decoder_logits(W, cfg, tok), M.decoder_logits(Wm, cfg_m, tok), rtol=0, atol=0)


def test_decoder_matches_hugging_face_qwen2():
    """The decoder restatement (without its fp16 stores) against the Hugging Face
    Qwen2 forward -- the library behind the reference's token oracle
    (tools/ref_qwen.py) -- on the same random weights: biases on q/k/v only,
    rotate-half RoPE with theta, RMSNorm, SwiGLU, grouped-query attention, tied
    lm_head.  Built from a config offline (no download); the library computes its
    norms and rotary tables in float32, hence the 1e-5 tolerance."""
    torch = pytest.importorskip("torch")
    tf = pytest.importorskip("transformers")
    cfg, W = _tiny(layers=2, Hq=4, Hkv=2, D=8, H=16, I=24, V=50, seed=11)
    for l in range(cfg.layers):  # non-trivial norm weights
        rng = np.random.default_rng(100 + l)
        W[f"ln1.{l}"] = (1 + 0.2 * rng.standard_normal(cfg.hidden)).astype(np.float16)
        W[f"ln2.{l}"] = (1 + 0.2 * rng.standard_normal(cfg.hidden)).astype(np.float16)
    hf_cfg = tf.Qwen2Config(vocab_size=cfg.vocab, hidden_size=cfg.hidden, intermediate_size=cfg.inter,
                            num_hidden_layers=cfg.layers, num_attention_heads=cfg.n_heads,
                            num_key_value_heads=cfg.n_kv_heads, head_dim=cfg.head_dim, rms_norm_eps=cfg.eps,
                            tie_word_embeddings=True,
                            rope_parameters={"rope_type": "default", "rope_theta": cfg.theta},
                            attn_implementation="eager")
    model = tf.Qwen2ForCausalLM(hf_cfg).to(torch.float64).eval()
    t = lambda a, *shape: torch.from_numpy(np.asarray(a, np.float64).reshape(shape))
    H, Hq, Hkv, D, I = cfg.hidden, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.inter
    sd = {"model.embed_tokens.weight": t(W["embed"], cfg.vocab, H), "model.norm.weight": t(W["norm"], H)}
    for l in range(cfg.layers):
        pre = f"model.layers.{l}."
        sd.update({pre + "self_attn.q_proj.weight": t(W[f"wq.{l}"], Hq * D, H),
                   pre + "self_attn.q_proj.bias": t(W[f"bq.{l}"], Hq * D),
                   pre + "self_attn.k_proj.weight": t(W[f"wk.{l}"], Hkv * D, H),
                   pre + "self_attn.k_proj.bias": t(W[f"bk.{l}"], Hkv * D),
                   pre + "self_attn.v_proj.weight": t(W[f"wv.{l}"], Hkv * D, H),
                   pre + "self_attn.v_proj.bias": t(W[f"bv.{l}"], Hkv * D),
                   pre + "self_attn.o_proj.weight": t(W[f"wo.{l}"], H, Hq * D),
                   pre + "mlp.gate_proj.weight": t(W[f"wg.{l}"], I, H),
                   pre + "mlp.up_proj.weight": t(W[f"wu.{l}"], I, H),
                   pre + "mlp.down_proj.weight": t(W[f"wd.{l}"], H, I),
                   pre + "input_layernorm.weight": t(W[f"ln1.{l}"], H),
                   pre + "post_attention_layernorm.weight": t(W[f"ln2.{l}"], H)})
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not unexpected and set(missing) <= {"lm_head.weight"}
    tok = np.array([5, 9, 13, 2, 30, 11, 49, 0, 7])
    with torch.no_grad():
        ref = model(torch.from_numpy(tok)[None]).logits[0].numpy()
    got = M.decoder_logits(W, cfg, tok, round16=False)
    assert np.abs(ref).max() > 1.0
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)
    # the GPU-shaped form (fp16 stores) stays within fp16 rounding of it
    np.testing.assert_allclose(M.decoder_logits(W, cfg, tok), ref, rtol=0, atol=0.05)
