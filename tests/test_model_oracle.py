"""Pins the model oracle (oracle/model.py) before it is used to check the GPU
model runner:
  * RoPE at position 0 is the identity, and it preserves each pair's norm;
  * the first position's attention output is its own V (softmax over one key);
  * an independent float64 Llama forward written with torch library routines
    (F.rms_norm, rotate-half RoPE, F.scaled_dot_product_attention with causal
    mask and grouped KV heads, F.silu) and no fp16 rounding agrees with the
    oracle's logits to within the fp16 rounding noise at every position.
A dropped term (residual, norm weight), a wrong RoPE pairing, a wrong GQA
head mapping or a non-causal mask each fail the last check by far more."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import model as om

CFG = om.ModelConfig(hidden_size=128, intermediate_size=256, layer_count=2, attention_head_count=4,
                     kv_head_count=2, head_dimension=32, vocabulary_size=96, max_position_embeddings=64)
SEED = 77


def test_rope_identity_and_norm():
    v = om.rounded(np.random.default_rng(0).standard_normal(4 * 32).astype(np.float32))
    assert np.array_equal(om.apply_rope(v, 4, 32, 0, 10000.0), v)
    r = om.apply_rope(v, 4, 32, 9, 10000.0).reshape(4, 2, 16)
    x = v.reshape(4, 2, 16)
    assert np.allclose(np.hypot(r[:, 0], r[:, 1]), np.hypot(x[:, 0], x[:, 1]), rtol=2e-3, atol=2e-3)


def test_seeded_weights_statistics():
    w = om.seeded_weight(SEED, 256, 256, om.weight_row(0, "q"))
    assert abs(float(w.mean())) < 1e-3 and abs(float(w.std()) - 0.02) < 1e-3
    assert not np.array_equal(w, om.seeded_weight(SEED, 256, 256, om.weight_row(0, "k")))


def _torch_logits(ref: om.ReferenceModel, tokens):
    """Float64 Llama forward over the whole sequence, no intermediate rounding."""
    c = ref.cfg
    D, QH, KVH = c.head_dimension, c.attention_head_count, c.kv_head_count
    t = lambda a: torch.from_numpy(np.asarray(a, dtype=np.float64))
    n = len(tokens)
    x = t(ref.embed[np.asarray(tokens)])                                        # [n][H]
    pos = torch.arange(n, dtype=torch.float64)
    inv = c.rope_theta ** (-torch.arange(0, D, 2, dtype=torch.float64) / D)   # [D/2]
    ang = pos[:, None] * inv[None, :]
    cos = torch.cat([ang.cos(), ang.cos()], -1)[None, :, None, :]
    sin = torch.cat([ang.sin(), ang.sin()], -1)[None, :, None, :]

    def rot(v):                                                                 # [1][n][h][D]
        half = torch.cat([-v[..., D // 2:], v[..., :D // 2]], -1)
        return v * cos + half * sin

    for W in ref.layers:
        h = F.rms_norm(x, (c.hidden_size,), weight=t(W["ln1"]), eps=c.rms_norm_epsilon)
        q = rot((h @ t(W["q"]).T).view(1, n, QH, D)).transpose(1, 2)
        k = rot((h @ t(W["k"]).T).view(1, n, KVH, D)).transpose(1, 2)
        v = (h @ t(W["v"]).T).view(1, n, KVH, D).transpose(1, 2)
        a = F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)
        x = x + a.transpose(1, 2).reshape(n, -1) @ t(W["o"]).T
        h = F.rms_norm(x, (c.hidden_size,), weight=t(W["ln2"]), eps=c.rms_norm_epsilon)
        x = x + (F.silu(h @ t(W["gate"]).T) * (h @ t(W["up"]).T)) @ t(W["down"]).T
    h = F.rms_norm(x, (c.hidden_size,), weight=t(ref.final_norm), eps=c.rms_norm_epsilon)
    return (h @ t(ref.head).T).numpy()


def test_oracle_matches_independent_float64_llama():
    ref = om.ReferenceModel(CFG, SEED)
    tokens = [5, 17, 3, 88, 41, 0, 63, 12, 9, 50]
    want = _torch_logits(ref, tokens)
    scale = float(np.abs(want).max())
    for p, tok in enumerate(tokens):
        got = ref.forward(tok, p)
        assert np.max(np.abs(got - want[p])) < 0.004 * scale + 1e-3, p   # measured 4e-4 at scale 0.8


def test_first_position_attention_is_value():
    ref = om.ReferenceModel(CFG, SEED)
    ref.forward(7, 0)
    # One key: every query head's output is its KV head's value row; the
    # first layer's stored V equals W_v . rmsnorm(embedding).
    x = om.rms_norm(ref.embed[7].copy(), ref.layers[0]["ln1"], CFG.rms_norm_epsilon)
    assert np.array_equal(ref.values[0][0], om.matvec(ref.layers[0]["v"], x))
    assert np.array_equal(ref.keys[0][0], om.matvec(ref.layers[0]["k"], x))   # RoPE at 0 is the identity


def test_wrong_structure_is_detected():
    """A planted mistake in the oracle (layer 0's attention output dropped)
    breaks the agreement with the float64 forward."""
    ref = om.ReferenceModel(CFG, SEED)
    tokens = [5, 17, 3, 88]
    want = _torch_logits(ref, tokens)
    # Plant the mistake: drop layer 0's output projection.
    ref.layers[0]["o"] = np.zeros_like(ref.layers[0]["o"])
    got = [ref.forward(tk, p) for p, tk in enumerate(tokens)]
    err = max(float(np.max(np.abs(g - w))) for g, w in zip(got, want))
    assert err > 0.05 * float(np.abs(want).max())


def test_threaded_weight_generation_is_identical():
    cfg = om.ModelConfig(hidden_size=64, intermediate_size=96, layer_count=3, attention_head_count=4,
                         kv_head_count=2, head_dimension=16, vocabulary_size=100, max_position_embeddings=64)
    a, b = om.ReferenceModel(cfg, 11), om.ReferenceModel(cfg, 11, threads=4)
    for la, lb in zip(a.layers, b.layers):
        for k in la:
            assert np.array_equal(la[k], lb[k]), k
    assert np.array_equal(a.embed, b.embed) and np.array_equal(a.head, b.head)
    c = b.fresh()
    assert np.array_equal(b.forward(5, 0), c.forward(5, 0)) and len(b.keys[0]) == 1 and len(c.keys[0]) == 1


def test_span_forward_matches_token_forward():
    """forward_span (a span's rows batched into matrix products, causal
    attention over the span at once) against the token-at-a-time forward on
    the same weights: the logits after every span end agree within fp16
    noise, so do the KV histories (the same values in almost every element,
    the rest one fp16 rounding step apart), and both agree with the
    independent float64 Llama."""
    tokens = [5, 17, 3, 88, 41, 0, 63, 12, 9, 50, 33, 71, 2]
    one = om.ReferenceModel(CFG, SEED)
    per_token = [one.forward(t, p) for p, t in enumerate(tokens)]
    span = one.fresh()
    want64 = _torch_logits(one, tokens)
    scale = float(np.abs(want64).max())
    for a, b in [(0, 4), (4, 9), (9, 10), (10, 13)]:
        got = span.forward_span(tokens[a:b], a)
        assert np.max(np.abs(got - per_token[b - 1])) < 2e-3 * scale, (a, b)
        assert np.max(np.abs(got - want64[b - 1])) < 0.004 * scale + 1e-3, (a, b)
    for l in range(CFG.layer_count):
        for hist_a, hist_b in ((one.keys[l], span.keys[l]), (one.values[l], span.values[l])):
            a, b = np.stack(hist_a), np.stack(hist_b)
            assert a.shape == b.shape
            ulp = np.spacing(np.abs(a).astype(np.float16)).astype(np.float32)
            assert np.all(np.abs(a - b) <= ulp * 1.01)
            assert np.mean(a == b) > 0.97
    # Planted mistakes fail the check: attention that ignores the causal mask
    # (earlier rows attend to later keys, which changes the next layer's keys
    # and so the last row), and RoPE at the span's first position for every row.
    leaky = one.fresh()
    leaky._span_mask = lambda positions, total: np.ones((len(positions), total), dtype=bool)
    assert np.max(np.abs(leaky.forward_span(tokens[:6], 0) - per_token[5])) > 0.02 * scale
    real = om.apply_rope_rows
    try:
        om.apply_rope_rows = lambda v, heads, dim, positions, theta: real(v, heads, dim, positions * 0 + positions[0],
                                                                          theta)
        stuck = one.fresh().forward_span(tokens[:6], 0)
    finally:
        om.apply_rope_rows = real
    # (attention over random small weights is nearly uniform, so RoPE moves the
    # logits little: still twice the agreement bound above)
    assert np.max(np.abs(stuck - per_token[5])) > 4e-3 * scale
