"""The oracle's model-level restatement (oracle/pymodel.py), pinned without a GPU.

* The reference's own invariant test of NativeModel on fixtures::tiny
  (src/model/native.rs:431-455): the logits of 70 tokens in one call equal
  those of calls of 3 tokens (1e-5), and a restored checkpoint reproduces the
  logits and last hidden row of the original.  Qwen2, Qwen3 and Qwen3.5.
* A closed form for the first token of a sequence.  With one cached token the
  softmax has a single weight 1 (math.rs:133-152) and RoPE at position 0 is
  the identity, so every attention head returns its KV head's value row
  (times sigmoid(gate)); a GDN layer starts from zero state and history, so
  its conv is silu(x w[K-1]) and the state is beta v k^T, giving
  beta v (k^.q^)/sqrt(Dk) (math.rs:158-239).  The first token's logits then
  follow from float64 matrix products, norms and residuals, written out
  here without the oracle: a dropped residual, a missing norm offset, a wrong
  q/gate split, key-head mapping or projection order changes them.
"""
import numpy as np
import pytest

from oracle import pymodel as M

FAMILIES = ["qwen2", "qwen3", "qwen35"]


@pytest.mark.parametrize("family", FAMILIES)
def test_tiny_whole_equals_chunked_and_restore(family):
    spec, w = M.tiny(family)
    tokens = [n % 8 for n in range(70)]
    whole = M.State.new(spec, 128)
    expected = M.forward(spec, w, tokens, whole, all_logits=True)
    state = M.State.new(spec, 128)
    actual = np.concatenate([M.forward(spec, w, tokens[i:i + 3], state, all_logits=True)
                             for i in range(0, 70, 3)])
    np.testing.assert_allclose(actual, expected, rtol=0, atol=1e-5)
    saved = state.checkpoint()
    first = M.forward(spec, w, [2, 3], state, all_logits=True)
    restored = saved.checkpoint()
    M.forward(spec, w, [7, 1, 5], restored)
    restored = saved
    repeated = M.forward(spec, w, [2, 3], restored, all_logits=True)
    np.testing.assert_allclose(repeated, first, rtol=0, atol=1e-5)
    np.testing.assert_allclose(restored.last_hidden, state.last_hidden, rtol=0, atol=1e-5)
    assert state.len == 72


def _rms(x, w, eps, offset):
    return x / np.sqrt(np.mean(x * x) + eps) * (w + (1.0 if offset else 0.0))


def _silu(x):
    return x / (1.0 + np.exp(-x))


def first_token_logits(spec, w, token):
    """float64 closed form of the logits of a sequence's first token (the
    family's switches read from its name, native.rs:534, :572-574, :607)."""
    f = lambda name: np.asarray(w[name], np.float64)
    x = f("model.embed_tokens.weight")[token]
    d = spec.head_dim
    offset = gated = spec.family == "qwen35"
    bias = spec.family == "qwen2"
    for i, kind in enumerate(spec.layers):
        p = f"model.layers.{i}"
        n = _rms(x, f(f"{p}.input_layernorm.weight"), spec.eps, offset)
        if kind == "attention":
            a = f"{p}.self_attn"
            q = f(f"{a}.q_proj.weight") @ n
            v = f(f"{a}.v_proj.weight") @ n
            if bias:
                v = v + f(f"{a}.v_proj.bias")
                q = q + f(f"{a}.q_proj.bias")
            group = spec.heads // spec.kv_heads
            att = []
            for h in range(spec.heads):
                kvh = h // group
                o = v[kvh * d:(kvh + 1) * d]
                if gated:
                    gate = q[h * 2 * d + d:(h + 1) * 2 * d]
                    o = o / (1.0 + np.exp(-gate))
                att.append(o)
            mixed = f(f"{a}.o_proj.weight") @ np.concatenate(att)
        else:
            g = f"{p}.linear_attn"
            kd, vd, hk, hv = spec.key_dim, spec.value_dim, spec.key_heads, spec.value_heads
            qkv = f(f"{g}.in_proj_qkv.weight") @ n
            z = f(f"{g}.in_proj_z.weight") @ n
            b = f(f"{g}.in_proj_b.weight") @ n
            conv = f(f"{g}.conv1d.weight").reshape(spec.channels, spec.conv_kernel)
            y = _silu(qkv * conv[:, -1])
            out = []
            for h in range(hv):
                kh = h // (hv // hk)
                qh = y[kh * kd:(kh + 1) * kd]
                kk = y[hk * kd + kh * kd:hk * kd + (kh + 1) * kd]
                vv = y[2 * hk * kd + h * vd:2 * hk * kd + (h + 1) * vd]
                qh = qh / np.sqrt(np.sum(qh * qh) + 1e-6)
                kk = kk / np.sqrt(np.sum(kk * kk) + 1e-6)
                beta = 1.0 / (1.0 + np.exp(-b[h]))
                o = beta * vv * np.dot(kk, qh) / np.sqrt(kd)
                o = _rms(o, f(f"{g}.norm.weight"), spec.eps, False)
                out.append(o * _silu(z[h * vd:(h + 1) * vd]))
            mixed = f(f"{g}.out_proj.weight") @ np.concatenate(out)
        r = x + mixed
        n2 = _rms(r, f(f"{p}.post_attention_layernorm.weight"), spec.eps, offset)
        act = _silu(f(f"{p}.mlp.gate_proj.weight") @ n2) * (f(f"{p}.mlp.up_proj.weight") @ n2)
        x = r + f(f"{p}.mlp.down_proj.weight") @ act
    h = _rms(x, f("model.norm.weight"), spec.eps, offset)
    head = f("model.embed_tokens.weight") if spec.tie else f("lm_head.weight")
    return head @ h


def small_random_spec(family):
    spec = M.Spec(family=family, hidden=32, intermediate=48, vocab=40,
                  layers=["gdn", "attention", "gdn"] if family == "qwen35"
                  else ["attention", "attention"],
                  heads=4, kv_heads=2, head_dim=8, rotary_dim=4 if family == "qwen35" else 8,
                  theta=1e7 if family == "qwen35" else 1e6, tie=False)
    if family == "qwen35":
        spec.key_heads, spec.value_heads, spec.key_dim, spec.value_dim = 2, 4, 8, 8
        spec.conv_kernel = 4
    return spec


@pytest.mark.parametrize("family", FAMILIES)
@pytest.mark.parametrize("weights", ["tiny", "random"])
def test_first_token_matches_the_closed_form(family, weights):
    if weights == "tiny":
        spec, w = M.tiny(family)
    else:
        spec = small_random_spec(family)
        w = M.random_weights(spec, np.random.default_rng(11))
    for token in range(min(spec.vocab, 8)):
        got = M.forward(spec, w, [token], M.State.new(spec, 16))[0]
        exp = first_token_logits(spec, w, token)
        np.testing.assert_allclose(got, exp, rtol=1e-4, atol=1e-5)


def test_argmax_takes_the_first_maximum():
    # sampling.rs:181-189
    assert M.argmax(np.array([1.0, 3.0, 3.0, 2.0], np.float32)) == 1
    assert M.argmax(np.array([5.0], np.float32)) == 0
    assert M.argmax(np.array([-1.0, -1.0], np.float32)) == 0
