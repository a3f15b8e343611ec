"""Greedy decoding through the plugin is argmax-identical to the oracle model.

A seeded random-init model of the Qwen3 and of the Qwen3.5-hybrid
architecture (head_dim 128; GDN key/value dims 128; bf16 weights) runs the
way the engine would run it with this plugin: every projection through the
ABI v1 `linear` (prepared bf16 weights), attention through
`attention_forward` on a paged bf16 KV pool, GDN through `gdn_forward`, and
the glue the engine computes on the CPU (embedding rows, RMSNorm of the
hidden rows, residual adds, SwiGLU, final norm; src/model/native.rs:249-312,
:526-562) as plain numpy f32.  The oracle is oracle/pymodel.py (bf16 KV
storage, as the plugin stores K/V).  A 40-token prompt, whole and in chunks
of 16 + 16 + 8 (prefill, prefill and verify kernels), then 32 greedy tokens
(decode kernels) with the first maximum winning (src/frontend/sampling.rs:
181-189): the token sequences must be identical.  The logits of every step
are also held to |d| <= 2e-2 + 2e-2 |ref| of the oracle's.
"""
import numpy as np
import pytest

from oracle import pymodel as M

pytestmark = pytest.mark.gpu

PROMPT, STEPS = 40, 32


def gpu_spec(family):
    if family == "qwen3":
        return M.Spec(family="qwen3", hidden=512, intermediate=1024, vocab=1024,
                      layers=["attention"] * 4, heads=4, kv_heads=2, head_dim=128,
                      rotary_dim=128, theta=1e6, tie=False)
    spec = M.Spec(family="qwen35", hidden=512, intermediate=1024, vocab=1024,
                  layers=["gdn", "gdn", "gdn", "attention"], heads=4, kv_heads=2,
                  head_dim=128, rotary_dim=32, theta=1e7, tie=False)
    spec.key_heads, spec.value_heads, spec.key_dim, spec.value_dim = 2, 4, 128, 128
    spec.conv_kernel = 4
    return spec


def _rms(x, w, eps, offset):
    ss = np.mean(x * x, axis=-1, keepdims=True, dtype=np.float32)
    return (x * (np.float32(1.0) / np.sqrt(ss + np.float32(eps)))
            * (w + np.float32(1.0 if offset else 0.0))).astype(np.float32)


def _silu(x):
    return (x / (np.float32(1.0) + np.exp(-x))).astype(np.float32)


class PluginModel:
    """One sequence of `spec`'s model on the plugin."""

    def __init__(self, pkg, backend, spec, w, context):
        self.pkg, self.backend, self.spec, self.w = pkg, backend, spec, w
        self.handles = {}
        for name, x in w.items():
            if x.ndim == 2 and name != "model.embed_tokens.weight":
                bits = (np.ascontiguousarray(x, np.float32).view(np.uint32) >> 16).astype(np.uint16)
                self.handles[name] = backend.create_weight(bits, pkg.DTYPE_BF16)
        self.layers = []
        for kind in spec.layers:
            if kind == "attention":
                pool = pkg.KvCache(backend, spec.kv_heads, spec.head_dim, 16,
                                   context // 16 + 4, context, 1)
            else:
                pool = pkg.GdnState(backend, spec.key_heads, spec.value_heads, spec.key_dim,
                                    spec.value_dim, spec.conv_kernel, 1)
            self.layers.append((pool, pool.open()))
        self.position = 0

    def close(self):
        for pool, _ in self.layers:
            pool.destroy()
        for h in self.handles.values():
            h.destroy()

    def lin(self, name, x):
        y = self.backend.linear(self.handles[f"{name}.weight"], x)
        b = self.w.get(f"{name}.bias")
        return y if b is None else (y + b).astype(np.float32)

    def forward(self, tokens):
        """Logits of the last row after appending `tokens`."""
        s, w, pkg = self.spec, self.w, self.pkg
        rows = len(tokens)
        x = np.ascontiguousarray(w["model.embed_tokens.weight"][np.asarray(tokens)], np.float32)
        pos = np.array([[self.position + i] * 3 for i in range(rows)], np.int32)
        for i, kind in enumerate(s.layers):
            p = f"model.layers.{i}"
            n = _rms(x, w[f"{p}.input_layernorm.weight"], s.eps, s.offset)
            pool, seq = self.layers[i]
            if kind == "attention":
                a = f"{p}.self_attn"
                q, k, v = self.lin(f"{a}.q_proj", n), self.lin(f"{a}.k_proj", n), \
                    self.lin(f"{a}.v_proj", n)
                att = np.zeros((rows, s.heads * s.head_dim), np.float32)
                pkg.attention_forward(self.backend, pool, [seq], [rows], q, k, v, pos, att,
                                      heads=s.heads, kv_heads=s.kv_heads, head_dim=s.head_dim,
                                      rotary_dim=s.rotary_dim, rope_theta=s.theta, eps=s.eps,
                                      q_norm=w.get(f"{a}.q_norm.weight"),
                                      k_norm=w.get(f"{a}.k_norm.weight"), gated=s.gated,
                                      norm_offset=s.offset)
                mixed = self.lin(f"{a}.o_proj", att)
            else:
                g = f"{p}.linear_attn"
                qkv, z = self.lin(f"{g}.in_proj_qkv", n), self.lin(f"{g}.in_proj_z", n)
                a_, b_ = self.lin(f"{g}.in_proj_a", n), self.lin(f"{g}.in_proj_b", n)
                out = np.zeros((rows, s.value_heads * s.value_dim), np.float32)
                conv = np.ascontiguousarray(w[f"{g}.conv1d.weight"].reshape(s.channels, -1))
                pkg.gdn_forward(self.backend, pool, [seq], [rows], qkv, z, a_, b_,
                                w[f"{g}.A_log"], w[f"{g}.dt_bias"], conv, w[f"{g}.norm.weight"],
                                out, eps=s.eps)
                mixed = self.lin(f"{g}.out_proj", out)
            r = (x + mixed).astype(np.float32)
            n2 = _rms(r, w[f"{p}.post_attention_layernorm.weight"], s.eps, s.offset)
            act = (_silu(self.lin(f"{p}.mlp.gate_proj", n2)) * self.lin(f"{p}.mlp.up_proj", n2))
            x = (r + self.lin(f"{p}.mlp.down_proj", act.astype(np.float32))).astype(np.float32)
        self.position += rows
        h = _rms(x[-1:], w["model.norm.weight"], s.eps, s.offset)
        return self.lin("lm_head", h)[0]


def oracle_run(spec, w, prompt):
    st = M.State.new(spec, PROMPT + STEPS + 8, bf16_kv=True)
    logits = M.forward(spec, w, list(prompt), st)[0]
    tokens, all_logits = [], []
    for _ in range(STEPS):
        all_logits.append(logits)
        t = M.argmax(logits)
        tokens.append(t)
        logits = M.forward(spec, w, [t], st)[0]
    return tokens, all_logits


@pytest.mark.parametrize("family", ["qwen3", "qwen35"])
def test_greedy_decode_is_argmax_identical_to_the_oracle(pkg, backend, family):
    spec = gpu_spec(family)
    rng = np.random.default_rng(0x5A5A0007 if family == "qwen3" else 0x5A5A0008)
    w = M.random_weights(spec, rng)
    prompt = [int(t) for t in rng.integers(0, spec.vocab, size=PROMPT)]
    ref_tokens, ref_logits = oracle_run(spec, w, prompt)
    gaps = [float(np.sort(l)[-1] - np.sort(l)[-2]) for l in ref_logits]
    print(f"{family}: oracle tokens {ref_tokens}, smallest top-2 gap {min(gaps):.4f}")
    for chunks in ([PROMPT], [16, 16, 8]):
        model = PluginModel(pkg, backend, spec, w, PROMPT + STEPS + 8)
        try:
            at = 0
            for c in chunks:
                logits = model.forward(prompt[at:at + c])
                at += c
            got, worst = [], 0.0
            for step in range(STEPS):
                ref = ref_logits[step]
                err = np.abs(logits.astype(np.float64) - ref)
                worst = max(worst, float(err.max()))
                assert (err <= 2e-2 + 2e-2 * np.abs(ref)).all(), (
                    f"{family} chunks {chunks}: step {step} logits off by {err.max():.3e}")
                t = M.argmax(logits)
                got.append(t)
                if t != ref_tokens[step]:
                    break
                logits = model.forward([t])
            print(f"{family} chunks {chunks}: largest logit difference {worst:.3e}")
            assert got == ref_tokens, (
                f"{family} chunks {chunks}: tokens differ at step {len(got) - 1} "
                f"(oracle top-2 gap there {gaps[len(got) - 1]:.4f})")
        finally:
            model.close()
