"""Model-level restatement of the reference's NativeModel, for the greedy
argmax-identity check of the plugin.

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker.  Nothing in the
plugin imports, links or runs it.

Restates, over the pinned C primitives of pyoracle:
* NativeModel::embed and forward / forward_embeddings
  (src/model/native.rs:212-312): embedding rows, the blocks on a checkpoint
  that is committed only when the whole chunk succeeds, the final RMSNorm
  (offset for Qwen3.5), logits of the last row or of all rows, positions
  [p; 3] from next_position;
* Block::forward (:526-562): RMSNorm, mixer, residual, RMSNorm, SwiGLU MLP,
  residual;
* Attention::forward (:598-647) through pyoracle.attention_rows (projections
  with the Qwen2 biases, QK-norm, RoPE, KV append, causal attention, gate);
* Gdn::forward (:704-744) through pyoracle.gdn_rows;
* fixtures::tiny (:316-418), the reference's synthetic test weights;
* argmax with the first maximum winning (src/frontend/sampling.rs:181-189).

Projections run through pyoracle.linear (the reference plugin's sequential
f32 sum).  `bf16_kv=True` stores appended K/V rounded to bf16, as the plugin
does; the reference keeps f32 (src/engine/state.rs:12-16).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional

import numpy as np

from . import pyoracle as O


@dataclass
class Spec:
    """The ModelSpec fields the forward path reads (src/model/spec.rs)."""
    family: str                 # "qwen2", "qwen3" or "qwen35"
    hidden: int
    intermediate: int
    vocab: int
    layers: List[str]           # "attention" or "gdn" per layer
    heads: int
    kv_heads: int
    head_dim: int
    rotary_dim: int
    theta: float
    eps: float = 1e-6
    mrope_section: Optional[List[int]] = None
    interleaved: bool = True
    key_heads: int = 0
    value_heads: int = 0
    key_dim: int = 0
    value_dim: int = 0
    conv_kernel: int = 0
    tie: bool = True
    max_position: int = 1 << 20

    @property
    def gated(self) -> bool:      # native.rs:607, Qwen3.5 output gate
        return self.family == "qwen35"

    @property
    def offset(self) -> bool:     # native.rs:534, norms weight + 1 for Qwen3.5
        return self.family == "qwen35"

    @property
    def qk_norm(self) -> bool:    # native.rs:572
        return self.family != "qwen2"

    @property
    def bias(self) -> bool:       # native.rs:573
        return self.family == "qwen2"

    @property
    def channels(self) -> int:
        return 2 * self.key_heads * self.key_dim + self.value_heads * self.value_dim


@dataclass
class GdnLayerState:
    matrix: np.ndarray   # [Hv][Dv][Dk] (state.rs:131)
    history: np.ndarray  # [C][K-1] (state.rs:133)


@dataclass
class State:
    """SequenceState: one KV cache or recurrent state per layer (state.rs:137-224)."""
    layers: list
    len: int = 0
    next_position: int = 0
    last_hidden: Optional[np.ndarray] = None

    @classmethod
    def new(cls, spec: Spec, context: int, bf16_kv: bool = False) -> "State":
        layers = []
        for kind in spec.layers:
            if kind == "attention":
                layers.append(O.KvCache(spec.kv_heads * spec.head_dim, context, 64, bf16=bf16_kv))
            else:
                layers.append(GdnLayerState(
                    np.zeros((spec.value_heads, spec.value_dim, spec.key_dim), np.float32),
                    np.zeros((spec.channels, spec.conv_kernel - 1), np.float32)))
        return cls(layers)

    def checkpoint(self) -> "State":  # state.rs:222-224
        layers = [l.clone() if isinstance(l, O.KvCache)
                  else GdnLayerState(l.matrix.copy(), l.history.copy()) for l in self.layers]
        last = None if self.last_hidden is None else self.last_hidden.copy()
        return State(layers, self.len, self.next_position, last)


def _linear(w: Dict[str, np.ndarray], name: str, x: np.ndarray) -> np.ndarray:
    """Projection::forward (native.rs:137-153): backend linear, then the bias."""
    y = O.linear(x, np.ascontiguousarray(w[f"{name}.weight"], np.float32), 1)
    bias = w.get(f"{name}.bias")
    if bias is not None:
        y = (y + bias.astype(np.float32)).astype(np.float32)
    return y


def _attention(spec: Spec, w, p: str, x, positions, cache) -> np.ndarray:
    q = _linear(w, f"{p}.self_attn.q_proj", x)
    k = _linear(w, f"{p}.self_attn.k_proj", x)
    v = _linear(w, f"{p}.self_attn.v_proj", x)
    qn = w.get(f"{p}.self_attn.q_norm.weight") if spec.qk_norm else None
    kn = w.get(f"{p}.self_attn.k_norm.weight") if spec.qk_norm else None
    att = O.attention_rows(q, k, v, positions, cache, heads=spec.heads, kv_heads=spec.kv_heads,
                           dim=spec.head_dim, rotary_dim=spec.rotary_dim, theta=spec.theta,
                           eps=spec.eps, q_norm=qn, k_norm=kn, gated=spec.gated,
                           mrope_section=spec.mrope_section, interleaved=spec.interleaved)
    return _linear(w, f"{p}.self_attn.o_proj", att)


def _gdn(spec: Spec, w, p: str, x, st: GdnLayerState) -> np.ndarray:
    a_ = f"{p}.linear_attn"
    qkv = _linear(w, f"{a_}.in_proj_qkv", x)
    z = _linear(w, f"{a_}.in_proj_z", x)
    a = _linear(w, f"{a_}.in_proj_a", x)
    b = _linear(w, f"{a_}.in_proj_b", x)
    conv = np.ascontiguousarray(w[f"{a_}.conv1d.weight"], np.float32).reshape(
        spec.channels, spec.conv_kernel)
    mixed = O.gdn_rows(qkv, z, a, b, w[f"{a_}.A_log"], w[f"{a_}.dt_bias"], conv,
                       spec.conv_kernel, w[f"{a_}.norm.weight"], spec.eps,
                       key_heads=spec.key_heads, value_heads=spec.value_heads,
                       key_dim=spec.key_dim, value_dim=spec.value_dim, history=st.history,
                       state=st.matrix)
    return _linear(w, f"{a_}.out_proj", mixed)


def block(spec: Spec, w, i: int, x: np.ndarray, positions: np.ndarray, st) -> np.ndarray:
    """Block::forward (native.rs:526-562)."""
    p = f"model.layers.{i}"
    normed = O.rms_norm(x, w[f"{p}.input_layernorm.weight"], spec.eps, spec.offset)
    if spec.layers[i] == "attention":
        mixed = _attention(spec, w, p, normed, positions, st)
    else:
        mixed = _gdn(spec, w, p, normed, st)
    residual = (x + mixed).astype(np.float32)
    normed = O.rms_norm(residual, w[f"{p}.post_attention_layernorm.weight"], spec.eps,
                        spec.offset)
    gate = _linear(w, f"{p}.mlp.gate_proj", normed)
    up = _linear(w, f"{p}.mlp.up_proj", normed)
    out = _linear(w, f"{p}.mlp.down_proj", O.silu_mul(gate, up))
    return (residual + out).astype(np.float32)


def embed(spec: Spec, w, tokens) -> np.ndarray:
    """NativeModel::embed (native.rs:212-228)."""
    emb = np.asarray(w["model.embed_tokens.weight"], np.float32)
    if any(int(t) >= spec.vocab for t in tokens):
        raise O.OracleError("input token is not in the vocabulary")
    return np.ascontiguousarray(emb[np.asarray(tokens, np.int64)])


def forward(spec: Spec, w, tokens, state: State, all_logits: bool = False) -> np.ndarray:
    """NativeModel::forward (native.rs:230-247) + forward_embeddings (:249-312).
    Returns the logits ([rows][vocab] with all_logits, else [1][vocab]); the
    state is replaced by the candidate only when the whole chunk succeeds."""
    rows = len(tokens)
    if rows == 0:
        raise O.OracleError("input is empty")
    positions = np.array([[state.next_position + i] * 3 for i in range(rows)], np.int64)
    hidden = embed(spec, w, tokens)
    candidate = state.checkpoint()
    for i in range(len(spec.layers)):
        hidden = block(spec, w, i, hidden, positions, candidate.layers[i])
        if not np.isfinite(hidden).all():
            raise O.OracleError("non-finite activation; state not committed")
    hidden = O.rms_norm(hidden, w["model.norm.weight"], spec.eps, spec.offset)
    head = w["model.embed_tokens.weight"] if spec.tie else w["lm_head.weight"]
    last = hidden[rows - 1:]
    logits = O.linear(hidden if all_logits else last, np.ascontiguousarray(head, np.float32), 1)
    candidate.len += rows
    candidate.next_position = max(int(positions.max()) + 1, state.next_position)
    candidate.last_hidden = last[0].copy()
    state.layers, state.len = candidate.layers, candidate.len
    state.next_position, state.last_hidden = candidate.next_position, candidate.last_hidden
    return logits


def argmax(logits) -> int:
    """sampling.rs:181-189: the first maximum wins."""
    best = 0
    for i in range(1, len(logits)):
        if logits[i] > logits[best]:
            best = i
    return best


def random_weights(spec: Spec, rng: np.random.Generator) -> Dict[str, np.ndarray]:
    """Seeded random-init weights of `spec`'s architecture (names as the
    reference loads them, native.rs:155-200, :482-526, :565-597, :650-702).
    Matrices ~N(0, 1/fan_in), embeddings ~N(0, 1), norm weights 1 + N(0, 0.1)
    (N(0, 0.1) for Qwen3.5's offset norms); every value is rounded to bf16,
    so a bf16 copy of a matrix widens back to exactly these values."""
    w: Dict[str, np.ndarray] = {}

    def put(name, shape, scale, mean=0.0):
        x = (mean + scale * rng.standard_normal(shape)).astype(np.float32)
        w[name] = O.bf16_round(x)

    norm_mean = 0.0 if spec.offset else 1.0
    put("model.embed_tokens.weight", (spec.vocab, spec.hidden), 1.0)
    if not spec.tie:
        put("lm_head.weight", (spec.vocab, spec.hidden), spec.hidden ** -0.5)
    put("model.norm.weight", (spec.hidden,), 0.1, norm_mean)
    q_width = spec.heads * spec.head_dim
    kv_width = spec.kv_heads * spec.head_dim
    for i, kind in enumerate(spec.layers):
        p = f"model.layers.{i}"
        for name in ("input_layernorm", "post_attention_layernorm"):
            put(f"{p}.{name}.weight", (spec.hidden,), 0.1, norm_mean)
        put(f"{p}.mlp.gate_proj.weight", (spec.intermediate, spec.hidden), spec.hidden ** -0.5)
        put(f"{p}.mlp.up_proj.weight", (spec.intermediate, spec.hidden), spec.hidden ** -0.5)
        put(f"{p}.mlp.down_proj.weight", (spec.hidden, spec.intermediate),
            spec.intermediate ** -0.5)
        if kind == "attention":
            a = f"{p}.self_attn"
            put(f"{a}.q_proj.weight", (q_width * (2 if spec.gated else 1), spec.hidden),
                spec.hidden ** -0.5)
            put(f"{a}.k_proj.weight", (kv_width, spec.hidden), spec.hidden ** -0.5)
            put(f"{a}.v_proj.weight", (kv_width, spec.hidden), spec.hidden ** -0.5)
            put(f"{a}.o_proj.weight", (spec.hidden, q_width), q_width ** -0.5)
            if spec.bias:
                for name, n in (("q_proj", q_width), ("k_proj", kv_width), ("v_proj", kv_width)):
                    put(f"{a}.{name}.bias", (n,), 0.1)
            if spec.qk_norm:
                put(f"{a}.q_norm.weight", (spec.head_dim,), 0.1, norm_mean)
                put(f"{a}.k_norm.weight", (spec.head_dim,), 0.1, norm_mean)
        else:
            g = f"{p}.linear_attn"
            width = spec.value_heads * spec.value_dim
            put(f"{g}.in_proj_qkv.weight", (spec.channels, spec.hidden), spec.hidden ** -0.5)
            put(f"{g}.in_proj_z.weight", (width, spec.hidden), spec.hidden ** -0.5)
            put(f"{g}.in_proj_a.weight", (spec.value_heads, spec.hidden), spec.hidden ** -0.5)
            put(f"{g}.in_proj_b.weight", (spec.value_heads, spec.hidden), spec.hidden ** -0.5)
            put(f"{g}.out_proj.weight", (spec.hidden, width), width ** -0.5)
            put(f"{g}.conv1d.weight", (spec.channels, 1, spec.conv_kernel),
                spec.conv_kernel ** -0.5)
            put(f"{g}.A_log", (spec.value_heads,), 0.5)
            put(f"{g}.dt_bias", (spec.value_heads,), 0.5)
            put(f"{g}.norm.weight", (spec.value_dim,), 0.1, 1.0)
    return w


def tiny(family: str):
    """fixtures::tiny (native.rs:316-418): (Spec, weights) of the reference's
    synthetic 2-layer model; weight i of a tensor is ((7i + 3) % 17) / 40 - 0.2
    unless it is a constant."""
    hybrid = family == "qwen35"
    spec = Spec(family=family, hidden=4, intermediate=6, vocab=8,
                layers=["gdn", "attention"] if hybrid else ["attention", "attention"],
                heads=2, kv_heads=1, head_dim=2, rotary_dim=2,
                theta=1e7 if hybrid else 1e6, max_position=128, tie=True)
    if hybrid:
        spec.key_heads, spec.value_heads, spec.key_dim, spec.value_dim = 1, 2, 2, 2
        spec.conv_kernel = 3
    w: Dict[str, np.ndarray] = {}

    def insert(name, shape, constant=None):
        n = int(np.prod(shape))
        if constant is None:
            values = ((np.arange(n) * 7 + 3) % 17).astype(np.float32) / np.float32(40.0) \
                - np.float32(0.2)
        else:
            values = np.full(n, constant, np.float32)
        w[name] = values.astype(np.float32).reshape(shape)

    norm = 0.0 if hybrid else 1.0
    insert("model.embed_tokens.weight", (8, 4))
    insert("model.norm.weight", (4,), norm)
    for i, kind in enumerate(spec.layers):
        p = f"model.layers.{i}"
        for name in ("input_layernorm", "post_attention_layernorm"):
            insert(f"{p}.{name}.weight", (4,), norm)
        for name, out, inp in (("gate_proj", 6, 4), ("up_proj", 6, 4), ("down_proj", 4, 6)):
            insert(f"{p}.mlp.{name}.weight", (out, inp))
        if kind == "attention":
            for name, out, inp in (("q_proj", 8 if hybrid else 4, 4), ("k_proj", 2, 4),
                                   ("v_proj", 2, 4), ("o_proj", 4, 4)):
                insert(f"{p}.self_attn.{name}.weight", (out, inp))
                if family == "qwen2" and name != "o_proj":
                    insert(f"{p}.self_attn.{name}.bias", (out,), 0.02)
            if family != "qwen2":
                for name in ("q_norm", "k_norm"):
                    insert(f"{p}.self_attn.{name}.weight", (2,), norm)
        else:
            for name, out, inp in (("in_proj_qkv", 8, 4), ("in_proj_z", 4, 4),
                                   ("in_proj_a", 2, 4), ("in_proj_b", 2, 4),
                                   ("out_proj", 4, 4)):
                insert(f"{p}.linear_attn.{name}.weight", (out, inp))
            insert(f"{p}.linear_attn.conv1d.weight", (8, 1, 3), 0.2)
            insert(f"{p}.linear_attn.norm.weight", (2,), 1.0)
            insert(f"{p}.linear_attn.A_log", (2,), -0.5)
            insert(f"{p}.linear_attn.dt_bias", (2,), 0.1)
    return spec, w
