"""Pins the CPU oracle (oracle/sr_oracle.c) before it is trusted as a checker.

Each check is one of: a known answer from the reference's own tests (cited
file:line in the reference repository), a closed form, or an independent f64
brute force written here in numpy.  Tolerances are stated per test.
"""
import ctypes
import ctypes.util
import math
from pathlib import Path

import numpy as np
import pytest

from oracle import pyoracle as O

RNG = np.random.default_rng(0x5A5A0000)


# ---------------------------------------------------------------------------
# f64 brute force (independent of the oracle's code)
# ---------------------------------------------------------------------------

_LIBM = ctypes.CDLL(ctypes.util.find_library("m"))
_LIBM.powf.restype = ctypes.c_float
_LIBM.powf.argtypes = [ctypes.c_float, ctypes.c_float]


def rope_angle_f32(pos: int, i: int, theta: float, rotary_dim: int) -> np.float32:
    """The reference's f32 angle: pos as f32 / theta.powf(2i/rotary_dim) (math.rs:90-91).

    Rust's f32::powf lowers to the C library powf on Linux.  numpy's float32
    power is a different function that is one ulp off for some exponents
    (e.g. 1e6^0.046875), which moves the angle at position 131k by ~0.01 rad;
    so the denominator comes from libm here, as in the reference.
    """
    exponent = np.float32(2 * i) / np.float32(rotary_dim)
    return np.float32(pos) / np.float32(_LIBM.powf(float(theta), float(exponent)))


def bf_rms_norm(x, w, eps, offset):
    x = np.asarray(x, np.float64).reshape(-1, len(w))
    inv = 1.0 / np.sqrt((x * x).mean(axis=1, keepdims=True) + eps)
    return (x * inv * (np.asarray(w, np.float64) + (1.0 if offset else 0.0))).ravel()


def bf_rope(x, head_dim, pos3, theta, rotary_dim, mrope=None, interleaved=True):
    x = np.asarray(x, np.float64).reshape(-1, head_dim).copy()
    half = rotary_dim // 2
    for i in range(half):
        axis = 0
        if mrope is not None:
            if interleaved:
                axis = 1 if (i % 3 == 1 and i < mrope[1] * 3) else (
                    2 if (i % 3 == 2 and i < mrope[2] * 3) else 0)
            else:
                axis = 0 if i < mrope[0] else (1 if i < mrope[0] + mrope[1] else 2)
        a = float(rope_angle_f32(pos3[axis], i, theta, rotary_dim))
        c, s = math.cos(a), math.sin(a)
        l, r = x[:, i].copy(), x[:, i + half].copy()
        x[:, i] = l * c - r * s
        x[:, i + half] = r * c + l * s
    return x.ravel()


def bf_attention(q, keys, values, heads, kv_heads, dim):
    """Two-pass softmax GQA attention in f64; keys/values [tokens][kv_heads*dim]."""
    q = np.asarray(q, np.float64).reshape(heads, dim)
    k = np.asarray(keys, np.float64).reshape(-1, kv_heads, dim)
    v = np.asarray(values, np.float64).reshape(-1, kv_heads, dim)
    out = np.empty((heads, dim))
    g = heads // kv_heads
    for h in range(heads):
        s = k[:, h // g, :] @ q[h] / math.sqrt(dim)
        p = np.exp(s - s.max())
        out[h] = (p[:, None] * v[:, h // g, :]).sum(0) / p.sum()
    return out.ravel()


def bf_gdn_step(qkv, a, b, a_log, dt_bias, hk, hv, dk, dv, state):
    """Delta rule in f64 (decay, predict, correct, read) on state [hv][dv][dk]."""
    qkv = np.asarray(qkv, np.float64)
    kw = hk * dk
    out = np.empty(hv * dv)
    for h in range(hv):
        st = (h // (hv // hk)) * dk
        q = qkv[st:st + dk]
        k = qkv[kw + st:kw + st + dk]
        qh = q / math.sqrt((q * q).sum() + 1e-6)
        kh = k / math.sqrt((k * k).sum() + 1e-6)
        x = float(a[h]) + float(dt_bias[h])
        sp = max(x, 0.0) + math.log1p(math.exp(-abs(x)))
        alpha = math.exp(-math.exp(float(a_log[h])) * sp)
        beta = 1.0 / (1.0 + math.exp(-float(b[h])))
        S = state[h]
        S *= alpha
        pred = S @ kh
        S += np.outer(beta * (qkv[2 * kw + h * dv:2 * kw + (h + 1) * dv] - pred), kh)
        out[h * dv:(h + 1) * dv] = S @ qh / math.sqrt(dk)
    return out


def close(actual, expected, atol, rtol):
    actual = np.asarray(actual, np.float64)
    expected = np.asarray(expected, np.float64)
    err = np.abs(actual - expected)
    assert np.all(err <= atol + rtol * np.abs(expected)), (
        f"max abs {err.max():.3e} (atol {atol}, rtol {rtol})")


# ---------------------------------------------------------------------------
# reference known answers (src/model/math.rs:245-324, src/engine/state.rs tests)
# ---------------------------------------------------------------------------

def test_attention_online_softmax_known_weighted_average():
    # src/model/math.rs:246-253
    kv = O.KvCache(1, 2, 1)
    kv.append([0.0], [2.0])
    kv.append([math.log(2.0)], [8.0])
    out = O.causal_attention([1.0, 0.0], kv, 2, 1, 1)
    assert abs(out[0] - 6.0) < 1e-6
    assert abs(out[1] - 5.0) < 1e-6


def test_delta_rule_decays_before_prediction_and_snapshot_restores():
    # src/model/math.rs:256-292
    state = np.zeros(2, np.float32)
    out = O.gated_delta_step([1.0, 0.0, 1.0, 0.0, 2.0], [0.0], [0.0], [0.0], [0.0], 1, 1, 2, 1,
                             state)
    assert abs(out[0] - 1.0 / math.sqrt(2.0)) < 2e-6
    saved = state.copy()
    out = O.gated_delta_step([1.0, 0.0, 1.0, 0.0, 0.0], [0.0], [0.0], [0.0], [0.0], 1, 1, 2, 1,
                             state)
    assert abs(out[0] - 0.25 / math.sqrt(2.0)) < 2e-6
    assert abs(saved[0] - 1.0) < 2e-6


def test_partial_rope_preserves_tail_and_uses_axis_positions():
    # src/model/math.rs:295-307
    x = O.apply_rope([1.0, 0.0, 7.0, 9.0], 4, [1, 8, 9], 10000.0, 2)
    assert abs(x[0] - math.cos(1.0)) < 1e-6
    assert abs(x[1] - math.sin(1.0)) < 1e-6
    assert list(x[2:]) == [7.0, 9.0]


def test_convolution_retains_only_prior_raw_inputs():
    # src/model/math.rs:310-324
    hist = np.zeros(2, np.float32)
    y = O.causal_conv_silu([2.0], [1.0, 2.0, 3.0], 3, hist)
    assert abs(y[0] - O.silu(6.0)) < 1e-6
    assert list(hist) == [0.0, 2.0]
    y = O.causal_conv_silu([1.0], [1.0, 2.0, 3.0], 3, hist)
    assert abs(y[0] - O.silu(7.0)) < 1e-6
    assert list(hist) == [2.0, 1.0]


def test_kv_snapshot_isolated_across_partial_and_full_page_boundaries():
    # src/engine/state.rs (tests): width 2, max 9 tokens, 4-token pages
    cache = O.KvCache(2, 9, 4)
    for n in range(3):
        cache.append([n, 1.0], [2.0, n])
    saved = cache.clone()
    for n in range(3, 9):
        cache.append([n, 1.0], [2.0, n])
    with pytest.raises(O.OracleError):
        cache.append([1.0, 1.0], [1.0, 1.0])
    cache.truncate(2)
    cache.append([99.0, 99.0], [88.0, 88.0])
    assert list(saved.get(2)[0]) == [2.0, 1.0]
    assert list(cache.get(2)[0]) == [99.0, 99.0]
    with pytest.raises(O.OracleError):
        saved.get(3)
    with pytest.raises(O.OracleError):
        cache.truncate(4)
    cache.truncate(0)
    assert len(cache) == 0


def test_kv_append_rejects_non_finite():
    # src/engine/state.rs:56-58
    cache = O.KvCache(2, 4, 4)
    with pytest.raises(O.OracleError):
        cache.append([float("nan"), 0.0], [0.0, 0.0])
    with pytest.raises(O.OracleError):
        cache.append([0.0, 0.0], [float("inf"), 0.0])
    assert len(cache) == 0


def test_rms_norm_rejects_bad_eps_and_overflow():
    # src/model/math.rs:29-35, :39-41
    with pytest.raises(O.OracleError):
        O.rms_norm([1.0, 2.0], [1.0, 1.0], 0.0, False)
    with pytest.raises(O.OracleError):
        O.rms_norm([3e38, 3e38], [1.0, 1.0], 1e-6, False)


def test_scalar_functions_match_closed_forms():
    for x in (-30.0, -3.5, -1e-3, 0.0, 1e-3, 2.0, 25.0):
        assert abs(O.sigmoid(x) - 1.0 / (1.0 + math.exp(-x))) <= 1e-7
        assert abs(O.silu(x) - x / (1.0 + math.exp(-x))) <= 1e-6 * max(1.0, abs(x))
        assert abs(O.softplus(x) - math.log1p(math.exp(x))) <= 1e-6 * max(1.0, abs(x))


# ---------------------------------------------------------------------------
# legacy vectors of the reference (src/gpu.rs, src/tensor/ops.rs tests)
# ---------------------------------------------------------------------------

def test_qk_rms_norm_rope_vector_pos5():
    # src/gpu.rs:6398-6460: q [3 heads x 4], k [2 x 4], per-head RMSNorm eps 1e-5,
    # RoPE at pos 5 with inverse frequencies [1.0, 0.1].  In the engine's
    # division form (math.rs:90-91) these are theta = 100 with rotary_dim 4.
    q = np.array([0.25, -0.5, 2.0, 1.5, -1.0, 0.75, 0.5, -0.25, 1.25, -1.5, 0.8, 0.1], np.float32)
    k = np.array([0.6, -1.4, 1.0, 0.25, -0.5, 1.1, 0.3, -0.7], np.float32)
    qw = np.array([1.0, 0.5, -0.75, 1.25], np.float32)
    kw = np.array([0.75, -1.0, 1.2, 0.4], np.float32)
    for x, w in ((q, qw), (k, kw)):
        got = O.apply_rope(O.rms_norm(x, w, 1e-5, False), 4, [5, 5, 5], 100.0, 4)
        normed = bf_rms_norm(x, w, 1e-5, False).reshape(-1, 4)
        exp = normed.copy()
        for i, inv_f in enumerate((1.0, 0.1)):
            a = 5 * inv_f
            exp[:, i] = normed[:, i] * math.cos(a) - normed[:, i + 2] * math.sin(a)
            exp[:, i + 2] = normed[:, i] * math.sin(a) + normed[:, i + 2] * math.cos(a)
        close(got, exp.ravel(), 1e-6, 1e-6)  # the GPU test's bar was 1e-4


def _decode_vector_case(q, key, value, num_heads, num_kv_heads, head_dim, max_len, seq_len):
    """Dense [kv_head][max_len][dim] legacy cache -> token rows for the oracle."""
    key = np.asarray(key, np.float32).reshape(num_kv_heads, max_len, head_dim)
    value = np.asarray(value, np.float32).reshape(num_kv_heads, max_len, head_dim)
    rows_k = key[:, :seq_len, :].transpose(1, 0, 2).reshape(seq_len, -1)
    rows_v = value[:, :seq_len, :].transpose(1, 0, 2).reshape(seq_len, -1)
    cache = O.KvCache(num_kv_heads * head_dim, seq_len, 64)
    cache.append_many(rows_k, rows_v)
    got = O.causal_attention(q, cache, num_heads, num_kv_heads, head_dim)
    exp = bf_attention(q, rows_k, rows_v, num_heads, num_kv_heads, head_dim)
    close(got, exp, 1e-6, 1e-5)


def test_decode_gqa_vector_seq3():
    # src/gpu.rs:6525-6582
    key = np.zeros(2 * 5 * 2, np.float32)
    value = np.zeros_like(key)
    key[0:6] = [1, 2, 3, 4, 5, 6]
    key[10:16] = [10, 20, 30, 40, 50, 60]
    value[0:6] = [0.5, 1.5, 2.5, 3.5, 4.5, 5.5]
    value[10:16] = [6, 7, 8, 9, 10, 11]
    q = [0.2, -0.4, 1.0, 0.5, -0.3, 0.7, 0.9, -0.2]
    _decode_vector_case(q, key, value, 4, 2, 2, 5, 3)


def test_decode_gqa_vector_long_2049():
    # src/gpu.rs:6590-6645 (serial-fallback case: 2049 tokens, head_dim 2)
    seq = 2049
    key = np.zeros((seq + 1) * 2, np.float32)
    value = np.zeros_like(key)
    for pos in range(seq):
        key[pos * 2] = ((pos % 17) - 8.0) * 0.01
        key[pos * 2 + 1] = ((pos % 23) - 11.0) * 0.01
        value[pos * 2] = ((pos % 29) - 14.0) * 0.02
        value[pos * 2 + 1] = ((pos % 31) - 15.0) * 0.02
    _decode_vector_case([0.2, -0.4, 0.7, 0.1], key, value, 2, 1, 2, seq + 1, seq)


@pytest.mark.parametrize("seq", [65, 128, 512, 2048])
def test_decode_gqa_vector_parallel(seq):
    # src/gpu.rs:6652-6720 (4 heads / 2 KV heads, head_dim 8)
    nh, nkv, hd = 4, 2, 8
    q = [((i % 13) - 6.0) * 0.03 for i in range(nh * hd)]
    key = np.zeros((nkv, seq, hd), np.float32)
    value = np.zeros_like(key)
    for h in range(nkv):
        for pos in range(seq):
            for d in range(hd):
                key[h, pos, d] = (((pos + d * 3 + h * 5) % 31) - 15.0) * 0.01
                value[h, pos, d] = (((pos * 2 + d * 7 + h * 11) % 37) - 18.0) * 0.015
    _decode_vector_case(q, key.ravel(), value.ravel(), nh, nkv, hd, seq, seq)


def test_gqa_equals_repeated_kv():
    # src/tensor/ops.rs:1130-1160: the GQA head map h -> h / (heads/kv_heads)
    # equals attention over K/V with each KV head repeated group times.
    q4 = np.array([0.1, 0.2, 0.3, 0.4, -0.2, 0.5, 0.7, -0.1, 0.6, 0.2, -0.4, 0.3, 0.9, -0.5, 0.1,
                   0.8], np.float32).reshape(4, 2, 2)  # [heads, rows, dim]
    k = np.array([0.2, -0.1, 0.4, 0.3, -0.2, 0.7, 0.5, 0.6, -0.3, 0.2, 0.8, -0.4],
                 np.float32).reshape(2, 3, 2)
    v = np.array([0.3, 0.1, -0.2, 0.4, 0.7, -0.5, -0.1, 0.8, 0.6, -0.3, 0.2, 0.5],
                 np.float32).reshape(2, 3, 2)
    rows_k = k.transpose(1, 0, 2).reshape(3, 4)
    rows_v = v.transpose(1, 0, 2).reshape(3, 4)
    rep_k = np.repeat(k, 2, axis=0).transpose(1, 0, 2).reshape(3, 8)
    rep_v = np.repeat(v, 2, axis=0).transpose(1, 0, 2).reshape(3, 8)
    gqa = O.KvCache(4, 3, 64)
    gqa.append_many(rows_k, rows_v)
    rep = O.KvCache(8, 3, 64)
    rep.append_many(rep_k, rep_v)
    for r in range(2):
        qrow = q4[:, r, :].ravel()
        a = O.causal_attention(qrow, gqa, 4, 2, 2)
        b = O.causal_attention(qrow, rep, 4, 4, 2)
        close(a, b, 1e-6, 0.0)
        close(a, bf_attention(qrow, rows_k, rows_v, 4, 2, 2), 1e-6, 1e-6)


# ---------------------------------------------------------------------------
# closed forms
# ---------------------------------------------------------------------------

def test_equal_scores_give_mean_of_values():
    cache = O.KvCache(8, 100, 16)
    keys = RNG.standard_normal((37, 8)).astype(np.float32)
    vals = RNG.standard_normal((37, 8)).astype(np.float32)
    cache.append_many(keys, vals)
    out = O.causal_attention(np.zeros(16, np.float32), cache, 4, 2, 4)
    exp = vals.reshape(37, 2, 4).mean(axis=0)
    close(out.reshape(4, 4), np.repeat(exp, 2, axis=0), 1e-6, 1e-5)


def test_single_token_cache_returns_its_value():
    cache = O.KvCache(4, 4, 4)
    v = np.array([1.5, -2.0, 3.25, 0.125], np.float32)
    cache.append(RNG.standard_normal(4), v)
    out = O.causal_attention(RNG.standard_normal(8), cache, 4, 2, 2)
    # heads 0,1 read KV head 0 = v[:2]; heads 2,3 read KV head 1 = v[2:]
    close(out, np.concatenate([v[:2], v[:2], v[2:], v[2:]]), 0.0, 1e-6)


def test_delta_rule_alpha_one_beta_one_orthonormal_keys_accumulates_outer_products():
    hk, hv, dk, dv = 1, 1, 4, 3
    state = np.zeros(hv * dv * dk, np.float32)
    vs = RNG.standard_normal((dk, dv)).astype(np.float32)
    for t in range(dk):
        k = np.zeros(dk, np.float32)
        k[t] = 2.0  # normalised to e_t
        q = np.ones(dk, np.float32)
        qkv = np.concatenate([q, k, vs[t]])
        # a -> softplus(a) ~ 1e-44: alpha == 1.0 in f32; b = 100: beta == 1.0
        O.gated_delta_step(qkv, [-100.0], [100.0], [0.0], [0.0], hk, hv, dk, dv, state)
    S = state.reshape(dv, dk)
    close(S, vs.T, 1e-6, 1e-6)


def test_delta_rule_alpha_zero_resets_state():
    hk, hv, dk, dv = 1, 2, 4, 2
    state = RNG.standard_normal(hv * dv * dk).astype(np.float32)
    qkv = RNG.standard_normal(2 * hk * dk + hv * dv).astype(np.float32)
    b = np.array([0.3, -0.7], np.float32)
    # A_log = 10, a = 10: alpha = exp(-e^10 * softplus(10)) == 0 in f32
    O.gated_delta_step(qkv, [10.0, 10.0], b, [10.0, 10.0], [0.0, 0.0], hk, hv, dk, dv, state)
    k = qkv[dk:2 * dk]
    kh = k / np.sqrt((k.astype(np.float64) ** 2).sum() + 1e-6)
    for h in range(hv):
        beta = 1.0 / (1.0 + math.exp(-float(b[h])))
        v = qkv[2 * dk + h * dv:2 * dk + (h + 1) * dv]
        close(state.reshape(hv, dv, dk)[h], beta * np.outer(v, kh), 1e-6, 1e-5)


def test_bf16_round_matches_torch_rne():
    torch = pytest.importorskip("torch")
    x = np.concatenate([RNG.standard_normal(10000).astype(np.float32) * 100,
                        np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 3.4e38, -1e-40],
                                 np.float32)])
    ours = O.bf16_round(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))
    # and the C oracle's scalar rounding agrees bit for bit
    for xv in x[:200]:
        assert np.float32(O.lib().sro_bf16_round(float(xv))) == ours[list(x).index(xv)]


# ---------------------------------------------------------------------------
# f64 brute force on random inputs
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("gated,offset,rotary,mrope", [
    (False, False, 64, None),
    (True, True, 16, (3, 3, 2)),
])
def test_attention_rows_match_f64_brute_force(gated, offset, rotary, mrope):
    heads, kv_heads, dim, ctx, rows = 8, 2, 64, 40, 5
    width = kv_heads * dim
    cache = O.KvCache(width, 64, 16)
    ck = RNG.standard_normal((ctx, width)).astype(np.float32)
    cv = RNG.standard_normal((ctx, width)).astype(np.float32)
    cache.append_many(ck, cv)
    qw = heads * dim * (2 if gated else 1)
    q = RNG.standard_normal((rows, qw)).astype(np.float32)
    k = RNG.standard_normal((rows, width)).astype(np.float32)
    v = RNG.standard_normal((rows, width)).astype(np.float32)
    gq = (1 + 0.02 * RNG.standard_normal(dim)).astype(np.float32)
    gk = (1 + 0.02 * RNG.standard_normal(dim)).astype(np.float32)
    pos = np.array([[ctx + r, ctx + r + 3, ctx + 2 * r] for r in range(rows)], np.int64)
    out = O.attention_rows(q, k, v, pos, cache, heads=heads, kv_heads=kv_heads, dim=dim,
                           rotary_dim=rotary, theta=1e6, eps=1e-6, q_norm=gq, k_norm=gk,
                           gated=gated, mrope_section=mrope)
    keys, vals = list(ck.astype(np.float64)), list(cv.astype(np.float64))
    for r in range(rows):
        qr = q[r].reshape(heads, -1)
        qq = qr[:, :dim].ravel() if gated else qr.ravel()
        qn = bf_rope(bf_rms_norm(qq, gq, 1e-6, gated), dim, pos[r], 1e6, rotary, mrope)
        kn = bf_rope(bf_rms_norm(k[r], gk, 1e-6, gated), dim, pos[r], 1e6, rotary, mrope)
        keys.append(kn)
        vals.append(v[r].astype(np.float64))
        exp = bf_attention(qn, np.array(keys), np.array(vals), heads, kv_heads, dim)
        if gated:
            g = qr[:, dim:].ravel().astype(np.float64)
            exp = exp / (1.0 + np.exp(-g))
        close(out[r], exp, 2e-5, 2e-5)
    assert len(cache) == ctx + rows


def test_rope_large_positions_use_the_f32_angle():
    # at pos ~131k one f32 ulp of the angle is ~0.008 rad; the oracle must use
    # exactly the f32 angle of math.rs:90-91, not the exact real angle
    dim = 128
    x = RNG.standard_normal(dim).astype(np.float32)
    for pos in (4095, 32768, 131071, 131076):
        got = O.apply_rope(x, dim, [pos, pos, pos], 1e6, dim)
        exp = bf_rope(x, dim, [pos, pos, pos], 1e6, dim)
        close(got, exp, 2e-6, 2e-6)


@pytest.mark.parametrize("hk,hv,dk,dv,K", [(1, 2, 4, 3, 3), (2, 4, 16, 8, 4)])
def test_gdn_rows_match_f64_brute_force(hk, hv, dk, dv, K):
    C = 2 * hk * dk + hv * dv
    rows = 7
    qkv = RNG.standard_normal((rows, C)).astype(np.float32)
    z = RNG.standard_normal((rows, hv * dv)).astype(np.float32)
    a = RNG.standard_normal((rows, hv)).astype(np.float32)
    b = RNG.standard_normal((rows, hv)).astype(np.float32)
    a_log = (0.1 * RNG.standard_normal(hv)).astype(np.float32)
    dt = (0.1 * RNG.standard_normal(hv)).astype(np.float32)
    w = (RNG.standard_normal((C, K)) / 2).astype(np.float32)
    norm = (1 + 0.1 * RNG.standard_normal(dv)).astype(np.float32)
    hist = (0.5 * RNG.standard_normal((C, K - 1))).astype(np.float32)
    state = (0.02 * RNG.standard_normal((hv, dv, dk))).astype(np.float32)
    h64, s64 = hist.astype(np.float64).copy(), state.astype(np.float64).copy()
    out = O.gdn_rows(qkv, z, a, b, a_log, dt, w, K, norm, 1e-6, key_heads=hk, value_heads=hv,
                     key_dim=dk, value_dim=dv, history=hist, state=state)
    for r in range(rows):
        x = qkv[r].astype(np.float64)
        conv = (h64 * w[:, :K - 1]).sum(1) + x * w[:, K - 1]
        conv = conv / (1.0 + np.exp(-conv))
        h64 = np.concatenate([h64[:, 1:], x[:, None]], axis=1)
        o = bf_gdn_step(conv, a[r], b[r], a_log, dt, hk, hv, dk, dv, s64)
        o = bf_rms_norm(o, norm, 1e-6, False)
        zz = z[r].astype(np.float64)
        exp = o * zz / (1.0 + np.exp(-zz))
        close(out[r], exp, 1e-5, 1e-5)
    close(state, s64, 1e-5, 1e-5)
    close(hist, h64, 0.0, 0.0)


@pytest.mark.parametrize("threads", [2, 3, 8])
def test_gdn_rows_threaded_equals_serial_bit_for_bit(threads):
    # the CPU baseline's all-cores GDN figure splits value heads over threads;
    # each head's operations are those of the serial loop, so outputs, state
    # and history are identical
    hk, hv, dk, dv, K, rows = 2, 6, 16, 8, 4, 9
    C = 2 * hk * dk + hv * dv
    qkv = RNG.standard_normal((rows, C)).astype(np.float32)
    z = RNG.standard_normal((rows, hv * dv)).astype(np.float32)
    a = RNG.standard_normal((rows, hv)).astype(np.float32)
    b = RNG.standard_normal((rows, hv)).astype(np.float32)
    a_log = (0.1 * RNG.standard_normal(hv)).astype(np.float32)
    dt = (0.1 * RNG.standard_normal(hv)).astype(np.float32)
    w = (RNG.standard_normal((C, K)) / 2).astype(np.float32)
    norm = (1 + 0.1 * RNG.standard_normal(dv)).astype(np.float32)
    hist = (0.5 * RNG.standard_normal((C, K - 1))).astype(np.float32)
    state = (0.02 * RNG.standard_normal((hv, dv, dk))).astype(np.float32)
    h1, s1, h2, s2 = hist.copy(), state.copy(), hist.copy(), state.copy()
    kw = dict(key_heads=hk, value_heads=hv, key_dim=dk, value_dim=dv)
    o1 = O.gdn_rows(qkv, z, a, b, a_log, dt, w, K, norm, 1e-6, history=h1, state=s1, **kw)
    o2 = O.gdn_rows(qkv, z, a, b, a_log, dt, w, K, norm, 1e-6, history=h2, state=s2,
                    threads=threads, **kw)
    assert np.array_equal(o1, o2) and np.array_equal(s1, s2) and np.array_equal(h1, h2)


# ---------------------------------------------------------------------------
# ABI v1 linear (native/cpu/safetyraise_cpu.c:203-239)
# ---------------------------------------------------------------------------

def test_linear_known_answer_and_non_finite_input():
    # src/backend/mod.rs:713-724
    w = np.array([[1.0, 0.0, -1.0], [2.0, 3.0, 4.0]], np.float32)
    x = np.array([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]], np.float32)
    assert np.array_equal(O.linear(x, w, 1), np.array([[-2.0, 20.0], [-2.0, 47.0]], np.float32))
    with pytest.raises(O.OracleError):
        O.linear(np.array([[np.nan, 2.0, 3.0]], np.float32), w, 1)


@pytest.mark.parametrize("dtype", [2, 3])
def test_linear_widens_every_16_bit_pattern_exactly(dtype):
    # one input of 1.0 against a weight column holding all 65536 patterns:
    # f16 widening is exact (numpy's float16), bf16 widening is the shift
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16).reshape(-1, 1)
    got = O.linear(np.ones((1, 1), np.float32), bits, dtype)[0]
    if dtype == 2:
        want = bits.view(np.float16).astype(np.float32)[:, 0]
    else:
        want = (bits.astype(np.uint32) << 16).view(np.float32)[:, 0]
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], want[~nan])  # 0.0 + (-0.0) is +0.0; == treats them alike


REF_PLUGIN = Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "libsafetyraise_cpu.so"


@pytest.mark.skipif(not REF_PLUGIN.exists(), reason="reference C plugin not built (oracle/_ref)")
@pytest.mark.parametrize("rows,cols,out", [(1, 37, 5), (5, 96, 19), (3, 1, 4)])
def test_linear_matches_the_reference_plugin_bit_for_bit(pkg, rows, cols, out):
    # the reference's own C plugin (built from native/cpu/safetyraise_cpu.c)
    # for the dtypes it supports: f32 and f16
    backend = pkg.NativeBackend.load(REF_PLUGIN)
    try:
        x = (3 * RNG.standard_normal((rows, cols))).astype(np.float32)
        w32 = RNG.standard_normal((out, cols)).astype(np.float32)
        assert np.array_equal(backend.linear(w32, x), O.linear(x, w32, 1))
        w16 = RNG.standard_normal((out, cols)).astype(np.float16).view(np.uint16)
        assert np.array_equal(backend.linear(w16, x, pkg.DTYPE_F16), O.linear(x, w16, 2))
    finally:
        backend.close()
