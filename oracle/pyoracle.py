"""ctypes wrapper of the C oracle (oracle/sr_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker and the timed CPU baseline.
Nothing in the plugin imports, links or runs it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path
from typing import Optional, Sequence

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libsr_oracle.so"
REF_PLUGIN = HERE / "_ref" / "libsafetyraise_cpu.so"

_lib: Optional[C.CDLL] = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(dtype=np.int64, flags="C_CONTIGUOUS")


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE), "all"], check=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = C.CDLL(str(LIB_PATH))
        sz, vp, i, f = C.c_size_t, C.c_void_p, C.c_int, C.c_float
        opt_f32 = C.c_void_p
        L.sro_sigmoid.restype = f
        L.sro_sigmoid.argtypes = [f]
        L.sro_silu.restype = f
        L.sro_silu.argtypes = [f]
        L.sro_softplus.restype = f
        L.sro_softplus.argtypes = [f]
        L.sro_bf16_round.restype = f
        L.sro_bf16_round.argtypes = [f]
        L.sro_rms_norm.restype = i
        L.sro_rms_norm.argtypes = [_f32p, sz, _f32p, sz, f, i, _f32p]
        L.sro_apply_rope.restype = i
        L.sro_apply_rope.argtypes = [_f32p, sz, sz, _i64p, f, sz, vp, i]
        L.sro_kv_new.restype = vp
        L.sro_kv_new.argtypes = [sz, sz, sz, i]
        L.sro_kv_free.argtypes = [vp]
        L.sro_kv_clone.restype = vp
        L.sro_kv_clone.argtypes = [vp]
        L.sro_kv_len.restype = sz
        L.sro_kv_len.argtypes = [vp]
        L.sro_kv_append.restype = i
        L.sro_kv_append.argtypes = [vp, _f32p, _f32p]
        L.sro_kv_append_many.restype = i
        L.sro_kv_append_many.argtypes = [vp, _f32p, _f32p, sz]
        L.sro_kv_get.restype = i
        L.sro_kv_get.argtypes = [vp, sz, _f32p, _f32p]
        L.sro_kv_truncate.restype = i
        L.sro_kv_truncate.argtypes = [vp, sz]
        L.sro_causal_attention.restype = i
        L.sro_causal_attention.argtypes = [_f32p, vp, sz, sz, sz, _f32p]
        L.sro_causal_attention_mt.restype = i
        L.sro_causal_attention_mt.argtypes = [_f32p, vp, sz, sz, sz, _f32p, i]
        L.sro_causal_conv_silu.restype = i
        L.sro_causal_conv_silu.argtypes = [_f32p, sz, _f32p, sz, _f32p, _f32p]
        L.sro_gated_delta_step.restype = i
        L.sro_gated_delta_step.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, sz, sz, sz, sz,
                                           _f32p, _f32p]
        L.sro_attention_rows.restype = i
        L.sro_attention_rows.argtypes = [_f32p, _f32p, _f32p, sz, _i64p, sz, sz, sz, i, opt_f32,
                                         opt_f32, f, f, sz, vp, i, vp, _f32p, i]
        L.sro_linear.restype = i
        L.sro_linear.argtypes = [_f32p, sz, sz, vp, C.c_uint32, sz, _f32p]
        L.sro_silu_mul.restype = None
        L.sro_silu_mul.argtypes = [_f32p, _f32p, sz, _f32p]
        L.sro_gdn_rows.restype = i
        L.sro_gdn_rows.argtypes = [_f32p, _f32p, _f32p, _f32p, sz, _f32p, _f32p, _f32p, sz, _f32p,
                                   f, sz, sz, sz, sz, _f32p, _f32p, _f32p]
        L.sro_gdn_rows_mt.restype = i
        L.sro_gdn_rows_mt.argtypes = [_f32p, _f32p, _f32p, _f32p, sz, _f32p, _f32p, _f32p, sz,
                                      _f32p, f, sz, sz, sz, sz, _f32p, _f32p, _f32p, i]
        _lib = L
    return _lib


class OracleError(ValueError):
    pass


def _ok(status: int, what: str) -> None:
    if status != 0:
        raise OracleError(f"{what} rejected its input (status {status})")


def f32(x) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round f32 values to bf16 (nearest even) and widen back to f32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7F800000) == 0x7F800000
    nan &= (u & 0x007FFFFF) != 0
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000)
    r = np.where(nan, (u | 0x00400000) & 0xFFFF0000, r)
    return r.astype(np.uint32).view(np.float32)


def sigmoid(x: float) -> float:
    return lib().sro_sigmoid(x)


def silu(x: float) -> float:
    return lib().sro_silu(x)


def softplus(x: float) -> float:
    return lib().sro_softplus(x)


def rms_norm(x, weight, eps: float, offset: bool) -> np.ndarray:
    x, w = f32(x), f32(weight)
    out = np.empty_like(x)
    _ok(lib().sro_rms_norm(x.ravel(), x.size, w, w.size, eps, int(offset), out.ravel()),
        "rms_norm")
    return out


def apply_rope(x, head_dim: int, position: Sequence[int], theta: float, rotary_dim: int,
               mrope_section=None, interleaved: bool = True) -> np.ndarray:
    v = f32(x).copy()
    pos = np.ascontiguousarray(position, dtype=np.int64)
    sec = None
    if mrope_section is not None:
        sec_arr = np.ascontiguousarray(mrope_section, dtype=np.int64)
        sec = sec_arr.ctypes.data
    _ok(lib().sro_apply_rope(v.ravel(), v.size, head_dim, pos, theta, rotary_dim, sec,
                             int(interleaved)), "apply_rope")
    return v


class KvCache:
    """PagedKvCache restatement (src/engine/state.rs:19-127)."""

    def __init__(self, width: int, max_tokens: int, page_tokens: int = 64, bf16: bool = False,
                 _handle: Optional[int] = None):
        self.width = width
        self.max_tokens = max_tokens
        self.page_tokens = page_tokens
        self.bf16 = bf16
        self.h = _handle if _handle is not None else lib().sro_kv_new(width, max_tokens,
                                                                      page_tokens, int(bf16))
        if not self.h:
            raise OracleError("KV geometry cannot be zero")

    def __del__(self):
        if getattr(self, "h", None):
            lib().sro_kv_free(self.h)
            self.h = None

    def __len__(self) -> int:
        return lib().sro_kv_len(self.h)

    def clone(self) -> "KvCache":
        return KvCache(self.width, self.max_tokens, self.page_tokens, self.bf16,
                       _handle=lib().sro_kv_clone(self.h))

    def append(self, key, value) -> None:
        _ok(lib().sro_kv_append(self.h, f32(key), f32(value)), "kv append")

    def append_many(self, keys, values) -> None:
        k, v = f32(keys), f32(values)
        _ok(lib().sro_kv_append_many(self.h, k.ravel(), v.ravel(), k.shape[0]), "kv append")

    def get(self, token: int):
        k = np.empty(self.width, np.float32)
        v = np.empty(self.width, np.float32)
        _ok(lib().sro_kv_get(self.h, token, k, v), "kv get")
        return k, v

    def truncate(self, n: int) -> None:
        _ok(lib().sro_kv_truncate(self.h, n), "kv truncate")


def causal_attention(query, cache: KvCache, heads: int, kv_heads: int, dim: int,
                     threads: int = 1) -> np.ndarray:
    q = f32(query)
    out = np.empty(heads * dim, np.float32)
    if threads > 1:
        _ok(lib().sro_causal_attention_mt(q.ravel(), cache.h, heads, kv_heads, dim, out, threads),
            "causal_attention")
    else:
        _ok(lib().sro_causal_attention(q.ravel(), cache.h, heads, kv_heads, dim, out),
            "causal_attention")
    return out


def causal_conv_silu(x, weight, kernel: int, history: np.ndarray) -> np.ndarray:
    """Updates `history` (f32, C*(K-1)) in place like the reference."""
    xi = f32(x)
    out = np.empty_like(xi)
    assert history.dtype == np.float32 and history.flags.c_contiguous
    _ok(lib().sro_causal_conv_silu(xi.ravel(), xi.size, f32(weight).ravel(), kernel,
                                   history.reshape(-1), out.ravel()), "causal_conv_silu")
    return out


def gated_delta_step(qkv, a, b, a_log, dt_bias, key_heads, value_heads, key_dim, value_dim,
                     state: np.ndarray) -> np.ndarray:
    out = np.empty(value_heads * value_dim, np.float32)
    assert state.dtype == np.float32 and state.flags.c_contiguous
    _ok(lib().sro_gated_delta_step(f32(qkv).ravel(), f32(a), f32(b), f32(a_log), f32(dt_bias),
                                   key_heads, value_heads, key_dim, value_dim,
                                   state.reshape(-1), out), "gated_delta_step")
    return out


def attention_rows(q_raw, k_raw, v_raw, positions, cache: KvCache, *, heads: int, kv_heads: int,
                   dim: int, rotary_dim: int, theta: float, eps: float = 1e-6, q_norm=None,
                   k_norm=None, gated: bool = False, mrope_section=None,
                   interleaved: bool = True, threads: int = 1) -> np.ndarray:
    q, k, v = f32(q_raw), f32(k_raw), f32(v_raw)
    rows = k.shape[0]
    pos = np.ascontiguousarray(positions, dtype=np.int64).reshape(rows, 3)
    out = np.empty((rows, heads * dim), np.float32)
    qn = f32(q_norm) if q_norm is not None else None
    kn = f32(k_norm) if k_norm is not None else None
    sec = np.ascontiguousarray(mrope_section, dtype=np.int64) if mrope_section is not None else None
    _ok(lib().sro_attention_rows(
        q.ravel(), k.ravel(), v.ravel(), rows, pos.ravel(), heads, kv_heads, dim, int(gated),
        qn.ctypes.data if qn is not None else None, kn.ctypes.data if kn is not None else None,
        eps, theta, rotary_dim, sec.ctypes.data if sec is not None else None, int(interleaved),
        cache.h, out.ravel(), threads), "attention_rows")
    return out


def gdn_rows(qkv, z, a, b, a_log, dt_bias, conv_weight, kernel: int, norm, eps: float, *,
             key_heads: int, value_heads: int, key_dim: int, value_dim: int,
             history: np.ndarray, state: np.ndarray, threads: int = 1) -> np.ndarray:
    q = f32(qkv)
    rows = q.shape[0]
    out = np.empty((rows, value_heads * value_dim), np.float32)
    assert history.dtype == np.float32 and state.dtype == np.float32
    args = (q.ravel(), f32(z).ravel(), f32(a).ravel(), f32(b).ravel(), rows, f32(a_log),
            f32(dt_bias), f32(conv_weight).ravel(), kernel, f32(norm), eps, key_heads,
            value_heads, key_dim, value_dim, history.reshape(-1), state.reshape(-1), out.ravel())
    if threads > 1:
        _ok(lib().sro_gdn_rows_mt(*args, threads), "gdn_rows")
    else:
        _ok(lib().sro_gdn_rows(*args), "gdn_rows")
    return out


def silu_mul(gate, up) -> np.ndarray:
    """silu(gate) * up element-wise (the MLP of Block::forward, native.rs:550-552)."""
    g, u = f32(gate), f32(up)
    assert g.shape == u.shape
    out = np.empty_like(g)
    lib().sro_silu_mul(g.ravel(), u.ravel(), g.size, out.ravel())
    return out


def linear(x, weight_bits: np.ndarray, dtype: int) -> np.ndarray:
    """ABI v1 linear (native/cpu/safetyraise_cpu.c:203-239): x [rows, cols]
    f32 times weight [out, cols]^T.  weight_bits holds the raw weight: float32
    for dtype 1, uint16 bit patterns for dtype 2 (f16) and 3 (bf16)."""
    x = f32(np.atleast_2d(x))
    w = np.ascontiguousarray(weight_bits)
    assert w.ndim == 2 and w.shape[1] == x.shape[1]
    assert w.dtype == (np.float32 if dtype == 1 else np.uint16)
    out = np.zeros((x.shape[0], w.shape[0]), np.float32)
    _ok(lib().sro_linear(x, x.shape[0], x.shape[1], w.ctypes.data, dtype, w.shape[0], out),
        "linear")
    return out
