"""Host-side bindings of the MI355X plugin, mirroring the engine's loader.

`NativeBackend.load` follows the reference's `NativeBackend::load`
(src/backend/mod.rs:137-234) step by step: resolve the nine v1 symbols
(`NativeApi::load`, :553-575), require `abi_version() == 1`, create a context
with `{abi_version: 1, struct_size: 16, flags: 0}`, read the capabilities with
`struct_size` pre-filled to 40, reject an ABI or struct-size mismatch, and
reject an empty name.  Errors carry the plugin status and `last_error` text the
way `plugin_error_message` (:593-610) formats them.

`KvCache`, `GdnState`, `attention_forward` and `gdn_forward` bind the optional
extension symbols (include/safetyraise_mi355x.h), which the loader resolves
only when `capabilities.flags` advertises them.  Tensors are numpy arrays
(host memory) or torch tensors on the GPU (device memory, passed with
DEVICE_POINTERS); torch is used only for memory and streams.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path
from typing import Optional, Sequence

import numpy as np

PKG = Path(__file__).resolve().parent
DEFAULT_LIBRARY = PKG / "libsafetyraise_mi355x.so"

ABI_VERSION = 1

# status codes (safetyraise_kernel_status)
STATUS_OK = 0
STATUS_INVALID_ARGUMENT = 1
STATUS_UNSUPPORTED_DTYPE = 2
STATUS_DIMENSION_OVERFLOW = 3
STATUS_OUT_OF_MEMORY = 4
STATUS_DEVICE_ERROR = 5
STATUS_INTERNAL_ERROR = 6
STATUS_ABI_MISMATCH = 7

# dtype numbers (safetyraise_kernel_dtype)
DTYPE_F32, DTYPE_F16, DTYPE_BF16, DTYPE_Q4_0, DTYPE_Q8_0, DTYPE_Q4K, DTYPE_Q6K = range(1, 8)

DEVICE_HOST, DEVICE_CUDA, DEVICE_OTHER = 1, 2, 3

CAP_ATTENTION = 0x1
CAP_GDN = 0x2
CAP_DEVICE_STATE = 0x4

DEVICE_POINTERS = 0x1
ASYNC = 0x2
INPUT_BF16 = 0x4
QK_NORM = 0x8
NORM_OFFSET = 0x10
GATED = 0x20
MROPE_INTERLEAVED = 0x40
KEEP_ROWS = 0x80

V1_SYMBOLS = (
    "safetyraise_kernel_abi_version",
    "safetyraise_kernel_create_context",
    "safetyraise_kernel_destroy_context",
    "safetyraise_kernel_get_capabilities",
    "safetyraise_kernel_create_weight",
    "safetyraise_kernel_destroy_weight",
    "safetyraise_kernel_linear",
    "safetyraise_kernel_last_error",
    "safetyraise_kernel_name",
)

EXTENSION_SYMBOLS = (
    "safetyraise_kernel_set_stream",
    "safetyraise_kernel_synchronize",
    "safetyraise_kernel_kv_create",
    "safetyraise_kernel_kv_destroy",
    "safetyraise_kernel_kv_open",
    "safetyraise_kernel_kv_fork",
    "safetyraise_kernel_kv_close",
    "safetyraise_kernel_kv_truncate",
    "safetyraise_kernel_kv_len",
    "safetyraise_kernel_kv_append",
    "safetyraise_kernel_kv_read",
    "safetyraise_kernel_attention_forward",
    "safetyraise_kernel_attention_forward_noalloc",
    "safetyraise_kernel_gdn_create",
    "safetyraise_kernel_gdn_destroy",
    "safetyraise_kernel_gdn_open",
    "safetyraise_kernel_gdn_fork",
    "safetyraise_kernel_gdn_close",
    "safetyraise_kernel_gdn_read",
    "safetyraise_kernel_gdn_write",
    "safetyraise_kernel_gdn_forward",
    "safetyraise_kernel_gdn_rollback",
    "safetyraise_kernel_linear_device",
    "safetyraise_kernel_timing_enable",
    "safetyraise_kernel_timing_read",
)


class ContextOptions(C.Structure):
    _fields_ = [("abi_version", C.c_uint32), ("struct_size", C.c_uint32), ("flags", C.c_uint64)]


class Capabilities(C.Structure):
    _fields_ = [
        ("abi_version", C.c_uint32),
        ("struct_size", C.c_uint32),
        ("dtype_mask", C.c_uint64),
        ("device_kind", C.c_uint32),
        ("flags", C.c_uint32),
        ("max_rows", C.c_uint64),
        ("max_cols", C.c_uint64),
    ]


class KvOptions(C.Structure):
    _fields_ = [
        ("struct_size", C.c_uint32),
        ("kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32),
        ("page_tokens", C.c_uint32),
        ("num_pages", C.c_uint64),
        ("max_tokens", C.c_uint64),
        ("max_sequences", C.c_uint32),
        ("page_order_seed", C.c_uint32),
    ]


class AttentionArgs(C.Structure):
    _fields_ = [
        ("struct_size", C.c_uint32),
        ("flags", C.c_uint32),
        ("heads", C.c_uint32),
        ("kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32),
        ("rotary_dim", C.c_uint32),
        ("eps", C.c_float),
        ("rope_theta", C.c_float),
        ("mrope_section", C.c_uint32 * 3),
        ("num_seqs", C.c_uint32),
        ("seq_ids", C.POINTER(C.c_uint32)),
        ("seq_rows", C.POINTER(C.c_uint32)),
        ("q", C.c_void_p),
        ("k", C.c_void_p),
        ("v", C.c_void_p),
        ("q_norm", C.c_void_p),
        ("k_norm", C.c_void_p),
        ("positions", C.c_void_p),
        ("out", C.c_void_p),
        ("kv", C.c_void_p),
    ]


class GdnOptions(C.Structure):
    _fields_ = [
        ("struct_size", C.c_uint32),
        ("key_heads", C.c_uint32),
        ("value_heads", C.c_uint32),
        ("key_dim", C.c_uint32),
        ("value_dim", C.c_uint32),
        ("conv_kernel", C.c_uint32),
        ("max_sequences", C.c_uint32),
        ("keep_rows", C.c_uint32),
    ]


class GdnArgs(C.Structure):
    _fields_ = [
        ("struct_size", C.c_uint32),
        ("flags", C.c_uint32),
        ("eps", C.c_float),
        ("num_seqs", C.c_uint32),
        ("seq_ids", C.POINTER(C.c_uint32)),
        ("seq_rows", C.POINTER(C.c_uint32)),
        ("qkv", C.c_void_p),
        ("z", C.c_void_p),
        ("a", C.c_void_p),
        ("b", C.c_void_p),
        ("a_log", C.c_void_p),
        ("dt_bias", C.c_void_p),
        ("conv_weight", C.c_void_p),
        ("norm", C.c_void_p),
        ("out", C.c_void_p),
        ("state", C.c_void_p),
    ]


class PluginError(RuntimeError):
    """A non-zero plugin status, formatted like the engine's WeightError."""

    def __init__(self, status: int, operation: str, message: str = ""):
        detail = f"status {status}: {message}" if message else f"status {status}"
        super().__init__(f"{operation} failed ({detail})")
        self.status = status
        self.message = message


def _declare(lib: C.CDLL) -> None:
    vp, u32, u64, i32 = C.c_void_p, C.c_uint32, C.c_uint64, C.c_int32
    pu32, pu64 = C.POINTER(C.c_uint32), C.POINTER(C.c_uint64)
    sig = {
        "safetyraise_kernel_abi_version": (u32, []),
        "safetyraise_kernel_name": (C.c_char_p, []),
        "safetyraise_kernel_create_context": (i32, [C.POINTER(ContextOptions), C.POINTER(vp)]),
        "safetyraise_kernel_destroy_context": (i32, [vp]),
        "safetyraise_kernel_get_capabilities": (i32, [vp, C.POINTER(Capabilities)]),
        "safetyraise_kernel_create_weight": (i32, [vp, vp, u64, u64, u64, u32, C.POINTER(vp)]),
        "safetyraise_kernel_destroy_weight": (i32, [vp, vp]),
        "safetyraise_kernel_linear": (i32, [vp, vp, vp, u64, u64, vp, u64, u64]),
        "safetyraise_kernel_last_error": (C.c_char_p, [vp]),
        "safetyraise_kernel_set_stream": (i32, [vp, vp]),
        "safetyraise_kernel_synchronize": (i32, [vp]),
        "safetyraise_kernel_kv_create": (i32, [vp, C.POINTER(KvOptions), C.POINTER(vp)]),
        "safetyraise_kernel_kv_destroy": (i32, [vp, vp]),
        "safetyraise_kernel_kv_open": (i32, [vp, vp, pu32]),
        "safetyraise_kernel_kv_fork": (i32, [vp, vp, u32, pu32]),
        "safetyraise_kernel_kv_close": (i32, [vp, vp, u32]),
        "safetyraise_kernel_kv_truncate": (i32, [vp, vp, u32, u64]),
        "safetyraise_kernel_kv_len": (i32, [vp, vp, u32, pu64]),
        "safetyraise_kernel_kv_append": (i32, [vp, vp, u32, vp, vp, u64, u32]),
        "safetyraise_kernel_kv_read": (i32, [vp, vp, u32, u64, u64, vp, vp]),
        "safetyraise_kernel_attention_forward": (i32, [vp, C.POINTER(AttentionArgs)]),
        "safetyraise_kernel_attention_forward_noalloc": (i32, [vp, C.POINTER(AttentionArgs)]),
        "safetyraise_kernel_gdn_create": (i32, [vp, C.POINTER(GdnOptions), C.POINTER(vp)]),
        "safetyraise_kernel_gdn_destroy": (i32, [vp, vp]),
        "safetyraise_kernel_gdn_open": (i32, [vp, vp, pu32]),
        "safetyraise_kernel_gdn_fork": (i32, [vp, vp, u32, pu32]),
        "safetyraise_kernel_gdn_close": (i32, [vp, vp, u32]),
        "safetyraise_kernel_gdn_read": (i32, [vp, vp, u32, vp, vp]),
        "safetyraise_kernel_gdn_write": (i32, [vp, vp, u32, vp, vp]),
        "safetyraise_kernel_gdn_forward": (i32, [vp, C.POINTER(GdnArgs)]),
        "safetyraise_kernel_gdn_rollback": (i32, [vp, vp, u32, u32, u32]),
        "safetyraise_kernel_linear_device": (i32, [vp, vp, vp, u64, u64, vp, u64, u64]),
        "safetyraise_kernel_timing_enable": (i32, [vp, u32]),
        "safetyraise_kernel_timing_read": (i32, [vp, u32, C.POINTER(C.c_char_p), pu64,
                                                 C.POINTER(C.c_double)]),
    }
    for name, (res, args) in sig.items():
        if hasattr(lib, name):
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args


def library_path() -> Path:
    return Path(os.environ.get("SAFETYRAISE_MI355X_LIBRARY", DEFAULT_LIBRARY))


def load_library(path: Optional[os.PathLike] = None) -> C.CDLL:
    """dlopens the plugin; raises if it has not been built (no fallback)."""
    p = Path(path) if path is not None else library_path()
    if not p.exists():
        raise FileNotFoundError(
            f"plugin library {p} is missing: build it with "
            "`python safetyraise-lmengine_amd/build.py` (there is no CPU fallback)")
    lib = C.CDLL(str(p))
    _declare(lib)
    return lib


def _ptr(x) -> Optional[int]:
    """Address of a numpy array (host) or a torch tensor (device)."""
    if x is None:
        return None
    if isinstance(x, np.ndarray):
        if not x.flags.c_contiguous:
            raise ValueError("arrays must be C-contiguous")
        return x.ctypes.data
    if hasattr(x, "data_ptr"):
        if not x.is_contiguous():
            raise ValueError("tensors must be contiguous")
        return x.data_ptr()
    if isinstance(x, int):
        return x
    raise TypeError(f"unsupported buffer type {type(x)!r}")


def _is_device(x) -> bool:
    return x is not None and not isinstance(x, np.ndarray) and getattr(x, "is_cuda", False)


class NativeBackend:
    """Loaded plugin with one resident context (src/backend/mod.rs:137-234)."""

    def __init__(self, lib: C.CDLL, context: int, name: str, caps: Capabilities):
        self.lib = lib
        self.context = C.c_void_p(context)
        self.name = name
        self.capabilities = caps

    @classmethod
    def load(cls, path: Optional[os.PathLike] = None) -> "NativeBackend":
        p = Path(path) if path is not None else library_path()
        lib = C.CDLL(str(p))
        for sym in V1_SYMBOLS:  # NativeApi::load (:553-575)
            if not hasattr(lib, sym):
                raise PluginError(STATUS_ABI_MISMATCH, f"resolving symbol '{sym}'", "missing")
        _declare(lib)
        version = lib.safetyraise_kernel_abi_version()
        if version != ABI_VERSION:
            raise PluginError(STATUS_ABI_MISMATCH, "checking plugin ABI",
                              f"need {ABI_VERSION}, plugin exports {version}")
        opts = ContextOptions(ABI_VERSION, C.sizeof(ContextOptions), 0)
        ctx = C.c_void_p()
        status = lib.safetyraise_kernel_create_context(C.byref(opts), C.byref(ctx))
        if status != STATUS_OK:
            if ctx.value:
                lib.safetyraise_kernel_destroy_context(ctx)
            raise PluginError(status, "creating the plugin context")  # no text (:587-591)
        if not ctx.value:
            raise PluginError(STATUS_INTERNAL_ERROR, "creating the plugin context", "NULL handle")
        caps = Capabilities()
        caps.struct_size = C.sizeof(Capabilities)
        status = lib.safetyraise_kernel_get_capabilities(ctx, C.byref(caps))
        if status != STATUS_OK:
            text = (lib.safetyraise_kernel_last_error(ctx) or b"").decode("utf-8", "replace")
            lib.safetyraise_kernel_destroy_context(ctx)
            raise PluginError(status, "reading plugin capabilities", text)
        if caps.abi_version != ABI_VERSION:
            lib.safetyraise_kernel_destroy_context(ctx)
            raise PluginError(STATUS_ABI_MISMATCH, "checking capability ABI",
                              f"need {ABI_VERSION}, plugin declares {caps.abi_version}")
        if caps.struct_size < C.sizeof(Capabilities):
            lib.safetyraise_kernel_destroy_context(ctx)
            raise PluginError(STATUS_ABI_MISMATCH, "checking capability size",
                              f"need at least {C.sizeof(Capabilities)}, got {caps.struct_size}")
        raw = lib.safetyraise_kernel_name()
        name = raw.decode("utf-8", "replace") if raw is not None else "native"
        if not name:
            lib.safetyraise_kernel_destroy_context(ctx)
            raise PluginError(STATUS_ABI_MISMATCH, "checking plugin name", "empty name")
        return cls(lib, ctx.value, name, caps)

    # -- error handling ---------------------------------------------------
    def check(self, status: int, operation: str) -> None:
        if status != STATUS_OK:
            text = (self.lib.safetyraise_kernel_last_error(self.context) or b"").decode(
                "utf-8", "replace")
            raise PluginError(status, operation, text)

    def supports(self, flag: int) -> bool:
        return bool(self.capabilities.flags & flag)

    def close(self) -> None:
        if self.context is not None and self.context.value:
            self.lib.safetyraise_kernel_destroy_context(self.context)
            self.context = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # -- v1 linear (src/backend/mod.rs:259-333: prepare once, then call) -------
    def create_weight(self, weight: np.ndarray, dtype: int = None) -> "Weight":
        """A device copy of weight[out][cols]: float32 values (dtype F32), or
        uint16 bit patterns with dtype F16 or BF16."""
        w = np.ascontiguousarray(weight)
        if dtype is None:
            dtype = DTYPE_F32
        if dtype == DTYPE_F32:
            w = np.ascontiguousarray(w, dtype=np.float32)
        elif w.dtype != np.uint16:
            raise ValueError("F16/BF16 weights are passed as uint16 bit patterns")
        handle = C.c_void_p()
        self.check(self.lib.safetyraise_kernel_create_weight(
            self.context, w.ctypes.data, w.nbytes, w.shape[0], w.shape[1], dtype,
            C.byref(handle)), "preparing a native weight")
        return Weight(self, handle, w.shape[0], w.shape[1], dtype)

    def linear(self, weight, inputs: np.ndarray, dtype: int = None) -> np.ndarray:
        """inputs [rows][cols] times weight^T; weight is a Weight or an array
        (prepared for this call only)."""
        own = not isinstance(weight, Weight)
        w = self.create_weight(weight, dtype) if own else weight
        try:
            x = np.ascontiguousarray(inputs, dtype=np.float32)
            rows, cols = x.shape
            out = np.zeros((rows, w.rows), dtype=np.float32)
            self.check(self.lib.safetyraise_kernel_linear(
                self.context, w.handle, x.ctypes.data, rows, cols, out.ctypes.data, rows, w.rows),
                "native linear")
            return out
        finally:
            if own:
                w.destroy()

    # -- extension ---------------------------------------------------------
    def set_stream(self, stream_handle: Optional[int]) -> None:
        self.check(self.lib.safetyraise_kernel_set_stream(self.context, stream_handle),
                   "setting the stream")

    def synchronize(self) -> None:
        self.check(self.lib.safetyraise_kernel_synchronize(self.context), "synchronizing")

    def timing(self, enable: bool) -> None:
        """Starts (and clears) or stops recording each kernel launch's device
        duration (hipExtLaunchKernelGGL start/stop events)."""
        self.check(self.lib.safetyraise_kernel_timing_enable(self.context, 1 if enable else 0),
                   "switching kernel timing")

    def kernel_times(self) -> dict:
        """{kernel name: (launches, mean microseconds)} since timing(True)."""
        out = {}
        i = 0
        while True:
            name, n, ms = C.c_char_p(), C.c_uint64(), C.c_double()
            st = self.lib.safetyraise_kernel_timing_read(self.context, i, C.byref(name),
                                                         C.byref(n), C.byref(ms))
            if st != STATUS_OK:
                break
            out[name.value.decode()] = (int(n.value), ms.value * 1e3 / max(int(n.value), 1))
            i += 1
        return out


class Weight:
    """A prepared native weight (create_weight / destroy_weight)."""

    def __init__(self, backend: NativeBackend, handle, rows: int, cols: int, dtype: int):
        self.backend, self.handle, self.rows, self.cols, self.dtype = backend, handle, rows, cols, dtype

    def destroy(self) -> None:
        if self.handle is not None:
            self.backend.check(self.backend.lib.safetyraise_kernel_destroy_weight(
                self.backend.context, self.handle), "destroying a native weight")
            self.handle = None


class KvCache:
    """Paged bf16 KV pool; sequences are slots (PagedKvCache per slot)."""

    def __init__(self, backend: NativeBackend, kv_heads: int, head_dim: int, page_tokens: int,
                 num_pages: int, max_tokens: int, max_sequences: int, page_order_seed: int = 0):
        """page_order_seed != 0 hands pages out in a seeded random order."""
        self.backend = backend
        self.kv_heads, self.head_dim, self.page_tokens = kv_heads, head_dim, page_tokens
        opts = KvOptions(C.sizeof(KvOptions), kv_heads, head_dim, page_tokens, num_pages,
                         max_tokens, max_sequences, page_order_seed)
        handle = C.c_void_p()
        backend.check(backend.lib.safetyraise_kernel_kv_create(backend.context, C.byref(opts),
                                                               C.byref(handle)), "kv_create")
        self.handle = handle

    @property
    def width(self) -> int:
        return self.kv_heads * self.head_dim

    def _call(self, name: str, *args):
        fn = getattr(self.backend.lib, f"safetyraise_kernel_kv_{name}")
        self.backend.check(fn(self.backend.context, self.handle, *args), f"kv_{name}")

    def open(self) -> int:
        out = C.c_uint32()
        self._call("open", C.byref(out))
        return out.value

    def fork(self, seq: int) -> int:
        out = C.c_uint32()
        self._call("fork", seq, C.byref(out))
        return out.value

    def close(self, seq: int) -> None:
        self._call("close", seq)

    def truncate(self, seq: int, length: int) -> None:
        self._call("truncate", seq, length)

    def len(self, seq: int) -> int:
        out = C.c_uint64()
        self._call("len", seq, C.byref(out))
        return out.value

    def append(self, seq: int, keys, values, flags: int = 0) -> None:
        tokens = keys.shape[0]
        if _is_device(keys):
            flags |= DEVICE_POINTERS
        if str(getattr(keys, "dtype", "")).endswith("bfloat16"):
            flags |= INPUT_BF16
        self._call("append", seq, _ptr(keys), _ptr(values), tokens, flags)

    def read(self, seq: int, start: int = 0, tokens: Optional[int] = None):
        if tokens is None:
            tokens = self.len(seq) - start
        k = np.zeros((tokens, self.width), dtype=np.float32)
        v = np.zeros((tokens, self.width), dtype=np.float32)
        self._call("read", seq, start, tokens, k.ctypes.data, v.ctypes.data)
        return k, v

    def destroy(self) -> None:
        if self.handle is not None and self.handle.value:
            self.backend.lib.safetyraise_kernel_kv_destroy(self.backend.context, self.handle)
            self.handle = None


def attention_forward(backend: NativeBackend, kv: KvCache, seq_ids: Sequence[int],
                      seq_rows: Sequence[int], q, k, v, positions, out, *, heads: int,
                      kv_heads: int, head_dim: int, rotary_dim: int, rope_theta: float,
                      eps: float = 1e-6, q_norm=None, k_norm=None, gated: bool = False,
                      norm_offset: bool = False, mrope_section=(0, 0, 0),
                      mrope_interleaved: bool = True, asynchronous: bool = False) -> None:
    """Attention::forward row loop (src/model/native.rs:615-645) for a batch."""
    flags = 0
    if _is_device(q):
        flags |= DEVICE_POINTERS
        if asynchronous:
            flags |= ASYNC
    if str(getattr(q, "dtype", "")).endswith("bfloat16"):
        flags |= INPUT_BF16
    if q_norm is not None:
        flags |= QK_NORM
    if norm_offset:
        flags |= NORM_OFFSET
    if gated:
        flags |= GATED
    if mrope_interleaved:
        flags |= MROPE_INTERLEAVED
    n = len(seq_ids)
    ids = (C.c_uint32 * n)(*seq_ids)
    rows = (C.c_uint32 * n)(*seq_rows)
    args = AttentionArgs()
    args.struct_size = C.sizeof(AttentionArgs)
    args.flags = flags
    args.heads, args.kv_heads, args.head_dim, args.rotary_dim = heads, kv_heads, head_dim, rotary_dim
    args.eps = eps
    args.rope_theta = rope_theta
    args.mrope_section = (C.c_uint32 * 3)(*mrope_section)
    args.num_seqs = n
    args.seq_ids = ids
    args.seq_rows = rows
    args.q, args.k, args.v = _ptr(q), _ptr(k), _ptr(v)
    args.q_norm, args.k_norm = _ptr(q_norm), _ptr(k_norm)
    args.positions = _ptr(positions)
    args.out = _ptr(out)
    args.kv = kv.handle
    backend.check(backend.lib.safetyraise_kernel_attention_forward(backend.context,
                                                                    C.byref(args)),
                  "attention_forward")


class GdnState:
    """Per-sequence GDN recurrent state pool (RecurrentState per slot)."""

    def __init__(self, backend: NativeBackend, key_heads: int, value_heads: int, key_dim: int,
                 value_dim: int, conv_kernel: int, max_sequences: int, keep_rows: int = 0):
        """keep_rows > 0: KEEP_ROWS calls of up to that many rows can be rolled back."""
        self.backend = backend
        self.key_heads, self.value_heads = key_heads, value_heads
        self.key_dim, self.value_dim, self.conv_kernel = key_dim, value_dim, conv_kernel
        self.channels = 2 * key_heads * key_dim + value_heads * value_dim
        opts = GdnOptions(C.sizeof(GdnOptions), key_heads, value_heads, key_dim, value_dim,
                          conv_kernel, max_sequences, keep_rows)
        handle = C.c_void_p()
        backend.check(backend.lib.safetyraise_kernel_gdn_create(backend.context, C.byref(opts),
                                                                C.byref(handle)), "gdn_create")
        self.handle = handle

    def _call(self, name: str, *args):
        fn = getattr(self.backend.lib, f"safetyraise_kernel_gdn_{name}")
        self.backend.check(fn(self.backend.context, self.handle, *args), f"gdn_{name}")

    def open(self) -> int:
        out = C.c_uint32()
        self._call("open", C.byref(out))
        return out.value

    def fork(self, seq: int) -> int:
        out = C.c_uint32()
        self._call("fork", seq, C.byref(out))
        return out.value

    def close(self, seq: int) -> None:
        self._call("close", seq)

    def read(self, seq: int):
        m = np.zeros((self.value_heads, self.value_dim, self.key_dim), dtype=np.float32)
        h = np.zeros((self.channels, self.conv_kernel - 1), dtype=np.float32)
        self._call("read", seq, m.ctypes.data, h.ctypes.data)
        return m, h

    def write(self, seq: int, matrix: np.ndarray, history: np.ndarray) -> None:
        m = np.ascontiguousarray(matrix, dtype=np.float32)
        h = np.ascontiguousarray(history, dtype=np.float32)
        self._call("write", seq, m.ctypes.data, h.ctypes.data)

    def rollback(self, seq: int, rows: int, asynchronous: bool = False) -> None:
        """State and history after the first `rows` rows of the last KEEP_ROWS call."""
        self._call("rollback", seq, rows, ASYNC if asynchronous else 0)

    def destroy(self) -> None:
        if self.handle is not None and self.handle.value:
            self.backend.lib.safetyraise_kernel_gdn_destroy(self.backend.context, self.handle)
            self.handle = None


def gdn_forward(backend: NativeBackend, state: GdnState, seq_ids: Sequence[int],
                seq_rows: Sequence[int], qkv, z, a, b, a_log, dt_bias, conv_weight, norm, out,
                *, eps: float = 1e-6, asynchronous: bool = False, keep_rows: bool = False) -> None:
    """Gdn::forward row loop (src/model/native.rs:720-742) for a batch; keep_rows
    records every row so that GdnState.rollback can return to any of them."""
    flags = KEEP_ROWS if keep_rows else 0
    if _is_device(qkv):
        flags |= DEVICE_POINTERS
        if asynchronous:
            flags |= ASYNC
    if str(getattr(qkv, "dtype", "")).endswith("bfloat16"):
        flags |= INPUT_BF16
    n = len(seq_ids)
    args = GdnArgs()
    args.struct_size = C.sizeof(GdnArgs)
    args.flags = flags
    args.eps = eps
    args.num_seqs = n
    args.seq_ids = (C.c_uint32 * n)(*seq_ids)
    args.seq_rows = (C.c_uint32 * n)(*seq_rows)
    args.qkv, args.z, args.a, args.b = _ptr(qkv), _ptr(z), _ptr(a), _ptr(b)
    args.a_log, args.dt_bias = _ptr(a_log), _ptr(dt_bias)
    args.conv_weight, args.norm = _ptr(conv_weight), _ptr(norm)
    args.out = _ptr(out)
    args.state = state.handle
    backend.check(backend.lib.safetyraise_kernel_gdn_forward(backend.context, C.byref(args)),
                  "gdn_forward")
