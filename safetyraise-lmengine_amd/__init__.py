"""MI355X (gfx950) attention / gated-delta-net backend for the rsinfer plugin ABI.

The product is the C-ABI shared library `libsafetyraise_mi355x.so` built from
`csrc/` (HIP kernels for gfx950 plus the host-side C++ of the plugin).  This
package holds its build script and the Python binding that mirrors the
engine's plugin loader (`plugin.py`).  Import it with
`importlib.import_module("safetyraise-lmengine_amd")`.
"""
from .plugin import (  # noqa: F401
    ASYNC,
    CAP_ATTENTION,
    CAP_DEVICE_STATE,
    CAP_GDN,
    DEVICE_POINTERS,
    DTYPE_BF16,
    DTYPE_F16,
    DTYPE_F32,
    EXTENSION_SYMBOLS,
    GATED,
    INPUT_BF16,
    MROPE_INTERLEAVED,
    NORM_OFFSET,
    QK_NORM,
    V1_SYMBOLS,
    GdnState,
    KvCache,
    NativeBackend,
    PluginError,
    Weight,
    attention_forward,
    gdn_forward,
    library_path,
    load_library,
)
