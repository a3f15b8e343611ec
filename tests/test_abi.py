"""The C-ABI boundary, checked without a GPU.

* the library exports every symbol include/*.h declares;
* the ctypes mirror of every struct has the C layout (compiled with gcc);
* the v1 loader contract of the engine (src/backend/mod.rs:137-234) holds:
  abi_version 1, a non-empty name, create_context argument checks, and no
  silent host fallback when no GPU is present;
* the loader mirror reproduces the reference C plugin's own known answer
  (src/backend/mod.rs:703-726) when that plugin has been built into
  oracle/_ref from the reference sources.
"""
import ctypes as C
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
INCLUDE = ROOT / "include"


def declared_symbols():
    names = set()
    for header in INCLUDE.glob("*.h"):
        text = header.read_text()
        for m in re.finditer(r"SAFETYRAISE_KERNEL_EXPORT\s+[\w\s\*]+?\b(safetyraise_kernel_\w+)\s*\(",
                             text):
            names.add(m.group(1))
    return names


def test_header_declares_v1_and_extension(pkg):
    names = declared_symbols()
    assert set(pkg.V1_SYMBOLS) <= names
    assert set(pkg.EXTENSION_SYMBOLS) == names - set(pkg.V1_SYMBOLS)


def test_library_exports_every_declared_symbol(pkg):
    lib = pkg.load_library()
    missing = [n for n in sorted(declared_symbols()) if not hasattr(lib, n)]
    assert not missing, f"missing exports: {missing}"


def test_library_exports_nothing_undeclared(pkg):
    out = subprocess.run(["nm", "-D", "--defined-only", str(pkg.library_path())],
                         capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    ours = {n for n in exported if n.startswith("safetyraise_kernel_")}
    assert ours == declared_symbols()


LAYOUT_PROBE = r"""
#include <stddef.h>
#include <stdio.h>
#include "safetyraise_mi355x.h"
#define S(t) printf(#t " %zu\n", sizeof(t));
#define F(t, f) printf(#t "." #f " %zu\n", offsetof(t, f));
int main(void) {
  S(safetyraise_kernel_context_options) S(safetyraise_kernel_capabilities)
  S(safetyraise_kernel_kv_options) S(safetyraise_kernel_attention_args)
  S(safetyraise_kernel_gdn_options) S(safetyraise_kernel_gdn_args)
  F(safetyraise_kernel_capabilities, dtype_mask) F(safetyraise_kernel_capabilities, max_cols)
  F(safetyraise_kernel_kv_options, num_pages) F(safetyraise_kernel_kv_options, max_sequences)
  F(safetyraise_kernel_attention_args, mrope_section) F(safetyraise_kernel_attention_args, seq_ids)
  F(safetyraise_kernel_attention_args, positions) F(safetyraise_kernel_attention_args, kv)
  F(safetyraise_kernel_gdn_args, seq_ids) F(safetyraise_kernel_gdn_args, state)
  return 0;
}
"""


def test_struct_layouts_match_the_header(pkg, tmp_path):
    src = tmp_path / "probe.c"
    src.write_text(LAYOUT_PROBE)
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c11", f"-I{INCLUDE}", str(src), "-o", str(exe)], check=True)
    got = dict(line.rsplit(" ", 1) for line in
               subprocess.run([str(exe)], capture_output=True, text=True, check=True)
               .stdout.splitlines())
    P = pkg.plugin
    sizes = {
        "safetyraise_kernel_context_options": P.ContextOptions,
        "safetyraise_kernel_capabilities": P.Capabilities,
        "safetyraise_kernel_kv_options": P.KvOptions,
        "safetyraise_kernel_attention_args": P.AttentionArgs,
        "safetyraise_kernel_gdn_options": P.GdnOptions,
        "safetyraise_kernel_gdn_args": P.GdnArgs,
    }
    for cname, ct in sizes.items():
        assert int(got[cname]) == C.sizeof(ct), cname
    # the engine's loader requires these exact v1 sizes (src/backend/mod.rs:145-150, :183-194)
    assert C.sizeof(P.ContextOptions) == 16
    assert C.sizeof(P.Capabilities) == 40
    for key, value in got.items():
        if "." in key:
            cname, field = key.split(".")
            assert getattr(sizes[cname], field).offset == int(value), key


def test_v1_entry_points_without_gpu(pkg):
    lib = pkg.load_library()
    assert lib.safetyraise_kernel_abi_version() == 1
    assert lib.safetyraise_kernel_name()  # non-empty (src/backend/mod.rs:198-211)
    P = pkg.plugin
    ctx = C.c_void_p()
    bad = P.ContextOptions(2, 16, 0)
    assert lib.safetyraise_kernel_create_context(C.byref(bad), C.byref(ctx)) == 1
    short = P.ContextOptions(1, 8, 0)
    assert lib.safetyraise_kernel_create_context(C.byref(short), C.byref(ctx)) == 1
    assert lib.safetyraise_kernel_create_context(None, C.byref(ctx)) == 1
    assert lib.safetyraise_kernel_last_error(None)  # NULL context still yields text


def test_no_host_fallback_when_no_gpu(pkg):
    """Without a GPU the plugin refuses to create a context (DEVICE_ERROR)."""
    if Path("/dev/kfd").exists():
        pytest.skip("a GPU is present; the GPU tests cover context creation")
    with pytest.raises(pkg.PluginError) as err:
        pkg.NativeBackend.load()
    assert err.value.status == 5


REF_PLUGIN = ROOT / "oracle" / "_ref" / "libsafetyraise_cpu.so"


@pytest.mark.skipif(not REF_PLUGIN.exists(), reason="reference C plugin not built (oracle/_ref)")
def test_loader_mirror_reproduces_reference_plugin_known_answer(pkg):
    # src/backend/mod.rs:703-726 with the reference's own C plugin
    backend = pkg.NativeBackend.load(REF_PLUGIN)
    try:
        caps = backend.capabilities
        assert caps.device_kind == 1  # HOST
        assert caps.dtype_mask & (1 << 1) and caps.dtype_mask & (1 << 2)
        w = np.array([[1.0, 0.0, -1.0], [2.0, 3.0, 4.0]], np.float32)
        x = np.array([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]], np.float32)
        expected = np.array([[-2.0, 20.0], [-2.0, 47.0]], np.float32)
        assert np.array_equal(backend.linear(w, x), expected)
        assert np.array_equal(backend.linear(w, x), expected)
        with pytest.raises(pkg.PluginError) as err:
            backend.linear(w, np.array([[np.nan, 2.0, 3.0]], np.float32))
        assert err.value.status == 1
    finally:
        backend.close()
