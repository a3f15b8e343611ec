"""GPU parity of ABI v1 linear (native/cpu/safetyraise_cpu.c:140-239) through the C-ABI.

linear computes output[r][o] = sum_c input[r][c] * weight[o][c] in f32 with
the weight widened exactly from F32, F16 or BF16.  The plugin sums in another
order (f32 MFMA over k blocks, or for bf16 weights x split exactly into three
bf16 parts on the bf16 MFMA, with partial sums per chain and wave), so random
inputs are held to |d| <= 1e-5 * sum_c |input * weight| + 1e-4 * |ref| (the
error bound of a reordered f32 sum scales with the magnitude of the terms, not
of the result), and integer-valued inputs, whose every partial sum is exact in
f32, must match the oracle bit for bit.  Calls with few output tiles split K
over several workgroups whose partial sums a second kernel adds (shapes
(1, 4096, 512), (3, 2001, 100), (5, 1030, 20), the 3072-column device call and
two of the projection shapes do); calls with at least two workgroups per CU
((16, 512, 8192), (32, 130, 4100)) keep two k blocks per register set instead
of four.  A bf16 weight is stored in 16 x 32 tiles padded with zeros, so
shapes whose rows are not a multiple of 16 or columns not a multiple of 32
((9, 1000, 48): vector loads of x with a part-filled last block; 2001, 1030,
3 columns: scalar loads of x) read padding that must add nothing.
"""
import zlib
import ctypes as C

import numpy as np
import pytest

from oracle import pyoracle as O

pytestmark = pytest.mark.gpu

F32, F16, BF16 = 1, 2, 3


@pytest.fixture
def rng(request):
    return np.random.default_rng(zlib.crc32(request.node.name.encode()))


@pytest.fixture(scope="module")
def torch_mod():
    import torch
    return torch


def weight_bits(w: np.ndarray, dtype: int) -> np.ndarray:
    if dtype == F32:
        return np.ascontiguousarray(w, np.float32)
    if dtype == F16:
        return np.ascontiguousarray(w.astype(np.float16).view(np.uint16))
    return np.ascontiguousarray((O.bf16_round(w.astype(np.float32)).view(np.uint32) >> 16)
                                .astype(np.uint16))


def widened(bits: np.ndarray, dtype: int) -> np.ndarray:
    if dtype == F32:
        return bits.astype(np.float64)
    if dtype == F16:
        return bits.view(np.float16).astype(np.float64)
    return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def test_known_answer_capabilities_and_errors(pkg, backend):
    # src/backend/mod.rs:713-724
    caps = backend.capabilities
    assert caps.dtype_mask == (1 << F32) | (1 << F16) | (1 << BF16)
    w = np.array([[1.0, 0.0, -1.0], [2.0, 3.0, 4.0]], np.float32)
    x = np.array([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]], np.float32)
    expected = np.array([[-2.0, 20.0], [-2.0, 47.0]], np.float32)
    prepared = backend.create_weight(w)
    try:
        assert np.array_equal(backend.linear(prepared, x), expected)
        assert np.array_equal(backend.linear(prepared, x), expected)  # the weight is reusable
        with pytest.raises(pkg.PluginError) as err:
            backend.linear(prepared, np.array([[np.nan, 2.0, 3.0]], np.float32))
        assert err.value.status == 1
        with pytest.raises(pkg.PluginError) as err:  # input width != weight cols
            backend.linear(prepared, np.ones((2, 4), np.float32))
        assert err.value.status == 1
    finally:
        prepared.destroy()
    lib, ctx = backend.lib, backend.context
    h = C.c_void_p()
    # byte length that does not match rows * cols * element size
    assert lib.safetyraise_kernel_create_weight(ctx, w.ctypes.data, w.nbytes - 4, 2, 3, F32,
                                                C.byref(h)) == 1
    # a dtype outside the mask
    assert lib.safetyraise_kernel_create_weight(ctx, w.ctypes.data, 6, 2, 3, 4, C.byref(h)) == 2
    assert lib.safetyraise_kernel_destroy_weight(ctx, None) == 1


@pytest.mark.parametrize("dtype", [F32, F16, BF16])
@pytest.mark.parametrize("rows,cols,out", [(1, 4096, 512), (7, 96, 33), (64, 1001, 257),
                                           (17, 3, 5), (40, 130, 16), (3, 2001, 100),
                                           (5, 1030, 20), (16, 512, 8192), (32, 130, 4100),
                                           (9, 1000, 48)])
def test_random_inputs_match_the_oracle(backend, rng, dtype, rows, cols, out):
    x = (2 * rng.standard_normal((rows, cols))).astype(np.float32)
    bits = weight_bits(rng.standard_normal((out, cols)), dtype)
    got = backend.linear(bits, x, dtype)
    ref = O.linear(x, bits, dtype)
    mag = np.abs(x.astype(np.float64)) @ np.abs(widened(bits, dtype)).T
    bad = np.abs(got - ref) > 1e-5 * mag + 1e-4 * np.abs(ref)
    assert not bad.any(), (dtype, rows, cols, out, np.abs(got - ref).max())


@pytest.mark.parametrize("dtype", [F32, F16, BF16])
def test_integer_inputs_are_bit_exact(backend, rng, dtype):
    # every product and partial sum is an integer below 2^24: exact in f32 in
    # any order, so the plugin must equal the reference's sequential sum
    x = rng.integers(-8, 9, size=(21, 515)).astype(np.float32)
    w = rng.integers(-8, 9, size=(70, 515)).astype(np.float32)
    bits = weight_bits(w, dtype)
    assert np.array_equal(backend.linear(bits, x, dtype), O.linear(x, bits, dtype))


@pytest.mark.parametrize("rows,cols,out", [(16, 4096, 12288), (16, 12288, 4096), (16, 4096, 4096),
                                           (16, 4096, 1024)])
def test_projection_shapes_integer_inputs_bit_exact(backend, rng, rows, cols, out):
    # Qwen3-8B's projection shapes at 16 rows cover the ways a call is cut:
    # three output tiles per wave unsplit (gate/up) and with K split over
    # three workgroups (down), one tile per wave unsplit (q/o) and with K
    # split (k/v).  Integer inputs keep every partial sum exact, so any order
    # must equal the reference bit for bit; the second call reuses the
    # partial-sum scratch.
    x = rng.integers(-8, 9, size=(rows, cols)).astype(np.float32)
    w = rng.integers(-8, 9, size=(out, cols)).astype(np.float32)
    bits = weight_bits(w, BF16)
    prepared = backend.create_weight(bits, BF16)
    try:
        ref = O.linear(x, bits, BF16)
        assert np.array_equal(backend.linear(prepared, x), ref)
        x2 = x[::-1].copy()
        assert np.array_equal(backend.linear(prepared, x2), O.linear(x2, bits, BF16))
    finally:
        prepared.destroy()


@pytest.mark.parametrize("rows,cols,out", [(7, 1000, 12010), (9, 12000, 4096)])
def test_multi_tile_plans_with_partial_blocks(backend, rng, rows, cols, out):
    # the plans with 3 (12010 outputs, last workgroup's tiles partly past N)
    # and 4 output tiles per wave (4096 outputs, K split over 4 workgroups),
    # with K not a multiple of 32: the waves' ranges end inside a block, so
    # the masked path reads the zero-padded last block of every tile
    x = (2 * rng.standard_normal((rows, cols))).astype(np.float32)
    bits = weight_bits(rng.standard_normal((out, cols)), BF16)
    got = backend.linear(bits, x, BF16)
    ref = O.linear(x, bits, BF16)
    mag = np.abs(x.astype(np.float64)) @ np.abs(widened(bits, BF16)).T
    bad = np.abs(got - ref) > 1e-5 * mag + 1e-4 * np.abs(ref)
    assert not bad.any(), (rows, cols, out, np.abs(got - ref).max())
    xi = rng.integers(-8, 9, size=(rows, cols)).astype(np.float32)
    wi = weight_bits(rng.integers(-8, 9, size=(out, cols)).astype(np.float32), BF16)
    assert np.array_equal(backend.linear(wi, xi, BF16), O.linear(xi, wi, BF16))


@pytest.mark.parametrize("rows,cols,out", [(256, 64, 8192), (130, 512, 16000), (300, 192, 6000),
                                           (2048, 128, 1024)])
def test_prefill_sized_calls_take_the_tiled_product(backend, rng, rows, cols, out):
    # 64+ rows with K a multiple of 64 on a bf16 weight, with at least 128
    # output tiles of 128 x 128, take the tiled product (x split once per
    # workgroup through LDS): calls with 2048+ outputs the 4-wave form, the
    # 1024-output call the 8-wave one; one, three and eight stage pairs, rows
    # and outputs past the last whole tile; random and integer inputs
    x = (2 * rng.standard_normal((rows, cols))).astype(np.float32)
    bits = weight_bits(rng.standard_normal((out, cols)), BF16)
    got = backend.linear(bits, x, BF16)
    ref = O.linear(x, bits, BF16)
    mag = np.abs(x.astype(np.float64)) @ np.abs(widened(bits, BF16)).T
    bad = np.abs(got - ref) > 1e-5 * mag + 1e-4 * np.abs(ref)
    assert not bad.any(), (rows, cols, out, np.abs(got - ref).max())
    xi = rng.integers(-8, 9, size=(rows, cols)).astype(np.float32)
    wi = weight_bits(rng.integers(-8, 9, size=(out, cols)).astype(np.float32), BF16)
    assert np.array_equal(backend.linear(wi, xi, BF16), O.linear(xi, wi, BF16))


def test_prefill_sized_integer_inputs_bit_exact(backend, rng):
    x = rng.integers(-8, 9, size=(256, 128)).astype(np.float32)
    w = rng.integers(-8, 9, size=(8200, 128)).astype(np.float32)
    bits = weight_bits(w, BF16)
    prepared = backend.create_weight(bits, BF16)
    try:
        assert np.array_equal(backend.linear(prepared, x), O.linear(x, bits, BF16))
        x2 = x[::-1].copy()  # a second call on the same weight
        assert np.array_equal(backend.linear(prepared, x2), O.linear(x2, bits, BF16))
    finally:
        prepared.destroy()


@pytest.mark.parametrize("dtype", [F32, F16])
def test_row_major_weights_on_the_three_tile_plan(backend, rng, dtype):
    # 12288 outputs take the 3-tiles-per-wave plan for f32 and f16 weights
    # too (row-major, widened to f32 on the f32 MFMA); K = 2056 leaves the
    # waves' ranges ending inside a block
    rows, cols, out = 6, 2056, 12288
    x = (2 * rng.standard_normal((rows, cols))).astype(np.float32)
    bits = weight_bits(rng.standard_normal((out, cols)), dtype)
    got = backend.linear(bits, x, dtype)
    ref = O.linear(x, bits, dtype)
    mag = np.abs(x.astype(np.float64)) @ np.abs(widened(bits, dtype)).T
    bad = np.abs(got - ref) > 1e-5 * mag + 1e-4 * np.abs(ref)
    assert not bad.any(), (dtype, np.abs(got - ref).max())


@pytest.mark.parametrize("cols", [256, 3072])  # 3072: K split over workgroups
def test_device_pointer_entry_matches_host_entry(backend, rng, torch_mod, cols):
    torch = torch_mod
    x = rng.standard_normal((9, cols)).astype(np.float32)
    bits = weight_bits(rng.standard_normal((130, cols)), BF16)
    prepared = backend.create_weight(bits, BF16)
    try:
        host = backend.linear(prepared, x)
        dx = torch.from_numpy(x).cuda()
        dy = torch.zeros((9, 130), device="cuda")
        backend.check(backend.lib.safetyraise_kernel_linear_device(
            backend.context, prepared.handle, C.c_void_p(dx.data_ptr()), 9, cols,
            C.c_void_p(dy.data_ptr()), 9, 130), "linear_device")
        backend.synchronize()
        assert np.array_equal(dy.cpu().numpy(), host)
        # the same shape checks as linear
        assert backend.lib.safetyraise_kernel_linear_device(
            backend.context, prepared.handle, C.c_void_p(dx.data_ptr()), 9, cols - 1,
            C.c_void_p(dy.data_ptr()), 9, 130) == 1
    finally:
        prepared.destroy()


def test_device_input_view_not_16_byte_aligned(backend, rng, torch_mod):
    # a device input that starts one float into an allocation (a tensor view):
    # the kernel must not read it with 16-byte vector loads
    torch = torch_mod
    x = rng.integers(-8, 9, size=(6, 264)).astype(np.float32)
    w = rng.integers(-8, 9, size=(40, 264)).astype(np.float32)
    bits = weight_bits(w, BF16)
    prepared = backend.create_weight(bits, BF16)
    try:
        flat = torch.zeros(6 * 264 + 1, device="cuda")
        flat[1:] = torch.from_numpy(x.ravel()).cuda()
        dx = flat[1:]
        assert dx.data_ptr() % 16 == 4
        dy = torch.zeros((6, 40), device="cuda")
        backend.check(backend.lib.safetyraise_kernel_linear_device(
            backend.context, prepared.handle, C.c_void_p(dx.data_ptr()), 6, 264,
            C.c_void_p(dy.data_ptr()), 6, 40), "linear_device")
        backend.synchronize()
        assert np.array_equal(dy.cpu().numpy(), O.linear(x, bits, BF16))
    finally:
        prepared.destroy()


def test_rows_beyond_one_launch_grid(backend, rng):
    # more rows than one launch's grid covers (65535 row tiles of 16): the
    # plugin splits the rows over launches (the reference takes any count)
    rows = 65535 * 16 + 37
    x = rng.integers(-4, 5, size=(rows, 8)).astype(np.float32)
    w = rng.integers(-4, 5, size=(3, 8)).astype(np.float32)
    got = backend.linear(w, x, F32)
    assert np.array_equal(got, O.linear(x, w, F32))


@pytest.mark.parametrize("dtype", [F32, BF16])
def test_weights_without_columns_give_zeros(backend, rng, torch_mod, dtype):
    # K = 0: every output is the empty sum, 0 (the reference's loop over no
    # inputs); rows below and above the tiled product's minimum, device
    # outputs prefilled with NaN, and a host call after a call that left
    # non-zero values in the plugin's output buffer
    torch = torch_mod
    for rows, out in ((5, 300), (100, 3000)):
        empty = weight_bits(np.zeros((out, 0)), dtype)
        prepared = backend.create_weight(empty, dtype)
        try:
            x = np.zeros((rows, 0), np.float32)
            dy = torch.full((rows, out), float("nan"), device="cuda")
            dx = torch.zeros((rows, 1), device="cuda")  # any valid pointer; no input is read
            backend.check(backend.lib.safetyraise_kernel_linear_device(
                backend.context, prepared.handle, C.c_void_p(dx.data_ptr()), rows, 0,
                C.c_void_p(dy.data_ptr()), rows, out), "linear_device")
            backend.synchronize()
            assert np.array_equal(dy.cpu().numpy(), np.zeros((rows, out), np.float32))
            full = weight_bits(rng.standard_normal((out, 64)), dtype)
            backend.linear(full, rng.standard_normal((rows, 64)).astype(np.float32), dtype)
            assert np.array_equal(backend.linear(prepared, x), np.zeros((rows, out), np.float32))
            assert np.array_equal(O.linear(x, empty, dtype), np.zeros((rows, out), np.float32))
        finally:
            prepared.destroy()


@pytest.mark.parametrize("rows,cols,out", [(9, 256, 130), (256, 128, 8200)])
def test_inputs_above_the_bf16_range(backend, rng, torch_mod, rows, cols, out):
    # finite f32 inputs above bf16's largest value (3.3895e38) round to
    # infinity as bf16; the exact three-part split of x takes its first part
    # from x clamped to that value, so products stay finite and exact.  Row
    # tile kernel (9 rows) and the tiled product (256 rows); one large input
    # per row, weights small powers of two times integers, so each output is
    # one exact product (ref rounding) plus ordinary terms
    torch = torch_mod
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    big = np.array([3.3896e38, 3.39e38, 3.4e38, np.finfo(np.float32).max], np.float32)
    col = rng.integers(0, cols, size=rows)
    x[np.arange(rows), col] = big[np.arange(rows) % 4] * np.where(np.arange(rows) % 3, 1, -1)
    w = (rng.integers(-4, 5, size=(out, cols)) / 64.0).astype(np.float32)
    bits = weight_bits(w, BF16)
    prepared = backend.create_weight(bits, BF16)
    try:
        ref = O.linear(x, bits, BF16)
        assert np.isfinite(ref).all()
        host = backend.linear(prepared, x)
        dx = torch.from_numpy(x).cuda()
        dy = torch.zeros((rows, out), device="cuda")
        backend.check(backend.lib.safetyraise_kernel_linear_device(
            backend.context, prepared.handle, C.c_void_p(dx.data_ptr()), rows, cols,
            C.c_void_p(dy.data_ptr()), rows, out), "linear_device")
        backend.synchronize()
        dev = dy.cpu().numpy()
        mag = np.abs(x.astype(np.float64)) @ np.abs(widened(bits, BF16)).T
        for got in (host, dev):
            assert np.isfinite(got).all()
            bad = np.abs(got.astype(np.float64) - ref) > 1e-6 * mag + 1e-4 * np.abs(ref)
            assert not bad.any(), (rows, np.abs(got - ref).max())
    finally:
        prepared.destroy()
