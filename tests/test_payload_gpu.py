"""Packed graft payloads unpacked on the GPU: bit-exact against the
oracle's law fp16(fp32(code) * scale) (core/graft_quant.py:136-144).

Covered: every packed depth, group sizes on the vector path (32, 64, 128)
and on the one-value path (16, 48), edge scales (fp16 subnormals, overflow
to inf, negative), a payload spanning two upload chunks, the
device-to-device entry, a misaligned output, and plain fp16 payloads
(uploaded as they are, core/graft_arena.py:3479-3492).
"""

import ctypes

import numpy as np
import pytest

import oracle
from graftrepository_amd import _lib, payload as pl

pytestmark = pytest.mark.gpu


def packed(arrays, bits=8, gs=32):
    out = {"format_version": np.asarray(1, np.int64),
           "storage_bits": np.asarray(bits, np.int64),
           "group_size": np.asarray(gs, np.int64)}
    for name, a in arrays.items():
        c, s = oracle.quantize_symmetric(a, bits, gs)
        out[f"{name}_codes"], out[f"{name}_scales"] = c, s
        out[f"{name}_shape"] = np.asarray(a.shape, np.int64)
    return out


@pytest.mark.parametrize("bits,gs", [(8, 32), (6, 32), (4, 64), (3, 128), (2, 32),
                                     (8, 16), (4, 48)])
def test_node_payload_unpacks_bit_exact(hip_lib, bits, gs):
    rng = np.random.default_rng(bits * 1000 + gs)
    d = 96 if gs == 48 else 128
    k = (rng.standard_normal((4, 8, 37, d)) * 3).astype(np.float16)
    v = (rng.standard_normal((4, 8, 37, d)) * 0.01).astype(np.float16)
    z = packed({"k": k, "v": v}, bits, gs)
    out = pl.unpack_node_device(z)
    try:
        for name in ("k", "v"):
            want = oracle.dequant_payload_bits(z[f"{name}_codes"], z[f"{name}_scales"])
            got = out[name].to_host()
            assert got.shape == k.shape
            np.testing.assert_array_equal(got.view(np.uint16), want.reshape(k.shape))
    finally:
        for a in out.values():
            a.close()


def test_edge_scales(hip_lib):
    codes = np.tile(np.arange(-128, 128, dtype=np.int8), 12).reshape(-1, 32)
    scales = np.array([1.0, 0.1, 1e-8, 2.0 ** -24, 9e-8, 300.0, 1000.0, -0.37,
                       65504.0 / 127, 3.0517578e-05, 7.0, 1 / 127] * 8,
                      dtype=np.float32)[:codes.shape[0], None]
    arr = pl.upload_packed(codes, scales, (codes.size,))
    try:
        np.testing.assert_array_equal(arr.to_host().view(np.uint16),
                                      oracle.dequant_payload_bits(codes, scales).reshape(-1))
    finally:
        arr.close()


def test_payload_larger_than_one_upload_chunk(hip_lib):
    rng = np.random.default_rng(9)
    n = (64 << 20) + 32 * 4099                       # two chunks, the second ragged
    codes = rng.integers(-128, 128, size=(n // 32, 32), dtype=np.int8)
    scales = (rng.random((n // 32, 1)) * 0.05).astype(np.float32)
    arr = pl.upload_packed(codes, scales, (n,))
    try:
        got = arr.to_host().view(np.uint16)
        want = oracle.dequant_payload_bits(codes, scales).reshape(-1)
        np.testing.assert_array_equal(got, want)
    finally:
        arr.close()


def test_device_to_device_and_misaligned_output(hip_lib):
    lib = _lib.load()
    rng = np.random.default_rng(10)
    n = 32 * 5000
    codes = rng.integers(-128, 128, size=(n // 32, 32), dtype=np.int8)
    scales = (rng.random((n // 32, 1)) * 2).astype(np.float32)
    want = oracle.dequant_payload_bits(codes, scales).reshape(-1)
    d_c, d_s = ctypes.c_void_p(), ctypes.c_void_p()
    _lib.check(lib.grm_hip_device_alloc(n, ctypes.byref(d_c)), "alloc")
    _lib.check(lib.grm_hip_device_alloc(scales.nbytes, ctypes.byref(d_s)), "alloc")
    out = pl.DeviceArray((n + 8,))
    try:
        _lib.check(lib.grm_hip_copy_to_device(d_c, codes.ctypes.data, n), "h2d")
        _lib.check(lib.grm_hip_copy_to_device(d_s, scales.ctypes.data, scales.nbytes), "h2d")
        ms = ctypes.c_float()
        # aligned output: the eight-values-per-thread kernel
        _lib.check(lib.grm_hip_payload_dequant(d_c, d_s, n, 32, out.ptr, ctypes.byref(ms)),
                   "dequant")
        np.testing.assert_array_equal(out.to_host().view(np.uint16)[:n], want)
        # output 2 bytes off a 16-byte boundary: the one-value kernel
        _lib.check(lib.grm_hip_payload_dequant(d_c, d_s, n, 32, out.ptr + 2, None), "dequant")
        np.testing.assert_array_equal(out.to_host().view(np.uint16)[1:n + 1], want)
        # a group size that does not divide the count is refused
        assert lib.grm_hip_payload_dequant(d_c, d_s, n - 1, 32, out.ptr, None) == -1
    finally:
        out.close()
        lib.grm_hip_device_free(d_c)
        lib.grm_hip_device_free(d_s)


def test_plain_fp16_payload_uploads_unchanged(hip_lib):
    rng = np.random.default_rng(11)
    z = {"c": rng.standard_normal((3, 5, 256)).astype(np.float16),
         "kpe": rng.standard_normal((3, 5, 32)).astype(np.float16)}
    out = pl.unpack_node_device(z, names=("c", "kpe"))
    try:
        for name in ("c", "kpe"):
            np.testing.assert_array_equal(out[name].to_host(), z[name])
        assert out["c"].sub(1) == out["c"].ptr + 5 * 256 * 2
    finally:
        for a in out.values():
            a.close()
