"""Packed graft payloads on the CPU: the oracle's unpack law pinned by an
independent route, the quantiser's invariants, and the fail-closed format
checks of the device unpack (which run before anything touches a GPU).

Law: core/graft_quant.py:136-144, fp16(fp32(code) * scale).  Quantiser:
:93-131.  Format checks: unpack_kv_arrays :232-268.
"""

import numpy as np
import pytest

import oracle
from graftrepository_amd import payload as pl


def law_via_fp64(codes, scales):
    """The law by another route: the product of an int8 code and an fp32
    scale is exact in fp64.  numpy then rounds it to fp32 and to fp16, both
    to nearest even; the oracle uses its own C conversion instead."""
    exact = codes.astype(np.float64) * scales.astype(np.float64)
    with np.errstate(over="ignore"):          # overflow to inf is part of the law
        return exact.astype(np.float32).astype(np.float16).view(np.uint16)


def test_unpack_law_over_every_code_and_edge_scales():
    codes = np.arange(-128, 128, dtype=np.int8)
    scales = np.array([1.0, 0.1, 1 / 127, 3.0517578e-05, 1e-8, 2.0 ** -24,
                       5.96e-8 * 1.5, 300.0, 1000.0, -0.37, 65504.0 / 127,
                       np.float32(np.nextafter(np.float32(1.0), 2))], dtype=np.float32)
    for s in scales:
        got = oracle.dequant_payload_bits(codes[None, :], np.array([[s]], np.float32))[0]
        np.testing.assert_array_equal(got, law_via_fp64(codes, np.float32(s)))
    # random codes and scales: the two routes agree on every value
    rng = np.random.default_rng(0)
    c = rng.integers(-128, 128, size=(4096, 32)).astype(np.int8)
    s = (rng.random((4096, 1)) * 8).astype(np.float32)
    np.testing.assert_array_equal(oracle.dequant_payload_bits(c, s), law_via_fp64(c, s))


@pytest.mark.parametrize("bits", [8, 6, 4, 3, 2])
def test_quantiser_invariants(bits):
    rng = np.random.default_rng(bits)
    x = (rng.standard_normal((3, 4, 64)) * 2).astype(np.float16)
    x[1, 2] = 0                                   # all-zero groups: scale 1, codes 0
    codes, scales = oracle.quantize_symmetric(x, bits, 32)
    qmax = (1 << (bits - 1)) - 1
    assert codes.shape == (3, 4, 2, 32) and scales.shape == (3, 4, 2, 1)
    assert codes.min() >= -qmax - 1 and codes.max() <= qmax
    assert np.all(scales[1, 2] == 1.0) and np.all(codes[1, 2] == 0)
    back = oracle.f16_to_f32(oracle.dequant_payload_bits(codes, scales)).reshape(x.shape)
    err = np.abs(back - x.astype(np.float32)).reshape(3, 4, 2, 32)
    # half a step of rounding, plus the final fp16 rounding of the result
    assert np.all(err <= scales * 0.5 + np.abs(back.reshape(err.shape)) * 2.0 ** -10 + 1e-7)
    if bits == 8:
        c8, s8 = oracle.quantize_int8(x, 32)
        np.testing.assert_array_equal(c8.reshape(codes.shape), codes)
        np.testing.assert_array_equal(s8.reshape(scales.shape), scales)


def packed(arrays, bits=8, gs=32):
    out = {"format_version": np.asarray(1, np.int64),
           "storage_bits": np.asarray(bits, np.int64),
           "group_size": np.asarray(gs, np.int64)}
    for name, a in arrays.items():
        c, s = oracle.quantize_symmetric(a, bits, gs)
        out[f"{name}_codes"], out[f"{name}_scales"] = c, s
        out[f"{name}_shape"] = np.asarray(a.shape, np.int64)
    return out


def test_format_checks_fail_closed():
    a = np.ones((2, 3, 4, 64), np.float16)
    good = packed({"k": a})
    assert pl.is_packed_payload(good) and not pl.is_packed_payload({"k": a})
    bad = dict(good)
    del bad["format_version"]
    with pytest.raises(pl.PayloadFormatError):
        pl.unpack_kv_arrays_device(bad, ["k"])
    for field, value in (("format_version", 2), ("storage_bits", 16),
                         ("storage_bits", 5), ("storage_bits", np.array([8, 8]))):
        bad = dict(good)
        bad[field] = np.asarray(value, np.int64)
        with pytest.raises(pl.PayloadFormatError):
            pl.unpack_kv_arrays_device(bad, ["k"])
    with pytest.raises(pl.PayloadFormatError):
        pl.unpack_kv_arrays_device(good, ["v"])            # missing fields
    with pytest.raises(pl.PayloadFormatError):
        pl.upload_packed(good["k_codes"], good["k_scales"], (2, 3, 4, 65))
    with pytest.raises(pl.PayloadFormatError):
        pl.upload_packed(good["k_codes"], good["k_scales"][..., :1, :], a.shape)
    with pytest.raises(pl.PayloadFormatError):
        pl.upload_packed(good["k_codes"].astype(np.int16), good["k_scales"], a.shape)
