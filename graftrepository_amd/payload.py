"""Packed graft payloads, unpacked on the device.

The packed format is core/graft_quant.py's (:177-268): per tensor ``name``,

* ``{name}_codes``: int8 ``(..., groups, group_size)``;
* ``{name}_scales``: fp32 ``(..., groups, 1)``;
* ``{name}_shape``: the pre-group shape;

plus scalar ``format_version``, ``storage_bits`` and ``group_size`` fields.
A tensor unpacks as ``fp16(fp32(code) * scale)`` (:136-144), for every
storage depth.

The reference's node unpack (core/graft_arena.py:3479-3492) dequantises on
the host and uploads fp16.  Here the codes and scales go to the device
(``grm_hip_payload_upload``), and the library writes the fp16 bit patterns
into a ``DeviceArray``.  Validation fails closed like ``unpack_kv_arrays``:
an unknown format version, a 16-bit or unsupported depth, a missing field,
or a shape that does not match raises ``PayloadFormatError``.
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _lib

FORMAT_VERSION = 1                       # core/graft_quant.py:65
SUPPORTED_BITS = (16, 8, 6, 4, 3, 2)     # core/graft_quant.py:66


class PayloadFormatError(ValueError):
    """Unknown or malformed packed payload (mirrors GraftQuantFormatError,
    core/graft_quant.py:74-76)."""


class DeviceArray:
    """Values in device memory owned by this object (row-major ``shape``,
    numpy ``dtype``, fp16 by default).  ``ptr`` is the device address;
    ``to_host()`` copies them back, ``from_host(a)`` makes one holding a
    copy of a host array.  ``sub(i)`` is the address of entry i along the
    first axis, e.g. one layer of an (L, H, S, D) node payload."""

    def __init__(self, shape, dtype=np.float16):
        self.shape = tuple(int(d) for d in shape)
        self.dtype = np.dtype(dtype)
        self.size = int(np.prod(self.shape, dtype=np.int64)) if self.shape else 1
        self.nbytes = self.dtype.itemsize * self.size
        self._lib = _lib.load()
        p = ctypes.c_void_p()
        _lib.check(self._lib.grm_hip_device_alloc(max(self.nbytes, 2), ctypes.byref(p)),
                   "device alloc")
        self.ptr = int(p.value)

    def to_host(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        _lib.check(self._lib.grm_hip_copy_to_host(out.ctypes.data, self.ptr, self.nbytes),
                   "device to host copy")
        return out

    @classmethod
    def from_host(cls, a) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        _lib.check(d._lib.grm_hip_copy_to_device(d.ptr, a.ctypes.data, a.nbytes),
                   "host to device copy")
        return d

    def sub(self, i: int) -> int:
        if not self.shape or not 0 <= i < self.shape[0]:
            raise IndexError(i)
        return self.ptr + i * (self.nbytes // self.shape[0])

    def data_ptr(self) -> int:
        return self.ptr

    def close(self) -> None:
        if getattr(self, "ptr", 0):
            self._lib.grm_hip_device_free(self.ptr)
            self.ptr = 0

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def is_packed_payload(payload) -> bool:
    """True when the payload carries a ``format_version`` field
    (core/graft_quant.py:271-279)."""
    try:
        keys = payload.files if hasattr(payload, "files") else payload.keys()
    except Exception:
        return False
    return "format_version" in keys


def _scalar(payload, name: str) -> int:
    arr = np.asarray(payload[name])
    if arr.shape == ():
        return int(arr)
    if arr.size == 1:
        return int(arr.reshape(-1)[0])
    raise PayloadFormatError(f"field {name!r} must be scalar-like, got shape {arr.shape}")


def upload_packed(codes, scales, shape) -> DeviceArray:
    """Unpack one packed tensor onto the device.  ``codes`` int8
    (..., groups, group_size), ``scales`` fp32 (..., groups, 1) or
    (..., groups), ``shape`` the pre-group shape."""
    c = np.ascontiguousarray(codes)
    if c.dtype != np.int8:
        raise PayloadFormatError(f"codes must be int8, got {c.dtype}")
    if c.ndim < 1:
        raise PayloadFormatError("codes need a group axis")
    gs = int(c.shape[-1])
    s = np.ascontiguousarray(scales, dtype=np.float32).reshape(-1)
    n = int(c.size)
    shape = tuple(int(d) for d in shape)
    if gs <= 0 or n % gs or s.size != n // gs:
        raise PayloadFormatError(
            f"scales ({s.size}) do not match codes {c.shape} in groups of {gs}")
    if int(np.prod(shape, dtype=np.int64)) != n:
        raise PayloadFormatError(f"shape {shape} does not hold {n} values")
    out = DeviceArray(shape)
    if n:
        ms = ctypes.c_float(0.0)
        rc = out._lib.grm_hip_payload_upload(c.ctypes.data, s.ctypes.data, n, gs, out.ptr,
                                             ctypes.byref(ms))
        if rc != 0:
            out.close()
            _lib.check(rc, "payload upload")
        out.device_ms = float(ms.value)
    return out


def unpack_kv_arrays_device(payload, names) -> dict[str, DeviceArray]:
    """Device counterpart of ``unpack_kv_arrays`` (core/graft_quant.py:
    232-268): same validation, fp16 results in device memory."""
    if "format_version" not in (payload.files if hasattr(payload, "files") else payload.keys()):
        raise PayloadFormatError("payload has no format_version field")
    version = _scalar(payload, "format_version")
    if version != FORMAT_VERSION:
        raise PayloadFormatError(f"unknown format_version {version}")
    bits = _scalar(payload, "storage_bits")
    if bits not in SUPPORTED_BITS or bits == 16:
        raise PayloadFormatError(f"storage_bits {bits} is not a packed depth")
    out: dict[str, DeviceArray] = {}
    try:
        for name in names:
            keys = (f"{name}_codes", f"{name}_scales", f"{name}_shape")
            if any(k not in payload for k in keys):
                raise PayloadFormatError(f"payload missing {'/'.join(keys)}")
            shape = tuple(int(v) for v in np.asarray(payload[keys[2]]))
            out[name] = upload_packed(payload[keys[0]], payload[keys[1]], shape)
    except Exception:
        for arr in out.values():
            arr.close()
        raise
    return out


def unpack_node_device(payload, names=("k", "v")) -> dict[str, DeviceArray]:
    """Device counterpart of ``unpack_node`` (core/graft_arena.py:
    3479-3492): a packed payload is unpacked on the device, and a plain
    fp16 payload is uploaded as it is.  Each result is the stacked
    ``(L, H, S, D)`` array; ``sub(li)`` addresses layer li."""
    if is_packed_payload(payload):
        return unpack_kv_arrays_device(payload, list(names))
    out: dict[str, DeviceArray] = {}
    for name in names:
        out[name] = DeviceArray.from_host(np.ascontiguousarray(payload[name], dtype=np.float16))
    return out


__all__ = ["DeviceArray", "PayloadFormatError", "is_packed_payload", "upload_packed",
           "unpack_kv_arrays_device", "unpack_node_device", "FORMAT_VERSION",
           "SUPPORTED_BITS"]
