"""Seeded synthetic route workloads.

The route inputs of a real deployment come from a model forward (latent
centroids, layer-0 keys and queries; core/kv_graft.py:132-171).  These
generators produce the same shapes and distributions without a model:

* MLA centroid banks: rows ~ N(0, 1), then L2-normalised per row (norm in
  fp64, division in fp32), optionally rounded to bf16; queries the same.
* Ragged GQA banks: per node a key block [kv_heads, L_i, head_dim] ~ N(0, 1)
  (bf16 by default), lengths uniform or lognormal; queries [H, Qt, hd].
  Stacked routing layers fold into the head axes: kv head g of layer y is
  bank head y*KV+g, query head h of layer y is y*H+h (so kv head = h'/R).
* INT8 ragged banks: N(0, 1) keys quantised per (kv head, token) row by the
  packed graft format's law with an fp16 scale (gqa_int8_bank).

Every generator is a pure function of its arguments and seed.
"""

from __future__ import annotations

import hashlib

import numpy as np

from .node_bank import as_bf16_bits


def _rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(np.random.SeedSequence(int(seed)))


def normalise_rows(x: np.ndarray) -> np.ndarray:
    """L2-normalise rows: norm accumulated in fp64, division in fp32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    step = 1 << 16
    for i in range(0, x.shape[0], step):
        blk = x[i:i + step]
        nrm = np.sqrt(np.einsum("ij,ij->i", blk.astype(np.float64),
                                blk.astype(np.float64)))
        nrm = np.where(nrm > 0, nrm, 1.0).astype(np.float32)
        out[i:i + step] = blk / nrm[:, None]
    return out


def mla_rows(nodes: int, dim: int, seed: int, dtype: str = "f32") -> np.ndarray:
    """Unit-norm Gaussian centroid rows [nodes, dim] (f32 or bf16 bits)."""
    rng = _rng(seed)
    out = np.empty((nodes, dim), dtype=np.float32 if dtype == "f32" else np.uint16)
    step = 1 << 16
    for i in range(0, nodes, step):
        n = min(step, nodes - i)
        blk = normalise_rows(rng.standard_normal((n, dim), dtype=np.float32))
        out[i:i + n] = blk if dtype == "f32" else as_bf16_bits(blk)
    return out


def mla_queries(count: int, dim: int, seed: int, dtype: str = "f32") -> np.ndarray:
    return mla_rows(count, dim, seed + 0x5EED, dtype)


def gqa_lengths(nodes: int, seed: int, *, kind: str = "uniform",
                lo: int = 16, hi: int = 512, median: float = 256.0,
                sigma: float = 0.5, cap: int = 4096) -> np.ndarray:
    """Per-node key token counts.

    uniform:   integers in [lo, hi]
    lognormal: round(exp(N(ln median, sigma))) clipped to [1, cap]
    """
    rng = _rng(seed + 0x1E9)
    if kind == "uniform":
        return rng.integers(lo, hi + 1, size=nodes).astype(np.uint64)
    if kind == "lognormal":
        x = np.exp(rng.normal(np.log(median), sigma, size=nodes))
        return np.clip(np.rint(x), 1, cap).astype(np.uint64)
    raise ValueError(f"unknown length kind {kind!r}")


def gqa_bank(lengths: np.ndarray, kv_heads: int, head_dim: int, seed: int,
             dtype: str = "bf16") -> tuple[np.ndarray, np.ndarray]:
    """CSR bank: flat keys (node blocks [kv, L_i, hd] back to back) and
    tok_offsets [N+1].  dtype f32 -> float32, bf16 -> uint16 bits,
    f16 -> uint16 bits."""
    lengths = np.asarray(lengths, dtype=np.uint64)
    offs = np.zeros(lengths.size + 1, dtype=np.uint64)
    offs[1:] = np.cumsum(lengths)
    total = int(offs[-1]) * kv_heads * head_dim
    rng = _rng(seed)
    out = np.empty(total, dtype=np.float32 if dtype == "f32" else np.uint16)
    step = 1 << 24
    for i in range(0, total, step):
        n = min(step, total - i)
        blk = rng.standard_normal(n, dtype=np.float32)
        if dtype == "f32":
            out[i:i + n] = blk
        elif dtype == "bf16":
            out[i:i + n] = as_bf16_bits(blk)
        elif dtype == "f16":
            out[i:i + n] = blk.astype(np.float16).view(np.uint16)
        else:
            raise ValueError(f"unknown dtype {dtype!r}")
    return out, offs


def quantize_rows_i8(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """The packed graft format's symmetric INT8 quantiser
    (core/graft_quant.py:93-131, bits = 8) with one group per row and the
    scale stored as fp16: scale = max|row| / 127 in fp32 (0 -> 1), rounded
    to fp16 (0 -> 1), codes = clip(round_half_even(row / scale), -128, 127)
    against the stored scale.  x: float32 [rows, d].  Returns (codes int8
    [rows, d], scales as fp16 bits [rows])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    scale = np.abs(x).max(axis=1) / np.float32(127.0)
    scale[scale == 0] = np.float32(1.0)
    s16 = scale.astype(np.float16)
    s16[s16 == 0] = np.float16(1.0)
    y = x / s16.astype(np.float32)[:, None]
    np.rint(y, out=y)
    np.clip(y, -128.0, 127.0, out=y)
    return y.astype(np.int8), s16.view(np.uint16)


_NORMAL_TABLE: np.ndarray | None = None


def _normal_table() -> np.ndarray:
    """The 65,536 quantiles Phi^-1((i + 0.5) / 65536) of N(0, 1) as
    float32: a uniform 16-bit index looked up here is a standard normal
    draw discretised to 2^16 equiprobable levels (tails to about 4.3)."""
    global _NORMAL_TABLE
    if _NORMAL_TABLE is None:
        from statistics import NormalDist

        inv = NormalDist().inv_cdf
        _NORMAL_TABLE = np.asarray([inv((i + 0.5) / 65536.0) for i in range(65536)],
                                   dtype=np.float32)
    return _NORMAL_TABLE


def int8_stream_key(seed: int) -> int:
    """The 64-bit key of the synthetic INT8 key stream for `seed`."""
    return (int(seed) * 0xD1B54A32D192ED03 + 0x2545F4914F6CDD1D) & 0xFFFFFFFFFFFFFFFF


def gqa_int8_bank(lengths: np.ndarray, kv_heads: int, head_dim: int, seed: int,
                  workers: int = 16) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """INT8 CSR bank in the packed graft format: N(0, 1) keys quantised row
    by row (the law of quantize_rows_i8: one fp16 scale per (kv head,
    token) row, group size = head_dim).  Returns codes (node blocks
    [kv, L_i, hd] back to back, int8), scales (fp16 bits, one per row, in
    row order) and tok_offsets [N+1].

    Row r's keys are normal quantiles (_normal_table) of the 16-bit words
    of a splitmix64 counter stream at word indices r * hd/4 ... (key
    int8_stream_key(seed)); the library's host generator
    (grm_hip_synth_int8_rows) draws and quantises them on `workers`
    threads, so the bank is a pure function of (lengths, kv_heads,
    head_dim, seed) and banks of tens of GB build in seconds."""
    from . import _lib

    if head_dim % 4:
        raise ValueError("head_dim must be a multiple of 4")
    lengths = np.asarray(lengths, dtype=np.uint64)
    offs = np.zeros(lengths.size + 1, dtype=np.uint64)
    offs[1:] = np.cumsum(lengths)
    rows = int(offs[-1]) * kv_heads
    codes = np.empty(rows * head_dim, dtype=np.int8)
    scales = np.empty(rows, dtype=np.uint16)
    table = _normal_table()
    _lib.check(_lib.load().grm_hip_synth_int8_rows(
        int8_stream_key(seed), 0, rows, head_dim, table.ctypes.data, max(1, workers),
        codes.ctypes.data, scales.ctypes.data), "synthetic INT8 rows")
    return codes, scales, offs


def gqa_queries(count: int, heads: int, tokens: int, head_dim: int, seed: int,
                dtype: str = "bf16") -> np.ndarray:
    rng = _rng(seed + 0x9E5)
    q = rng.standard_normal((count, heads, tokens, head_dim), dtype=np.float32)
    if dtype == "f32":
        return q
    if dtype == "bf16":
        return as_bf16_bits(q)
    raise ValueError(f"unknown dtype {dtype!r}")


def digest(*arrays: np.ndarray) -> str:
    """sha256 over the raw bytes of the arrays (fixture identity check)."""
    h = hashlib.sha256()
    for a in arrays:
        a = np.ascontiguousarray(a)
        h.update(str(a.dtype).encode())
        h.update(str(a.shape).encode())
        h.update(memoryview(a.view(np.uint8).reshape(-1)))
    return h.hexdigest()


# Named configurations (sizes of the benchmarked route workloads).
MLA_HEADLINE = dict(nodes=1_000_000, dim=288, topk=3, seed=2)
MLA_SMALL = dict(nodes=10_000, dim=288, topk=3, seed=1)
MLA_BATCHED = dict(nodes=1_000_000, dim=288, queries=256, topk=8, seed=3)
GQA_RAGGED = dict(nodes=512, layers=4, kv_heads=8, heads=32, head_dim=128,
                  lo=16, hi=512, tokens=1, topk=3, seed=4)
GQA_INT8 = dict(nodes=100_000, layers=1, kv_heads=8, heads=32, head_dim=128,
                median=256.0, sigma=0.5, cap=4096, queries=16, topk=5, seed=5)
