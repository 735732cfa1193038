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


_SM1 = np.uint64(0x9E3779B97F4A7C15)
_SM2 = np.uint64(0xBF58476D1CE4E5B9)
_SM3 = np.uint64(0x94D049BB133111EB)


def _splitmix_fill(out: np.ndarray, start: int, seed: int) -> None:
    """out[i] = splitmix64 finaliser of ((start + i) * golden + seed): a
    counter-based stream, so any slice can be filled independently."""
    blk = 1 << 18
    tmp = np.empty(min(blk, out.size), dtype=np.uint64)
    key = np.uint64(seed & 0xFFFFFFFFFFFFFFFF)
    for i in range(0, out.size, blk):
        n = min(blk, out.size - i)
        z = out[i:i + n]
        t = tmp[:n]
        z[:] = np.arange(start + i, start + i + n, dtype=np.uint64)
        z *= _SM1
        z += key
        np.right_shift(z, np.uint64(30), out=t)
        z ^= t
        z *= _SM2
        np.right_shift(z, np.uint64(27), out=t)
        z ^= t
        z *= _SM3
        np.right_shift(z, np.uint64(31), out=t)
        z ^= t


def gqa_int8_bank(lengths: np.ndarray, kv_heads: int, head_dim: int, seed: int,
                  workers: int = 16) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """INT8 CSR bank in the packed graft format: codes (node blocks
    [kv, L_i, hd] back to back, int8), one fp16 scale per (kv head, token)
    row (group size = head_dim; fp16 bits) and tok_offsets [N+1].

    Codes are uniform in [-127, 127] (the bytes of a splitmix64 counter
    stream, -128 folded to -127) and scales uniform in [2, 4] / 127 (the
    symmetric code range of rows whose absolute maximum lies in [2, 4]).
    `workers` threads fill fixed 32 MiB chunks of the counter stream, so
    banks of tens of GB build in seconds on the host and the result
    depends only on (lengths, kv_heads, head_dim, seed)."""
    from concurrent.futures import ThreadPoolExecutor

    lengths = np.asarray(lengths, dtype=np.uint64)
    offs = np.zeros(lengths.size + 1, dtype=np.uint64)
    offs[1:] = np.cumsum(lengths)
    rows = int(offs[-1]) * kv_heads
    n_codes = rows * head_dim
    words = np.empty((n_codes + 7) // 8, dtype=np.uint64)
    step = 1 << 22
    key = (int(seed) * 0xD1B54A32D192ED03 + 0x2545F4914F6CDD1D) & 0xFFFFFFFFFFFFFFFF

    def fill(i):
        seg = words[i:i + step]
        _splitmix_fill(seg, i, key)
        b = seg.view(np.int8)
        np.maximum(b, -127, out=b)

    with ThreadPoolExecutor(max_workers=max(1, workers)) as ex:
        list(ex.map(fill, range(0, words.size, step)))
    codes = words.view(np.int8)[:n_codes]
    rng = _rng(seed + 0x5CA1E)
    scales = (rng.uniform(2.0, 4.0, size=rows) / 127.0).astype(np.float16).view(np.uint16)
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
