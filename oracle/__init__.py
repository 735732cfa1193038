"""CPU oracle for the GRM graft route -- TEST INFRASTRUCTURE ONLY.

This package is the checker the HIP route library is compared against.  Only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import it; the product package ``graftrepository_amd`` never does.

``grm_oracle.c`` restates the reference's fp64 route laws (citations in that
file's header).  This module binds it with ctypes and adds the numpy-level
storage laws the tests need:

* bf16 rounding of fp32 values (round to nearest even, the conversion every
  bf16 bank/query goes through before the law is applied);
* the INT8 symmetric quantiser of ``core/graft_quant.py:93-131`` (group-32,
  fp32 scales) generalised to any group size and fp16 scales, and its
  dequant law ``core/graft_quant.py:136-144``.

Pinning (which check fixes which function) is listed in ``PINNING`` below and
exercised by ``tests/test_oracle_pinning.py``.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libgrm_oracle.so"
REF_LIB_PATH = HERE / "_ref" / "libgrm_runtime.so"

F32, BF16, F16, I8 = 0, 1, 2, 3

# function -> the checks that pin it (see tests/test_oracle_pinning.py)
PINNING = {
    "mla_route": "reference C++ grm_store_route goldens (tests/golden) + "
                 "orthonormal closed form + duplicate-row tie blocks + NaN rows",
    "mla_route_numpy": "closed forms (basis rows, scaled rows: a dot, not a "
                       "cosine), stable tie order, NaN rows dropped, and its "
                       "distance from the fp64 law within the fp32 dot's "
                       "rounding bound",
    "mla_route_normed": "equal to mla_route (ids and score bits) on random banks",
    "mla_row_norms": "closed form (unit vectors, Pythagorean triples) + "
                     "reference goldens via route order",
    "gqa_route": "reference C++ grm_store_route_gqa goldens on its fp64 path "
                 "(tests/golden) + hand cases [1,2,0], ties [0,1,2] + "
                 "single-token closed form (one key per node; multi-key "
                 "nodes are not modelled)",
    "store_route_gqa": "the reference store's grm_store_route_gqa (oracle/_ref, fp64 "
                       "law path) on random stores with lexical keys, metadata and "
                       "filters, single- and multi-key entries (tests/test_store_route.py)",
    "store_route": "the reference store's grm_store_route_filtered (oracle/_ref) on "
                   "random stores with lexical keys, metadata, filters, single- and "
                   "multi-row entries (tests/test_store_route.py)",
    "f16 conversion": "exhaustive agreement with numpy astype(float16)",
    "bf16 rounding": "agreement with torch.bfloat16 conversion",
    "int8 quantise/dequant": "round-trip invariants of "
                             "tests/test_graft_quant_format.py:54-78 + numpy law",
}

_lib = None


def build(force: bool = False) -> Path:
    """Compile libgrm_oracle.so with the committed Makefile."""
    if force or not LIB_PATH.exists():
        subprocess.run(["make", "-s", "-C", str(HERE), "all"], check=True)
    return LIB_PATH


def build_ref() -> Path | None:
    """Compile the reference CPU router into oracle/_ref when its sources exist."""
    src = Path(os.environ.get("GRM_REFERENCE_CPP", "/root/reference/cpp"))
    if not (src / "grm_runtime.cpp").exists():
        return REF_LIB_PATH if REF_LIB_PATH.exists() else None
    subprocess.run(["make", "-s", "-C", str(HERE), "ref", f"REF_DIR={src}"],
                   check=True)
    return REF_LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        build()
        L = ctypes.CDLL(str(LIB_PATH))
        u64, vp, i32 = ctypes.c_uint64, ctypes.c_void_p, ctypes.c_int
        L.grm_oracle_mla_row_norms.argtypes = [vp, u64, u64, vp, i32]
        L.grm_oracle_mla_row_norms.restype = None
        L.grm_oracle_mla_qnorm.argtypes = [vp, u64]
        L.grm_oracle_mla_qnorm.restype = ctypes.c_double
        L.grm_oracle_mla_scores.argtypes = [vp, u64, u64, vp, vp, u64, vp, i32]
        L.grm_oracle_mla_scores.restype = None
        L.grm_oracle_mla_route.argtypes = [
            vp, u64, u64, vp, vp, vp, u64, u64, i32, vp, vp, vp]
        L.grm_oracle_mla_route.restype = i32
        L.grm_oracle_mla_route_normed.argtypes = [
            vp, u64, u64, vp, vp, u64, u64, i32, vp, vp, vp]
        L.grm_oracle_mla_route_normed.restype = i32
        L.grm_oracle_gqa_scores.argtypes = [
            vp, i32, vp, i32, u64, vp, u64, u64, u64, vp, u64, u64, u64, vp,
            i32]
        L.grm_oracle_gqa_scores.restype = i32
        L.grm_oracle_gqa_route.argtypes = [
            vp, i32, vp, i32, u64, vp, u64, u64, u64, vp, vp, vp, u64, u64,
            u64, u64, i32, vp, vp, vp]
        L.grm_oracle_gqa_route.restype = i32
        L.grm_oracle_select_topk.argtypes = [vp, vp, vp, u64, u64, vp, vp, vp]
        L.grm_oracle_select_topk.restype = None
        L.grm_oracle_f16_from_f32.argtypes = [vp, u64, vp]
        L.grm_oracle_f16_from_f32.restype = None
        L.grm_oracle_f32_from_f16.argtypes = [vp, u64, vp]
        L.grm_oracle_f32_from_f16.restype = None
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


# ------------------------------------------------------------------ storage laws

def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round to nearest even; NaN stays a quiet NaN."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    rounded = u + (np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1)))
    out = (rounded >> np.uint32(16)).astype(np.uint16)
    nan = np.isnan(np.ascontiguousarray(x, dtype=np.float32))
    if np.any(nan):
        out[nan] = ((u[nan] >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16)
    return out


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """fp32 values rounded to the nearest bf16 value (returned as fp32)."""
    return bf16_to_f32(bf16_bits(x)).reshape(np.shape(x))


def f16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> fp16 bit patterns via the oracle's own RNE conversion."""
    xs = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(xs.shape, dtype=np.uint16)
    lib().grm_oracle_f16_from_f32(_p(xs), xs.size, _p(out))
    return out


def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(b.shape, dtype=np.float32)
    lib().grm_oracle_f32_from_f16(_p(b), b.size, _p(out))
    return out


def quantize_int8(x: np.ndarray, group_size: int, scale_dtype: str = "f32"):
    """Symmetric INT8 quantiser, core/graft_quant.py:93-131 (bits=8).

    ``scale = max|g| / 127`` in fp32 (0 -> 1.0); for ``scale_dtype='f16'`` the
    scale is rounded to fp16 first and the codes are computed against the
    rounded scale.  ``codes = clip(round_half_even(g / scale), -128, 127)``.
    Returns (codes int8 [..., D], scales [..., D/group] as f32 or f16 bits).
    """
    xf = np.ascontiguousarray(x, dtype=np.float32)
    d = xf.shape[-1]
    if d % group_size:
        raise ValueError("last axis not divisible by group_size")
    g = xf.reshape(*xf.shape[:-1], d // group_size, group_size)
    scale = np.abs(g).max(axis=-1, keepdims=True) / np.float32(127.0)
    scale = np.where(scale == 0, np.float32(1.0), scale).astype(np.float32)
    if scale_dtype == "f16":
        sbits = f16_bits(scale)
        scale = f16_to_f32(sbits)
        scale = np.where(scale == 0, np.float32(1.0), scale).astype(np.float32)
        sbits = f16_bits(scale)
        stored = sbits.reshape(*xf.shape[:-1], d // group_size)
    elif scale_dtype == "f32":
        stored = scale.reshape(*xf.shape[:-1], d // group_size)
    else:
        raise ValueError("scale_dtype must be 'f32' or 'f16'")
    codes = np.clip(np.round(g / scale), -128, 127).astype(np.int8)
    return codes.reshape(xf.shape), stored


def dequantize_int8(codes: np.ndarray, scales: np.ndarray, group_size: int,
                    scale_dtype: str = "f32") -> np.ndarray:
    """Dequant law core/graft_quant.py:136-144, returned as fp32 values."""
    c = np.ascontiguousarray(codes, dtype=np.int8)
    d = c.shape[-1]
    s = (f16_to_f32(scales) if scale_dtype == "f16"
         else np.ascontiguousarray(scales, dtype=np.float32))
    s = s.reshape(*c.shape[:-1], d // group_size, 1)
    g = c.reshape(*c.shape[:-1], d // group_size, group_size)
    prod = (g.astype(np.float32) * s).reshape(c.shape)
    return f16_to_f32(f16_bits(prod))


def quantize_symmetric(x: np.ndarray, bits: int, group_size: int = 32):
    """Packed-format quantiser, core/graft_quant.py:93-131, any depth 2..8.

    ``qmax = 2^(bits-1) - 1``; per group of ``group_size`` values along
    the last axis, ``scale = max|g| / qmax`` in fp32 (0 -> 1.0) and
    ``codes = clip(round_half_even(g / scale), -qmax-1, qmax)`` as int8.
    Returns ``codes (..., groups, group_size)`` and ``scales (..., groups,
    1)`` fp32, the shapes pack_kv_arrays stores.
    """
    if not 2 <= bits <= 8:
        raise ValueError("bits must be in 2..8")
    xf = np.ascontiguousarray(x, dtype=np.float32)
    d = xf.shape[-1]
    if d % group_size:
        raise ValueError("last axis not divisible by group_size")
    g = xf.reshape(*xf.shape[:-1], d // group_size, group_size)
    qmax = (1 << (bits - 1)) - 1
    scale = np.abs(g).max(axis=-1, keepdims=True) / np.float32(qmax)
    scale = np.where(scale == 0, np.float32(1.0), scale).astype(np.float32)
    codes = np.clip(np.round(g / scale), -qmax - 1, qmax).astype(np.int8)
    return codes, scale


def dequant_payload_bits(codes: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """Unpack law core/graft_quant.py:136-144 as fp16 bit patterns (uint16,
    codes' shape): the fp32 product of each code and its group's scale,
    rounded to fp16 (nearest even)."""
    c = np.ascontiguousarray(codes, dtype=np.int8)
    s = np.ascontiguousarray(scales, dtype=np.float32).reshape(*c.shape[:-1], 1)
    return f16_bits(c.astype(np.float32) * s)


# ------------------------------------------------------------ store route

_FILTER_SHIFTS = (0, 16, 32, 48)
_FILTER_DEFAULT = ("turn", "conversation", "session", "ephemeral")
_FILTER_KNOWN = (
    ("turn", "doc", "digest", "era", "fact", "task_state", "recall", "cull_span"),
    ("conversation", "project", "user", "task", "global", "session"),
    ("volatile", "session", "project", "permanent"),
    ("ephemeral", "stable", "mutable", "immutable"),
)


def _entry_max(key_scores, owners, n_entries):
    """Entry scores of multi-key entries: the largest finite score among an
    entry's keys, NaN when it has none (exact_mla_entry_score,
    cpp/grm_runtime.cpp:3518-3545; max_gqa_raw_score, :3031-3051).
    owners[j] is the entry of key j."""
    out = np.full(n_entries, np.nan, dtype=np.float32)
    for j, e in enumerate(owners):
        v = key_scores[j]
        if np.isfinite(v) and (not np.isfinite(out[e]) or v > out[e]):
            out[e] = v
    return out


def length_debias(scores, key_lengths) -> np.ndarray:
    """The reference's length-debiased latent score
    (core/graft_arena.py:839-874), one node at a time: K = max(1, key
    length), n = sqrt(log2(K + 1)) (numpy float64, :839-846), and the score
    s (a float32 law score, widened) becomes s / n when s >= 0 and s * n
    below zero (:866-873).  Returns float64."""
    out = np.empty(len(scores), dtype=np.float64)
    for i, (sc, kl) in enumerate(zip(scores, key_lengths)):
        try:
            k = max(1, int(kl))
        except (TypeError, ValueError, OverflowError):
            k = 1
        n = float(np.sqrt(np.log2(k + 1.0)))
        v = float(np.float32(sc))
        out[i] = v / n if v >= 0.0 else v * n
    return out


def rank_entries(scores, node_ids, topk: int):
    """(ids uint64[topk], scores float64[topk]) of the best finite scores,
    score descending then node id ascending; unfilled UINT64_MAX / NaN
    (the tie law score_node_better, cpp/grm_runtime.cpp:75-82)."""
    sc = np.asarray(scores, dtype=np.float64)
    ids = np.asarray(node_ids, dtype=np.uint64)
    keep = np.isfinite(sc)
    pairs = sorted(zip((-sc[keep]).tolist(), ids[keep].tolist()))[:topk]
    out_ids = np.full(topk, np.iinfo(np.uint64).max, dtype=np.uint64)
    out_sc = np.full(topk, np.nan, dtype=np.float64)
    for j, (ns, nid) in enumerate(pairs):
        out_ids[j] = nid
        out_sc[j] = -ns
    return out_ids, out_sc


def store_route(rows: np.ndarray, node_ids, lexical: list, meta: list, query: np.ndarray,
                query_lexical=(), filters=((), (), (), ()), topk: int = 3, owners=None):
    """The store's MLA route law, route_mla_arena (cpp/grm_runtime.cpp:
    4299-4361).  One row per entry, or with ``owners`` (entry index of each
    row) entries of any number of rows, scored as their best row.

    * meta[i] holds the values passed to set_route_metadata after the
      route was set (:2922-2946): an empty value keeps the entry's default,
      turn / conversation / session / ephemeral (cpp/grm_runtime.hpp:
      483-494).
    * Filters (:3053-3104): per category with filter values, the node's
      known-value bit (:2797-2838) must be among the filters' bits, or,
      when any filter value is unknown, the node's string must be listed.
    * The exact score must be finite; the route score is
      float(score) + float(hits) / float(|query lexical|) in fp32, where
      hits counts the query keys found among the node's keys (:3107-3170).
    * A non-finite sum drops the node; the order is (score desc, node id
      asc).

    Returns (node ids, route scores fp32) of the best topk."""
    ids = np.asarray(node_ids, dtype=np.uint64)
    if len(rows):
        base = mla_scores(rows, np.asarray(query, np.float32)[None])[0]
    else:
        base = np.zeros(0, np.float32)
    if owners is not None:
        base = _entry_max(base, owners, ids.size)
    qlex = [s for s in query_lexical if s]
    out = []
    for i in range(base.size):
        ok = True
        for c in range(4):
            fl = [v for v in filters[c] if v]
            if not fl:
                continue
            val = meta[i][c] or _FILTER_DEFAULT[c]
            if all(v in _FILTER_KNOWN[c] for v in fl):
                ok = ok and val in fl and val in _FILTER_KNOWN[c]
            else:
                ok = ok and val in fl
        if not ok or not np.isfinite(base[i]):
            continue
        hits = sum(1 for s in qlex if s in lexical[i])
        bonus = (np.float32(hits) / np.float32(len(qlex))) if qlex else np.float32(0.0)
        total = np.float32(base[i]) + bonus
        if np.isfinite(total):
            out.append((-float(total), int(ids[i]), total))
    out.sort()
    top = out[:topk]
    return [n for _, n, _ in top], np.asarray([t for _, _, t in top], dtype=np.float32)


def _route_allowed(meta_i, filters) -> bool:
    """Route filters (cpp/grm_runtime.cpp:3053-3104) for one entry whose
    metadata values are meta_i (empty: the entry default)."""
    for c in range(4):
        fl = [v for v in filters[c] if v]
        if not fl:
            continue
        val = meta_i[c] or _FILTER_DEFAULT[c]
        if all(v in _FILTER_KNOWN[c] for v in fl):
            if not (val in fl and val in _FILTER_KNOWN[c]):
                return False
        elif val not in fl:
            return False
    return True


def store_route_gqa(keys, tok_offsets, kv_heads: int, head_dim: int, node_ids, lexical: list,
                    meta: list, query, query_lexical=(), filters=((), (), (), ()),
                    topk: int = 3, owners=None):
    """The store's GQA route law, route_gqa_raw (cpp/grm_runtime.cpp:
    4498-4881), over fp32 keys in CSR layout (key j's [kv][L_j][hd] block at
    tok_offsets[j] * kv * hd): one key per entry, or with ``owners`` (entry
    index of each key) entries of any number of keys, scored as their best
    key.

    * raw = the fp64 GQA law (gqa_raw_score, :2980-3029) as float; entries
      that fail the route filters or whose raw score is not finite drop out;
    * no query lexical keys: order (raw desc, node id asc) (:4796-4821);
    * with them: norm = float(max |raw| over the entries left) + 1e-8f and
      score = raw / norm + float(hits) / float(|query lexical|) in fp32,
      order (score desc, node id asc) (:4823-4880).

    Returns (node ids, route scores fp32) of the best topk."""
    q = np.ascontiguousarray(query, dtype=np.float32)
    ids = np.asarray(node_ids, dtype=np.uint64)
    if len(tok_offsets) > 1:
        raw = gqa_scores(keys, F32, tok_offsets, kv_heads, head_dim, q[None])[0]
    else:
        raw = np.zeros(0, np.float32)
    if owners is not None:
        raw = _entry_max(raw, owners, ids.size)
    qlex = [s for s in query_lexical if s]
    have = [i for i in range(raw.size)
            if _route_allowed(meta[i], filters) and np.isfinite(raw[i])]
    if not qlex:
        order = sorted(have, key=lambda i: (-float(raw[i]), int(ids[i])))[:topk]
        return [int(ids[i]) for i in order], np.asarray([raw[i] for i in order], np.float32)
    max_abs = np.float32(0.0)
    for i in have:
        max_abs = max(max_abs, np.float32(abs(raw[i])))
    norm = np.float32(max_abs + np.float32(1.0e-8))
    den = np.float32(len(qlex))
    out = []
    for i in have:
        hits = sum(1 for s in qlex if s in lexical[i])
        score = np.float32(np.float32(raw[i]) / norm) + np.float32(np.float32(hits) / den)
        out.append((-float(score), int(ids[i]), np.float32(score)))
    out.sort()
    top = out[:topk]
    return [n for _, n, _ in top], np.asarray([t for _, _, t in top], dtype=np.float32)


# ------------------------------------------------------------------ MLA

def mla_row_norms(rows: np.ndarray, threads: int = 0) -> np.ndarray:
    r = np.ascontiguousarray(rows, dtype=np.float32)
    out = np.empty(r.shape[0], dtype=np.float32)
    lib().grm_oracle_mla_row_norms(_p(r), r.shape[0], r.shape[1], _p(out),
                                   threads)
    return out


def mla_qnorm(q: np.ndarray) -> float:
    qq = np.ascontiguousarray(q, dtype=np.float32).reshape(-1)
    return float(lib().grm_oracle_mla_qnorm(_p(qq), qq.size))


def mla_scores(rows: np.ndarray, queries: np.ndarray, threads: int = 0):
    r = np.ascontiguousarray(rows, dtype=np.float32)
    q = np.ascontiguousarray(queries, dtype=np.float32).reshape(-1, r.shape[1])
    norms = mla_row_norms(r, threads)
    out = np.empty((q.shape[0], r.shape[0]), dtype=np.float32)
    lib().grm_oracle_mla_scores(_p(r), r.shape[0], r.shape[1], _p(norms),
                                _p(q), q.shape[0], _p(out), threads)
    return out


def mla_route_numpy(rows: np.ndarray, queries: np.ndarray, topk: int):
    """The reference's Python MLA route law, in numpy, for the CPU baseline.

    ``ArenaCache._vector_route_scores`` (core/graft_arena.py:778-801)
    scores ``np.stack(rows).astype(float32) @ q`` -- an fp32 dot, no
    norms (the centroids are unit-norm) -- and keeps the finite scores;
    the route (:733-768) then sorts the candidates by ``-score`` with
    Python's stable sort, so ties keep ascending graft order.  With no
    lexical keys and the default length/normalisation hooks off (:813,
    :847-862) the first ``topk`` entries are the route.

    Returns (row indices [Q,k] int64, scores [Q,k] f32, counts [Q]);
    unfilled slots hold -1 / NaN.  The dot's summation order is numpy's
    BLAS sgemv and is not fixed by the reference; the tests pin the law
    by closed forms and by its distance from the fp64 law, not bit for
    bit."""
    r = np.ascontiguousarray(rows, dtype=np.float32)
    q = np.ascontiguousarray(queries, dtype=np.float32).reshape(-1, r.shape[1])
    out_ids = np.full((q.shape[0], topk), -1, dtype=np.int64)
    out_sc = np.full((q.shape[0], topk), np.nan, dtype=np.float32)
    counts = np.zeros(q.shape[0], dtype=np.int64)
    for j in range(q.shape[0]):
        s = r @ q[j]
        keep = np.flatnonzero(np.isfinite(s))
        sk = s[keep]
        kk = min(topk, keep.size)
        if kk < keep.size:
            # the stable sort's first kk entries: every score at or above the
            # kk-th largest (ties at that value included), in row order,
            # then sorted stably by -score
            part = np.argpartition(-sk, kk - 1)[:kk]
            keep = keep[sk >= sk[part].min()]
            sk = s[keep]
        order = keep[np.argsort(-sk, kind="stable")][:topk]
        out_ids[j, :order.size] = order
        out_sc[j, :order.size] = s[order]
        counts[j] = order.size
    return out_ids, out_sc, counts


def mla_route(rows: np.ndarray, queries: np.ndarray, topk: int, *,
              node_ids: np.ndarray | None = None,
              live: np.ndarray | None = None, threads: int = 0):
    """fp64 MLA law route; returns (ids [Q,k] uint64, scores [Q,k] f32, counts)."""
    r = np.ascontiguousarray(rows, dtype=np.float32)
    q = np.ascontiguousarray(queries, dtype=np.float32).reshape(-1, r.shape[1])
    ids = None if node_ids is None else np.ascontiguousarray(node_ids, np.uint64)
    lv = None if live is None else np.ascontiguousarray(live, np.uint8)
    out_ids = np.empty((q.shape[0], topk), dtype=np.uint64)
    out_scores = np.empty((q.shape[0], topk), dtype=np.float32)
    counts = np.empty(q.shape[0], dtype=np.uint64)
    rc = lib().grm_oracle_mla_route(
        _p(r), r.shape[0], r.shape[1], _p(ids), _p(lv), _p(q), q.shape[0],
        topk, threads, _p(out_ids), _p(out_scores), _p(counts))
    if rc != 0:
        raise RuntimeError(f"oracle mla_route failed: {rc}")
    return out_ids, out_scores, counts


def mla_route_normed(rows: np.ndarray, norms: np.ndarray, queries: np.ndarray,
                     topk: int, threads: int = 0):
    """fp64 MLA law route over precomputed row norms (``mla_row_norms``):
    the reference route's per-call work, with the norms held by its arena
    as the reference's arena holds them.  Same returns as ``mla_route``."""
    r = np.ascontiguousarray(rows, dtype=np.float32)
    nr = np.ascontiguousarray(norms, dtype=np.float32)
    q = np.ascontiguousarray(queries, dtype=np.float32).reshape(-1, r.shape[1])
    if nr.shape != (r.shape[0],):
        raise ValueError("norms must have one value per row")
    out_ids = np.empty((q.shape[0], topk), dtype=np.uint64)
    out_scores = np.empty((q.shape[0], topk), dtype=np.float32)
    counts = np.empty(q.shape[0], dtype=np.uint64)
    rc = lib().grm_oracle_mla_route_normed(
        _p(r), r.shape[0], r.shape[1], _p(nr), _p(q), q.shape[0], topk,
        threads, _p(out_ids), _p(out_scores), _p(counts))
    if rc != 0:
        raise RuntimeError(f"oracle mla_route_normed failed: {rc}")
    return out_ids, out_scores, counts


# ------------------------------------------------------------------ GQA

def _gqa_args(keys, key_dtype, scales, scale_dtype):
    k = np.ascontiguousarray(keys)
    s = None if scales is None else np.ascontiguousarray(scales)
    sd = F16 if scale_dtype == "f16" else F32
    return k, s, sd


def gqa_scores(keys, key_dtype: int, tok_offsets, kv_heads: int, head_dim: int,
               queries, *, scales=None, scale_dtype: str = "f32",
               group_size: int = 0, threads: int = 0) -> np.ndarray:
    """Exact GQA scores [Q, N] (fp64 law) over a CSR key bank."""
    k, s, sd = _gqa_args(keys, key_dtype, scales, scale_dtype)
    offs = np.ascontiguousarray(tok_offsets, dtype=np.uint64)
    q = np.ascontiguousarray(queries, dtype=np.float32)
    if q.ndim == 3:
        q = q[None]
    n = offs.size - 1
    out = np.empty((q.shape[0], n), dtype=np.float32)
    rc = lib().grm_oracle_gqa_scores(
        _p(k), key_dtype, _p(s), sd, group_size, _p(offs), n, kv_heads,
        head_dim, _p(q), q.shape[0], q.shape[1], q.shape[2], _p(out), threads)
    if rc != 0:
        raise RuntimeError(f"oracle gqa_scores failed: {rc}")
    return out


def gqa_route(keys, key_dtype: int, tok_offsets, kv_heads: int, head_dim: int,
              queries, topk: int, *, scales=None, scale_dtype: str = "f32",
              group_size: int = 0, node_ids=None, live=None, threads: int = 0):
    k, s, sd = _gqa_args(keys, key_dtype, scales, scale_dtype)
    offs = np.ascontiguousarray(tok_offsets, dtype=np.uint64)
    q = np.ascontiguousarray(queries, dtype=np.float32)
    if q.ndim == 3:
        q = q[None]
    n = offs.size - 1
    ids = None if node_ids is None else np.ascontiguousarray(node_ids, np.uint64)
    lv = None if live is None else np.ascontiguousarray(live, np.uint8)
    out_ids = np.empty((q.shape[0], topk), dtype=np.uint64)
    out_scores = np.empty((q.shape[0], topk), dtype=np.float32)
    counts = np.empty(q.shape[0], dtype=np.uint64)
    rc = lib().grm_oracle_gqa_route(
        _p(k), key_dtype, _p(s), sd, group_size, _p(offs), n, kv_heads,
        head_dim, _p(ids), _p(lv), _p(q), q.shape[0], q.shape[1], q.shape[2],
        topk, threads, _p(out_ids), _p(out_scores), _p(counts))
    if rc != 0:
        raise RuntimeError(f"oracle gqa_route failed: {rc}")
    return out_ids, out_scores, counts


def select_topk(scores, topk: int, node_ids=None, live=None):
    s = np.ascontiguousarray(scores, dtype=np.float32)
    ids = None if node_ids is None else np.ascontiguousarray(node_ids, np.uint64)
    lv = None if live is None else np.ascontiguousarray(live, np.uint8)
    out_ids = np.empty(topk, dtype=np.uint64)
    out_scores = np.empty(topk, dtype=np.float32)
    count = np.zeros(1, dtype=np.uint64)
    lib().grm_oracle_select_topk(_p(s), _p(ids), _p(lv), s.size, topk,
                                 _p(out_ids), _p(out_scores), _p(count))
    return out_ids, out_scores, int(count[0])
