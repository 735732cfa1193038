"""Arena bridge: epoch-gated device route banks that follow an arena's
grafts with evictions and appends.

The reference keeps its CUDA route bank in step with the arena like this.

* The arena bumps an epoch on every mutation (core/graft_arena.py:278-291,
  2922-2931).
* While the epoch holds, the cached bank is reused with no walk at all.
* When the epoch moves, a walk over the grafts builds the eligible rows and
  their signature: one ``(node_id, shape, dtype, id(cent))`` entry per row
  (MLA core/graft_arena.py:1124-1162, GQA :2933-2977).
* If the signature is unchanged, the bank stays.
* Otherwise the whole bank is stacked again and uploaded as a new sidecar
  bank (:1164-1198, :3055-3160, :1247-1280, :3161-3203; store attach
  core/grm_native.py:1498-1673), and any route-key mutation on the store
  drops the bank (:1391-1444).

The bridges here keep the epoch gate, the walk, the signature law and the
reverse maps.  On a signature change they keep the one device bank
(``MlaNodeBank`` / ``GqaNodeBank``) and move it to the new row set:

* evict the resident node ids that left, or whose signature entry changed;
* append the rows that are new or changed;
* when an append needs more room: a GQA bank first compacts its token
  arena, and otherwise the bank is rebuilt once with twice the capacity.

Each refresh records an event in the reference's vocabulary
(``reused``, ``signature_reused``, ``ineligible``, ...) plus the rows moved
and the bytes uploaded.

A route result depends only on the set of (node id, row) pairs, not on the
slots that hold them: ties go to the lower node id.  So a bank updated this
way answers exactly as a bank built from scratch over the same rows.

Two cases send the reference's arena to its CPU path; the bridges serve
both on the device:

* Digest nodes (grafts with ``child_cents``) score the best of their own
  key and their children's (core/graft_arena.py:803-811), the law of a
  store entry with several keys (cpp/grm_runtime.cpp:3518-3545, 3031-3051).
  The reference's CUDA walk declines any arena holding one (:1141-1142,
  2951).  Here their keys sit in a second device bank of the same kind,
  scored exactly on every route, and each digest node's best finite key
  score joins the main bank's top k.
* ``length_debias`` (:839-874): the route ranks raw / sqrt(log2(K + 1))
  (raw * that factor for a negative raw score), K the node's route key
  length (:813-837).  The reference leaves its native and CUDA routes for
  its Python path when it is on (:686-687).  Here every eligible node is
  scored exactly on the device and the ranking applies the factor.

Route receipts follow the reference's route profile (core/graft_arena.py:
161-256): with ``route_profile=True`` or ``GRM_ROUTE_SEAMS_PROFILE`` set to
1 / true / yes / on, every ``route_order`` leaves a JSON-ready dict in
``last_route_receipt`` (and appends it to ``route_receipt_history``): the
time of each phase in ``terms_ms``, the bank's refresh event under
``rebuilds``, the reasons a route fell back to the caller's CPU path under
``fallbacks``, and the ranking's length and first 16 graft indices.  An
unprofiled route leaves ``last_route_receipt`` None.  The history keeps
every profiled route's receipt, as the reference's does (:249-254); a
long-running caller that profiles clears it when it has read it.
"""

from __future__ import annotations

import os
import time
from typing import NamedTuple

import numpy as np

from .node_bank import GqaNodeBank, MlaNodeBank

MAX_TOPK = 16  # reference ABI cap (scripts/grm_mla_cuda_probe.py:355-358)
ROUTE_RECEIPT_SCHEMA = "grm_route_seams_route_v1"


def route_profile_env() -> bool:
    """GRM_ROUTE_SEAMS_PROFILE asks for route receipts
    (core/graft_arena.py:161-165)."""
    return os.environ.get("GRM_ROUTE_SEAMS_PROFILE", "").strip().lower() in (
        "1", "true", "yes", "on")


class RowSet(NamedTuple):
    """What a walk found, in arrays: row i is node ``node_ids[i]``.  Its
    centroid object has ``cent_ids[i] = id(cent)``, and its extent is
    ``extents[i]`` (the dim for MLA, the token count for GQA).  These are
    the parts of the reference's signature entry
    ``(node_id, shape, dtype, id(cent))`` that can change.  The dtype after
    the walk's conversion is always float32, and the other dims are uniform
    or the walk declines."""
    node_ids: np.ndarray
    cent_ids: np.ndarray
    extents: np.ndarray

    def same(self, other) -> bool:
        return (other is not None and np.array_equal(self.node_ids, other.node_ids)
                and np.array_equal(self.cent_ids, other.cent_ids)
                and np.array_equal(self.extents, other.extents))


class Digest(NamedTuple):
    """Digest nodes of a walk: node ``node_ids[i]`` (graft ``gidx[i]``) has
    the keys ``keys[offs[i]:offs[i + 1]]``, its own centroid first and then
    its ``child_cents`` (core/graft_arena.py:803-811).  ``sig`` holds each
    node's id with the ids and extents of its key objects: an unchanged
    ``sig`` keeps the side bank."""
    node_ids: np.ndarray
    offs: np.ndarray
    keys: list
    gidx: list
    sig: tuple
    pinned: list


def route_key_length(g) -> int:
    """The reference's route key length K of a graft
    (core/graft_arena.py:813-837): the token axis of a key with two or
    more dims, else the graft's ``ntok``; 1 when missing or malformed."""
    cent = g.get("cent")
    if cent is not None:
        shape = np.asarray(cent).shape
        if len(shape) >= 2:
            try:
                return max(1, int(shape[-2]))
            except (TypeError, ValueError, OverflowError):
                pass
    try:
        return max(1, int(g.get("ntok", 1)))
    except (TypeError, ValueError, OverflowError):
        return 1


def length_debias_factor(key_length) -> np.ndarray:
    """sqrt(log2(K + 1)) in float64 (core/graft_arena.py:839-846), K >= 1."""
    k = np.maximum(np.asarray(key_length, dtype=np.float64), 1.0)
    return np.sqrt(np.log2(k + 1.0))


def apply_length_debias(scores, key_length) -> np.ndarray:
    """raw / sqrt(log2(K + 1)) for raw >= 0, raw * sqrt(log2(K + 1)) below
    zero, in float64 (core/graft_arena.py:848-874)."""
    raw = np.asarray(scores, dtype=np.float32).astype(np.float64)
    n = length_debias_factor(key_length)
    return np.where(raw >= 0.0, raw / n, raw * n)


def _digest(nids, keysets, gidx):
    offs = np.zeros(len(keysets) + 1, dtype=np.int64)
    offs[1:] = np.cumsum([len(k) for k in keysets])
    keys = [k for ks in keysets for k, _ in ks]
    pinned = [o for ks in keysets for _, o in ks]
    sig = tuple((int(n), tuple(id(o) for _, o in ks), tuple(k.shape for k, _ in ks))
                for n, ks in zip(nids, keysets))
    return Digest(np.asarray(nids, dtype=np.uint64), offs, keys, list(gidx), sig, pinned)


def _walk_mla(grafts, digests: bool = False, lengths: bool = False):
    """The MLA walk (core/graft_arena.py:1124-1162): rows are the grafts
    that are neither retired nor recall entries (:1139-1140).  Returns
    ``(RowSet, rows, graft_indices, cents, Digest or None, key lengths or
    None)`` or None.  A graft with ``child_cents`` makes the walk decline,
    as the reference's does, unless ``digests``: its keys then go to the
    Digest part.  ``lengths``: each row's and digest node's K."""
    rows, nids, cids, gidx = [], [], [], []
    add_row, add_nid, add_cid, add_g = rows.append, nids.append, cids.append, gidx.append
    d_nids, d_keys, d_gidx = [], [], []
    klen, d_klen = [], []
    dim = None
    f32 = np.dtype(np.float32)
    ndarray = np.ndarray
    for i, g in enumerate(grafts):
        get = g.get
        if get("retired") or get("kind", "turn") == "recall":
            continue
        children = get("child_cents")
        if children and not digests:
            return None
        node_id = get("native_node_id")
        cent = get("cent")
        if node_id is None or (cent is None and "cent" not in g):
            return None
        if type(cent) is ndarray and cent.dtype == f32 and cent.ndim == 1:
            key = cent
        else:
            key = np.asarray(cent, dtype=np.float32).reshape(-1)
        n = key.shape[0]
        if n != dim:
            if dim is not None:
                return None
            dim = n
        nid = node_id if type(node_id) is int else int(node_id)
        if children:
            ks = [(key, cent)]
            for ch in children:
                k = np.asarray(ch, dtype=np.float32).reshape(-1)
                if k.shape[0] != dim:
                    return None
                ks.append((k, ch))
            d_nids.append(nid)
            d_keys.append(ks)
            d_gidx.append(i)
            if lengths:
                d_klen.append(route_key_length(g))
            continue
        add_row(key)
        add_nid(nid)
        add_cid(id(cent))
        add_g(i)
        if lengths:
            klen.append(route_key_length(g))
    if not rows and not d_nids:
        return None
    rs = RowSet(np.asarray(nids, dtype=np.uint64), np.asarray(cids, dtype=np.int64),
                np.full(len(rows), dim, dtype=np.int64))
    cents = [g["cent"] for g in (grafts[i] for i in gidx)]
    dg = _digest(d_nids, d_keys, d_gidx) if d_nids else None
    kl = (np.asarray(klen, dtype=np.int64), np.asarray(d_klen, dtype=np.int64)) if lengths else None
    return rs, rows, gidx, cents, dg, kl


def _gqa_key(cent):
    key = np.asarray(cent, dtype=np.float32)
    if key.ndim != 3 or any(int(d) <= 0 for d in key.shape):
        return None
    if not np.isfinite(key).all():
        return None
    return key


def _walk_gqa(grafts, digests: bool = False, lengths: bool = False):
    """The GQA walk (core/graft_arena.py:2933-2977): keys are
    ``[kv_heads, tokens, head_dim]``, may differ only in their token
    extent, and must be finite.  Returns ``(RowSet, rows, graft_indices,
    cents, Digest or None, key lengths or None)`` or None; ``digests`` and
    ``lengths`` as in the MLA walk."""
    rows, nids, cids, lens, gidx, cents = [], [], [], [], [], []
    d_nids, d_keys, d_gidx = [], [], []
    klen, d_klen = [], []
    geometry = None
    for i, g in enumerate(grafts):
        if g.get("retired") or g.get("kind", "turn") == "recall":
            continue
        node_id = g.get("native_node_id")
        children = g.get("child_cents")
        if node_id is None or (children and not digests) or "cent" not in g:
            return None
        cent = g["cent"]
        ks = [(cent, cent)] + [(ch, ch) for ch in (children or ())]
        checked = []
        for raw, obj in ks:
            key = _gqa_key(raw)
            if key is None:
                return None
            geo = (int(key.shape[0]), int(key.shape[2]))
            if geometry is None:
                geometry = geo
            elif geo != geometry:
                return None
            checked.append((key, obj))
        if children:
            d_nids.append(int(node_id))
            d_keys.append(checked)
            d_gidx.append(i)
            if lengths:
                d_klen.append(route_key_length(g))
            continue
        key = checked[0][0]
        rows.append(key)
        nids.append(int(node_id))
        cids.append(id(cent))
        lens.append(int(key.shape[1]))
        gidx.append(i)
        cents.append(cent)
        if lengths:
            klen.append(route_key_length(g))
    if not rows and not d_nids:
        return None
    rs = RowSet(np.asarray(nids, dtype=np.uint64), np.asarray(cids, dtype=np.int64),
                np.asarray(lens, dtype=np.int64))
    dg = _digest(d_nids, d_keys, d_gidx) if d_nids else None
    kl = (np.asarray(klen, dtype=np.int64), np.asarray(d_klen, dtype=np.int64)) if lengths else None
    return rs, rows, gidx, cents, dg, kl


def _reference_form(walk, shape_of):
    if walk is None or not walk[0].node_ids.size:
        return None
    rs, rows = walk[0], walk[1]
    sig = tuple((int(n), shape_of(r), r.dtype.str, int(c))
                for n, r, c in zip(rs.node_ids, rows, rs.cent_ids))
    return rs.node_ids, sig, rows


def mla_bank_walk(grafts):
    """Eligible MLA rows in the reference's form ``(node_ids uint64[N],
    signature, rows)``, signature entries ``(node_id, dim, dtype,
    id(cent))`` (core/graft_arena.py:1124-1162).  None when the arena has
    no attachable bank: a multi-row entry, a missing native id or centroid,
    mixed dims, or no rows."""
    return _reference_form(_walk_mla(grafts), lambda r: int(r.shape[0]))


def gqa_bank_walk(grafts):
    """Eligible GQA rows in the reference's form, signature entries
    ``(node_id, shape, dtype, id(cent))`` (core/graft_arena.py:2933-2977),
    or None."""
    return _reference_form(_walk_gqa(grafts), lambda r: tuple(int(d) for d in r.shape))


def plan_delta(old, new):
    """Evictions and appends that take the resident rows ``old`` (a RowSet,
    or None for an empty bank) to the rows ``new``.

    Returns ``(evict_ids uint64[], append_positions int64[])``.  Evicted
    are the resident node ids that left, or whose centroid object or
    extent changed.  Appended are the positions in ``new`` of rows that are
    new or changed, in row order.  Raises ValueError on a repeated node id
    in ``new``.
    """
    nn = new.node_ids
    if np.unique(nn).size != nn.size:
        raise ValueError("a node id appears twice")
    if old is None or old.node_ids.size == 0:
        return np.empty(0, dtype=np.uint64), np.arange(nn.size, dtype=np.int64)
    on = old.node_ids
    common, io, inew = np.intersect1d(on, nn, assume_unique=True, return_indices=True)
    changed = ((old.cent_ids[io] != new.cent_ids[inew])
               | (old.extents[io] != new.extents[inew]))
    gone = on[~np.isin(on, nn, assume_unique=True)]
    evict = np.concatenate([gone, common[changed]]).astype(np.uint64)
    add = ~np.isin(nn, on, assume_unique=True)
    add[inew[changed]] = True
    return evict, np.flatnonzero(add).astype(np.int64)


class _Bridge:
    """Shared epoch gate, walk, delta and exclude-aware route order."""

    _full_walk = None

    def __init__(self, *, dtype: str = "f32", headroom: float = 1.25,
                 length_debias: bool = False, route_profile: bool = False):
        if headroom < 1.0:
            raise ValueError("headroom must be >= 1")
        self.dtype = dtype
        self.headroom = float(headroom)
        self.length_debias = bool(length_debias)
        self.route_profile = bool(route_profile)
        self.last_route_receipt = None
        self.route_receipt_history: list = []
        self._receipt = None           # the route being profiled
        self._refresh_ms = 0.0         # refresh time since the last route
        self.bank = None               # single-key nodes
        self.side = None               # digest nodes' keys, ids 0..keys-1
        self._epoch = None
        self._eligible_bank = False
        self._resident = None          # RowSet on the device
        self._pinned: list = []
        self._digest = None            # Digest held by the side bank
        self._side_owner = np.empty(0, dtype=np.int64)   # digest node of each side key
        self._klen_main = np.empty(0, dtype=np.int64)
        self._klen_digest = np.empty(0, dtype=np.int64)
        self._sorted_nid = np.empty(0, dtype=np.uint64)
        self._sorted_gidx = np.empty(0, dtype=np.int64)
        self._in_bank = np.zeros(0, dtype=bool)
        self.last_event: dict = {}
        self.totals = {"appended": 0, "evicted": 0, "rebuilt": 0,
                       "bytes_uploaded": 0}

    # --------------------------------------------------------- lifecycle
    def close(self) -> None:
        for b in (self.bank, self.side):
            if b is not None:
                b.close()
        self.bank = None
        self.side = None
        self._digest = None
        self._resident = None
        self._pinned = []
        self._epoch = None
        self._eligible_bank = False

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def bank_size(self) -> int:
        """Nodes the bridge routes: single-key rows plus digest nodes."""
        if not self._eligible_bank or self._resident is None:
            return 0
        d = 0 if self._digest is None else int(self._digest.node_ids.size)
        return int(self._resident.node_ids.size) + d

    def refresh(self, grafts, epoch: int) -> dict:
        """Bring the device bank in step with ``grafts`` at ``epoch``.

        Epoch unchanged: O(1), nothing walked (``reused`` /
        ``ineligible_reused``).  Otherwise the walk runs; unchanged rows
        keep the bank (``signature_reused``); changed ones are applied as
        evictions and appends (``updated``; ``rebuilt`` when the bank had
        to grow), or as a first upload (``created``).  Digest nodes' keys
        go to the side bank, which is built again when they change.
        Returns the event (also ``last_event``).
        """
        t0 = time.perf_counter()
        try:
            return self._refresh(grafts, epoch, t0)
        finally:
            self._refresh_ms += (time.perf_counter() - t0) * 1.0e3

    def _refresh(self, grafts, epoch: int, t0: float) -> dict:
        if self._epoch is not None and epoch == self._epoch:
            self.last_event = {
                "status": "reused" if self._eligible_bank else "ineligible_reused",
                "epoch": int(epoch), "signature_walk": False}
            return self.last_event
        walk = type(self)._full_walk(grafts, True, self.length_debias)
        if walk is None:
            self._epoch = epoch
            # The device bank stays allocated: a later epoch may make the
            # arena eligible again, and the delta then starts from it.
            self._eligible_bank = False
            self.last_event = {"status": "ineligible", "epoch": int(epoch),
                               "signature_walk": True}
            return self.last_event
        rs, rows, gidx, cents, dg, klen = walk
        # Reverse map, native node id -> graft index: row i is the i-th
        # eligible graft (core/graft_arena.py:1200-1245, 3205-3262).  A
        # repeated id fails closed.
        all_nid = rs.node_ids if dg is None else np.concatenate([rs.node_ids, dg.node_ids])
        g = np.asarray(gidx + ([] if dg is None else dg.gidx), dtype=np.int64)
        order = np.argsort(all_nid, kind="stable")
        snid = all_nid[order]
        if snid.size > 1 and np.any(snid[1:] == snid[:-1]):
            self._epoch = epoch
            self._eligible_bank = False
            self.last_event = {"status": "ineligible", "epoch": int(epoch),
                               "signature_walk": True,
                               "reason": "duplicate native id"}
            return self.last_event
        self._sorted_nid, self._sorted_gidx = snid, g[order]
        self._in_bank = np.zeros(len(grafts), dtype=bool)
        self._in_bank[g] = True
        if klen is not None:
            self._klen_main, self._klen_digest = klen
        n_digest = 0 if dg is None else int(dg.node_ids.size)
        side_same = (dg is None and self._digest is None) or (
            dg is not None and self._digest is not None and dg.sig == self._digest.sig
            and np.array_equal(dg.node_ids, self._digest.node_ids))
        main_same = (self._resident is not None and rs.same(self._resident)
                     and (self.bank is not None or not rs.node_ids.size))
        if main_same and side_same:
            self._epoch = epoch
            self._eligible_bank = True
            self._pinned = cents
            if dg is not None:
                self._digest = dg
            self.last_event = {"status": "signature_reused", "epoch": int(epoch),
                               "signature_walk": True,
                               "node_count": int(rs.node_ids.size) + n_digest}
            return self.last_event
        # Fail closed (core/graft_arena.py:1270-1281): until the device bank
        # holds exactly this row set the route is unavailable, and an error
        # part-way through an update leaves no epoch that a retry could
        # take as current; the bank, in an unknown state, is dropped.
        self._eligible_bank = False
        self._epoch = None
        moved = 0
        status, evicted, appended = "updated", 0, 0
        try:
            if not main_same:
                if self.bank is None:
                    if rs.node_ids.size:
                        moved += self._create(rs.node_ids, rows)
                    status, appended = "created", int(rs.node_ids.size)
                else:
                    evict_ids, append_pos = plan_delta(self._resident, rs)
                    m, rebuilt = self._apply(evict_ids, append_pos, rs.node_ids, rows)
                    moved += m
                    status = "rebuilt" if rebuilt else "updated"
                    evicted, appended = int(evict_ids.size), int(append_pos.size)
                    if rebuilt:
                        self.totals["rebuilt"] += 1
            if not side_same:
                if self.side is not None:
                    self.side.close()
                    self.side = None
                self._digest = None
                if dg is not None:
                    moved += self._create_side(dg.keys)
                    self._side_owner = np.repeat(np.arange(n_digest, dtype=np.int64),
                                                 np.diff(dg.offs))
                    self._digest = dg
        except BaseException:
            self.close()
            raise
        self._epoch = epoch
        self._resident = rs
        # The row set holds id(cent); keeping the resident centroid objects
        # alive means no later object can take one of those ids while its
        # row is on the device (a recycled id would read as "unchanged").
        # The Digest keeps the digest keys' objects.
        self._pinned = cents
        self._eligible_bank = True
        self.totals["appended"] += appended
        self.totals["evicted"] += evicted
        self.totals["bytes_uploaded"] += moved
        self.last_event = {
            "status": status, "epoch": int(epoch), "signature_walk": True,
            "node_count": int(rs.node_ids.size) + n_digest, "appended": appended,
            "evicted": evicted, "bytes_uploaded": int(moved),
            "digest_nodes": n_digest,
            "digest_keys": 0 if dg is None else len(dg.keys),
            "seconds": time.perf_counter() - t0}
        return self.last_event

    # ------------------------------------------------------------- route
    def _route_main(self, query, topk: int):
        raise NotImplementedError

    def _score_main(self, query, node_ids):
        raise NotImplementedError

    def _score_side(self, query):
        raise NotImplementedError

    def _digest_scores(self, query) -> np.ndarray:
        """Each digest node's best finite key score, NaN when none is
        finite (cpp/grm_runtime.cpp:3518-3545, 3031-3051)."""
        dg = self._digest
        ks = self._score_side(query)
        out = np.full(dg.node_ids.size, -np.inf, dtype=np.float32)
        fin = np.isfinite(ks)
        np.maximum.at(out, self._side_owner[fin], ks[fin])
        out[out == -np.inf] = np.nan
        return out

    def route_scored(self, query, topk: int):
        """The best ``topk`` nodes for one query: (node ids uint64[topk],
        scores float64[topk]), unfilled UINT64_MAX / NaN, ranked by score
        (descending) then node id.  Scores are the law's (float32 values);
        with ``length_debias`` they are the debiased float64 scores the
        ranking uses."""
        ids_out = np.full(topk, np.iinfo(np.uint64).max, dtype=np.uint64)
        sc_out = np.full(topk, np.nan, dtype=np.float64)
        if not self._eligible_bank or topk <= 0:
            return ids_out, sc_out
        main_n = int(self._resident.node_ids.size)
        t = self._clock()
        if self.length_debias:
            ids = self._resident.node_ids
            sc = (self._score_main(query, ids) if main_n
                  else np.empty(0, dtype=np.float32))
            kl = self._klen_main
            t = self._term("device_score_all_ms", t)
            if self._digest is not None:
                ids = np.concatenate([ids, self._digest.node_ids])
                sc = np.concatenate([sc, self._digest_scores(query)])
                kl = np.concatenate([kl, self._klen_digest])
                t = self._term("device_digest_score_ms", t)
            score = apply_length_debias(sc, kl)
        else:
            ids = np.empty(0, dtype=np.uint64)
            sc = np.empty(0, dtype=np.float32)
            if main_n:
                ids, sc = self._route_main(query, min(topk, main_n, MAX_TOPK))
                keep = ids != np.iinfo(np.uint64).max
                ids, sc = ids[keep], sc[keep]
                t = self._term("device_route_call_ms", t)
            if self._digest is not None:
                ids = np.concatenate([ids, self._digest.node_ids])
                sc = np.concatenate([sc, self._digest_scores(query)])
                t = self._term("device_digest_score_ms", t)
            score = sc.astype(np.float64)
        fin = np.isfinite(score)
        ids, score = ids[fin], score[fin]
        order = np.lexsort((ids, -score))[:topk]
        ids_out[:order.size] = ids[order]
        sc_out[:order.size] = score[order]
        self._term("ranking_ms", t)
        return ids_out, sc_out

    def _graft_index(self, nid) -> int | None:
        i = int(np.searchsorted(self._sorted_nid, np.uint64(nid)))
        if i < self._sorted_nid.size and int(self._sorted_nid[i]) == int(nid):
            return int(self._sorted_gidx[i])
        return None

    # ----------------------------------------------------------- receipts
    def _profiling(self) -> bool:
        return self.route_profile or route_profile_env()

    def _clock(self):
        return time.perf_counter_ns() if self._receipt is not None else None

    def _term(self, name: str, started):
        """Add the time since ``started`` to term ``name`` of the receipt
        being built; returns a new start (None when not profiling)."""
        if started is None or self._receipt is None:
            return None
        now = time.perf_counter_ns()
        terms = self._receipt["terms_ms"]
        terms[name] = terms.get(name, 0.0) + (now - started) / 1.0e6
        return now

    def _fallback(self, reason: str) -> None:
        if self._receipt is not None and reason not in self._receipt["fallbacks"]:
            self._receipt["fallbacks"].append(reason)

    def route_order(self, query, limit: int, exclude=(), cand_count=None):
        """Graft indices of the best ``limit`` nodes, or None (the caller's
        CPU path); with route profiling on, the route's receipt goes to
        ``last_route_receipt`` (module docstring)."""
        refresh_ms, self._refresh_ms = self._refresh_ms, 0.0
        if not self._profiling():
            self.last_route_receipt = None
            return self._route_order(query, limit, exclude, cand_count)
        receipt = {
            "schema": ROUTE_RECEIPT_SCHEMA,
            "epoch": None if self._epoch is None else int(self._epoch),
            "terms_ms": {"bank_refresh_ms": refresh_ms},
            "rebuilds": {"device_bank": dict(self.last_event)},
            "parity": {"checked": False, "ok": None},
            "fallbacks": [],
        }
        self._receipt = receipt
        t0 = time.perf_counter_ns()
        try:
            out = self._route_order(query, limit, exclude, cand_count)
        finally:
            self._receipt = None
        receipt["route_backend"] = "hip" if out is not None else None
        receipt["candidate_count"] = self.bank_size
        if out is not None:
            receipt["ranking_count"] = len(out)
            receipt["ranking_prefix"] = [int(i) for i in out[:16]]
        receipt["terms_ms"]["route_wall_ms"] = (time.perf_counter_ns() - t0) / 1.0e6
        self.last_route_receipt = receipt
        self.route_receipt_history.append(receipt)
        return out

    def _route_order(self, query, limit: int, exclude=(), cand_count=None):
        """Graft indices of the best ``limit`` nodes, excluded indices
        dropped.  Follows core/graft_arena.py:1282-1364:

        * ask the bank for ``min(16, bank_size, want + excludes in bank)``;
        * map node ids back through the reverse map and drop excluded
          indices;
        * if the ask would be cut below ``want``, or too few rows survive,
          return None, which sends the caller to its CPU path.

        ``cand_count``, when given, must equal the bank size minus the
        excludes in the bank, else None (the reference's fail-closed
        candidate check).
        """
        if limit is None:
            self._fallback("requires_limited_route")
            return None
        if not self._eligible_bank:
            self._fallback("bank_ineligible")
            return None
        size = self.bank_size
        exclude_set = set(exclude) if exclude else None
        n_g = self._in_bank.size
        in_bank = (sum(1 for i in exclude_set if 0 <= i < n_g and self._in_bank[i])
                   if exclude_set else 0)
        if cand_count is not None and int(cand_count) != size - in_bank:
            self._fallback("candidate_subset_mismatch")
            return None
        want = min(max(0, int(limit)), size - in_bank)
        if want <= 0:
            return []
        topk = min(MAX_TOPK, size, want + in_bank)
        if topk < want:
            self._fallback("topk_cap")
            return None
        ranked = self.route_scored(query, topk)[0]
        t = self._clock()
        out = []
        for nid in ranked:
            if nid == np.iinfo(np.uint64).max:
                continue
            gi = self._graft_index(nid)
            if gi is None or (exclude_set is not None and gi in exclude_set):
                continue
            out.append(gi)
            if len(out) >= want:
                break
        self._term("result_remap_ms", t)
        if len(out) < want:
            self._fallback("short_result")
            return None
        return out


class MlaRouteBankBridge(_Bridge):
    """MLA arena bridge (one flat centroid per node)."""

    _full_walk = staticmethod(_walk_mla)

    def _create(self, node_ids, rows):
        stacked = np.ascontiguousarray(np.stack(rows), dtype=np.float32)
        cap = int(np.ceil(stacked.shape[0] * self.headroom))
        self.bank = MlaNodeBank(stacked, node_ids, dtype=self.dtype,
                                capacity=cap)
        return self._bytes(stacked.shape[0], stacked.shape[1])

    def _bytes(self, n, dim):
        return int(n) * int(dim) * (4 if self.dtype == "f32" else 2)

    def _apply(self, evict_ids, append_pos, node_ids, rows):
        bank = self.bank
        dim = bank.dim
        if any(rows[p].shape[0] != dim for p in append_pos):
            # A new dim cannot share the bank: rebuild over the new rows.
            self.bank.close()
            self.bank = None
            return self._create(node_ids, rows), True
        info = bank.info()
        room = info["capacity"] - (info["live"] - len(evict_ids))
        if len(append_pos) > room:
            self.bank.close()
            self.bank = None
            stacked = np.ascontiguousarray(np.stack(rows), dtype=np.float32)
            cap = max(int(np.ceil(stacked.shape[0] * self.headroom)),
                      2 * int(info["capacity"]))
            self.bank = MlaNodeBank(stacked, node_ids, dtype=self.dtype,
                                    capacity=cap)
            return self._bytes(stacked.shape[0], dim), True
        if evict_ids.size:
            bank.evict(evict_ids)
        if append_pos.size:
            add = np.ascontiguousarray(np.stack([rows[p] for p in append_pos]),
                                       dtype=np.float32)
            bank.append(add, node_ids[append_pos])
        return self._bytes(append_pos.size, dim), False

    def _create_side(self, keys):
        stacked = np.ascontiguousarray(np.stack(keys), dtype=np.float32)
        self.side = MlaNodeBank(stacked, np.arange(len(keys), dtype=np.uint64),
                                dtype=self.dtype)
        return self._bytes(stacked.shape[0], stacked.shape[1])

    def _route_main(self, query, topk):
        q = np.ascontiguousarray(query, dtype=np.float32).reshape(1, -1)
        r = self.bank.route(q, topk)
        return r.ids[0], r.scores[0]

    def _score_main(self, query, node_ids):
        return self.bank.score_nodes(np.asarray(query, dtype=np.float32).reshape(-1), node_ids)

    def _score_side(self, query):
        n = len(self._digest.keys)
        return self.side.score_nodes(np.asarray(query, dtype=np.float32).reshape(-1),
                                     np.arange(n, dtype=np.uint64))


class GqaRouteBankBridge(_Bridge):
    """GQA arena bridge (ragged ``[kv_heads, tokens, head_dim]`` keys)."""

    _full_walk = staticmethod(_walk_gqa)
    _TOK_ALIGN = 8  # the bank pads each node block to a multiple of 8 rows

    def _padded(self, rows):
        a = self._TOK_ALIGN
        return sum((int(r.shape[1]) + a - 1) // a * a for r in rows)

    def _flat(self, rows):
        return np.concatenate([np.ascontiguousarray(r, dtype=np.float32).reshape(-1)
                               for r in rows])

    def _elem(self):
        return 4 if self.dtype == "f32" else 2

    def _create(self, node_ids, rows, min_nodes=0, min_tokens=0):
        kv, _, hd = rows[0].shape
        counts = np.asarray([r.shape[1] for r in rows], dtype=np.uint64)
        offs = np.zeros(len(rows) + 1, dtype=np.uint64)
        offs[1:] = np.cumsum(counts)
        cap_nodes = max(int(np.ceil(len(rows) * self.headroom)), int(min_nodes))
        cap_tokens = max(int(np.ceil(self._padded(rows) * self.headroom)),
                         int(min_tokens))
        self.bank = GqaNodeBank(self._flat(rows), offs, kv_heads=int(kv),
                                head_dim=int(hd), node_ids=node_ids,
                                dtype=self.dtype, capacity_nodes=cap_nodes,
                                capacity_tokens=cap_tokens)
        return int(offs[-1]) * int(kv) * int(hd) * self._elem()

    def _apply(self, evict_ids, append_pos, node_ids, rows):
        bank = self.bank
        if not rows:
            # every single-key node left (digest nodes may remain)
            if evict_ids.size:
                bank.evict(evict_ids)
            return 0, False
        kv, _, hd = rows[0].shape
        if (kv, hd) != (bank.kv_heads, bank.head_dim):
            self.bank.close()
            self.bank = None
            return self._create(node_ids, rows), True
        if evict_ids.size:
            bank.evict(evict_ids)
        add = [rows[p] for p in append_pos]
        need_tok = self._padded(add)
        info = bank.info()
        node_room = info["capacity_nodes"] - info["live"]
        if need_tok > info["capacity_tokens"] - info["tokens_in_use"]:
            bank.compact()
            info = bank.info()
        if (len(add) > node_room
                or need_tok > info["capacity_tokens"] - info["tokens_in_use"]):
            old = info
            self.bank.close()
            self.bank = None
            moved = self._create(node_ids, rows,
                                 min_nodes=2 * int(old["capacity_nodes"]),
                                 min_tokens=2 * int(old["capacity_tokens"]))
            return moved, True
        if add:
            counts = np.asarray([r.shape[1] for r in add], dtype=np.uint64)
            bank.append(self._flat(add), counts, node_ids[append_pos])
            return int(counts.sum()) * int(kv) * int(hd) * self._elem(), False
        return 0, False

    def _create_side(self, keys):
        kv, _, hd = keys[0].shape
        counts = np.asarray([k.shape[1] for k in keys], dtype=np.uint64)
        offs = np.zeros(len(keys) + 1, dtype=np.uint64)
        offs[1:] = np.cumsum(counts)
        self.side = GqaNodeBank(self._flat(keys), offs, kv_heads=int(kv), head_dim=int(hd),
                                node_ids=np.arange(len(keys), dtype=np.uint64),
                                dtype=self.dtype)
        return int(offs[-1]) * int(kv) * int(hd) * self._elem()

    @staticmethod
    def _query3(query):
        q = np.ascontiguousarray(query, dtype=np.float32)
        return q[0] if q.ndim == 4 else q

    def _route_main(self, query, topk):
        r = self.bank.route(self._query3(query)[None], topk, query_dtype="f32")
        return r.ids[0], r.scores[0]

    def _score_main(self, query, node_ids):
        return self.bank.score_nodes(self._query3(query), node_ids)

    def _score_side(self, query):
        n = len(self._digest.keys)
        return self.side.score_nodes(self._query3(query), np.arange(n, dtype=np.uint64))


__all__ = ["MlaRouteBankBridge", "GqaRouteBankBridge", "RowSet", "Digest", "mla_bank_walk",
           "gqa_bank_walk", "plan_delta", "route_key_length", "length_debias_factor",
           "apply_length_debias"]
