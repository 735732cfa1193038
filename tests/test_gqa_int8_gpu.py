"""Large ragged GQA route over INT8 graft storage on the GPU.

Workload: node lengths lognormal (median 256, sigma 0.5, capped at 4096),
8 kv heads x head_dim 128: N(0, 1) keys quantised to INT8 codes with one
fp16 scale per (kv head, token) row (the packed graft format's quantiser,
core/graft_quant.py:93-131, group = head_dim; dequantised as
fp16(code * scale), :136-144), 32 query heads in bf16, 16 queries batched,
top-5, with 1% of the nodes evicted and as many appended between routes.

* At a size the oracle finishes in seconds: node ids and scores bit-exact
  against the oracle's route over the live nodes after every churn round.
* At the full 100,000-node size (about 30 GB of codes), before and after a
  1% churn round:
  - the certified screen path against the exact fp64 path of the same
    library (ids and score bits, all 16 queries);
  - 2 of the 16 queries through the oracle over every live node (ids and
    score bits);
  - the other queries: the returned nodes plus a random sample of 2,000
    nodes through the oracle (its top-5 over that subset must be the GPU's
    global top-5, scores bit-exact).
"""

import os

import numpy as np
import pytest

import oracle
from graftrepository_amd import GqaNodeBank, workloads as wl
from graftrepository_amd.node_bank import bf16_bits_to_f32

pytestmark = pytest.mark.gpu
NO_ID = np.iinfo(np.uint64).max
KV, HD, H = 8, 128, 32


def assert_same(res, want_ids, want_scores):
    np.testing.assert_array_equal(res.ids, want_ids)
    filled = want_ids != NO_ID
    assert np.all(np.isnan(res.scores[~filled]))
    np.testing.assert_array_equal(res.scores[filled].view(np.uint32),
                                  want_scores[filled].view(np.uint32))


class HostMirror:
    """Host copy of the live nodes: id -> (codes block, scales block, L)."""

    def __init__(self):
        self.nodes = {}

    def add(self, codes, scales, offs, ids):
        for j, nid in enumerate(np.asarray(ids, np.uint64).tolist()):
            a, b = int(offs[j]), int(offs[j + 1])
            self.nodes[nid] = (codes[a * KV * HD:b * KV * HD], scales[a * KV:b * KV], b - a)

    def drop(self, ids):
        for nid in np.asarray(ids, np.uint64).tolist():
            del self.nodes[nid]

    def bank(self, ids=None):
        keys = sorted(self.nodes) if ids is None else [int(i) for i in ids]
        lens = np.asarray([self.nodes[i][2] for i in keys], np.uint64)
        offs = np.zeros(len(keys) + 1, np.uint64)
        offs[1:] = np.cumsum(lens)
        codes = np.concatenate([self.nodes[i][0] for i in keys])
        scales = np.concatenate([self.nodes[i][1] for i in keys])
        return codes, scales, offs, np.asarray(keys, np.uint64)

    def route(self, qf, k, ids=None):
        codes, scales, offs, nid = self.bank(ids)
        return oracle.gqa_route(codes, oracle.I8, offs, KV, HD, qf, k, scales=scales,
                                scale_dtype="f16", group_size=HD, node_ids=nid,
                                threads=min(16, os.cpu_count() or 1))


def lognormal_lengths(n, seed):
    cfg = wl.GQA_INT8
    return wl.gqa_lengths(n, seed, kind="lognormal", median=cfg["median"],
                          sigma=cfg["sigma"], cap=cfg["cap"])


def test_int8_lognormal_churn_matches_oracle(hip_lib):
    n = 1500
    lens = lognormal_lengths(n, 81)
    lens[:3] = 4096   # the length cap
    lens[3:5] = 1
    codes, scales, offs = wl.gqa_int8_bank(lens, KV, HD, seed=81)
    ids0 = np.arange(n, dtype=np.uint64) * 3 + 11
    qs = wl.gqa_queries(16, H, 1, HD, seed=81, dtype="bf16")
    qf = bf16_bits_to_f32(qs).reshape(qs.shape)
    mirror = HostMirror()
    mirror.add(codes, scales, offs, ids0)
    rng = np.random.default_rng(82)
    with GqaNodeBank(codes, offs, kv_heads=KV, head_dim=HD, node_ids=ids0, dtype="i8",
                     scales=scales, scale_dtype="f16", group_size=HD,
                     capacity_nodes=n + 100, capacity_tokens=int(offs[-1]) + 60_000) as bank:
        for rnd in range(3):
            res = bank.route(qs, 5, query_dtype="bf16")
            ids, sc, _ = mirror.route(qf, 5)
            assert_same(res, ids, sc)
            ev = rng.choice(np.asarray(sorted(mirror.nodes), np.uint64), size=15, replace=False)
            bank.evict(ev)
            mirror.drop(ev)
            nl = lognormal_lengths(15, 90 + rnd)
            nc, ns, no = wl.gqa_int8_bank(nl, KV, HD, seed=90 + rnd)
            nid = np.arange(15, dtype=np.uint64) + 100_000 + 100 * rnd
            bank.append(nc, nl, nid, scales=ns)
            mirror.add(nc, ns, no, nid)
        res = bank.route(qs, 5, query_dtype="bf16")
        ids, sc, _ = mirror.route(qf, 5)
        assert_same(res, ids, sc)


@pytest.mark.timeout(1100)
def test_int8_config_size_screen_vs_exact_and_oracle(hip_lib):
    cfg = wl.GQA_INT8
    n, k = cfg["nodes"], cfg["topk"]
    lens = lognormal_lengths(n, cfg["seed"])
    codes, scales, offs = wl.gqa_int8_bank(lens, KV, HD, seed=cfg["seed"])
    print(f"[int8 config] {n} nodes, {int(offs[-1])} tokens, {codes.size / 1e9:.1f} GB codes",
          flush=True)
    qs = wl.gqa_queries(cfg["queries"], H, 1, HD, seed=cfg["seed"], dtype="bf16")
    qf = bf16_bits_to_f32(qs).reshape(qs.shape)
    ids0 = np.arange(n, dtype=np.uint64)
    kw = dict(kv_heads=KV, head_dim=HD, node_ids=ids0, dtype="i8", scales=scales,
              scale_dtype="f16", group_size=HD, capacity_nodes=n + 2000,
              capacity_tokens=int(offs[-1]) + 2_000_000)
    mirror = HostMirror()
    mirror.add(codes, scales, offs, ids0)
    rng = np.random.default_rng(83)
    with GqaNodeBank(codes, offs, **kw) as fast:
        os.environ["GRM_HIP_GQA_SCREEN"] = "0"
        try:
            exact = GqaNodeBank(codes, offs, **kw)
        finally:
            del os.environ["GRM_HIP_GQA_SCREEN"]
        with exact:
            for rnd in range(2):
                r1 = fast.route(qs, k, query_dtype="bf16")
                r2 = exact.route(qs, k, query_dtype="bf16")
                assert_same(r1, r2.ids, r2.scores)
                live = np.asarray(sorted(mirror.nodes), np.uint64)
                sample = np.union1d(r1.ids.reshape(-1),
                                    rng.choice(live, size=2000, replace=False))
                ids, sc, _ = mirror.route(qf, k, ids=sample)
                assert_same(r1, ids, sc)
                # two whole queries through the oracle over every live node
                # (the first round routes the generated arrays as they are)
                full = [0, 1 + 7 * rnd]
                if rnd == 0:
                    ids, sc, _ = oracle.gqa_route(
                        codes, oracle.I8, offs, KV, HD, qf[full], k, scales=scales,
                        scale_dtype="f16", group_size=HD, node_ids=ids0,
                        threads=min(16, os.cpu_count() or 1))
                else:
                    ids, sc, _ = mirror.route(qf[full], k)
                np.testing.assert_array_equal(r1.ids[full], ids)
                np.testing.assert_array_equal(r1.scores[full].view(np.uint32),
                                              sc.view(np.uint32))
                print(f"[int8 config] round {rnd}: screen path == exact path; oracle "
                      f"on {sample.size} nodes, and queries {full} on all {live.size} "
                      f"nodes", flush=True)
                ev = rng.choice(live, size=n // 100, replace=False)
                fast.evict(ev)
                exact.evict(ev)
                mirror.drop(ev)
                nl = lognormal_lengths(n // 100, 95 + rnd)
                nc, ns, no = wl.gqa_int8_bank(nl, KV, HD, seed=95 + rnd)
                nid = np.arange(n // 100, dtype=np.uint64) + 10 * n + n * rnd
                fast.append(nc, nl, nid, scales=ns)
                exact.append(nc, nl, nid, scales=ns)
                mirror.add(nc, ns, no, nid)
