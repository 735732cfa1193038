"""The screens' error bounds, held pair by pair on inputs built to stress them.

Both matrix-core screens rest on a proven bound between a screened value and
the law's value:

* batched MLA (bf16 MFMA 32x32x16): |s~ - score| <= B per query, the
  certificate's margin (law: cpp/grm_runtime.cpp:3518-3545);
* GQA (bf16/f16 MFMA 16x16x32, INT8 dequantised or factored, fp32 banks
  through their fp16 key copy, whose rounding the bound carries):
  |m - scale * max_t |q . k_t|| <= E = coef * K + eabs per (node, kv head,
  query column) (law: cpp/grm_runtime.cpp:2980-3029), with E = +inf where
  the fp32 accumulation could overflow (K >= kcap).

The library's probe entries run the production screen kernels and return
the screened values with the bounds the route would use; these tests check
every pair against the oracle's fp64 law on banks mixing signs, exponents
over a wide range, pairwise cancellation, subnormal and zero rows, and
magnitudes near the fp32 overflow threshold.  Those banks are then routed
for real on every GQA path and must give the oracle's ids and score bits.
"""

import numpy as np
import pytest

import oracle
from graftrepository_amd import GqaNodeBank, MlaNodeBank
from graftrepository_amd.node_bank import as_bf16_bits, bf16_bits_to_f32

pytestmark = pytest.mark.gpu
NO_ID = np.iinfo(np.uint64).max


def spread(rng, shape, lo, hi):
    """Values sign * 2^U(lo, hi) * U(1, 2): mixed signs, wide exponents."""
    e = rng.uniform(lo, hi, size=shape)
    return (rng.choice([-1.0, 1.0], size=shape) * np.exp2(e) * rng.uniform(1, 2, size=shape))


def cancelling(rng, shape, noise):
    """Rows (x0, -x0, x1, -x1, ...) plus a small perturbation: their dot
    with a query of equal pairs cancels down to the perturbation."""
    x = rng.standard_normal(shape[:-1] + (shape[-1] // 2,))
    out = np.repeat(x, 2, axis=-1)
    out[..., 1::2] *= -1.0
    return out + noise * rng.standard_normal(shape)


def paired(rng, shape):
    x = rng.standard_normal(shape[:-1] + (shape[-1] // 2,))
    return np.repeat(x, 2, axis=-1)


# ------------------------------------------------------------------- MLA

def mla_rows(rng, n, dim, adversarial):
    fam = np.array_split(np.arange(n), 6 if adversarial else 3)
    rows = np.empty((n, dim))
    rows[fam[0]] = rng.standard_normal((fam[0].size, dim))
    rows[fam[1]] = spread(rng, (fam[1].size, dim), -40, 40)
    rows[fam[2]] = cancelling(rng, (fam[2].size, dim), 2.0 ** -12)
    if adversarial:
        rows[fam[3]] = spread(rng, (fam[3].size, dim), -133, -118)  # subnormal bf16 included
        rows[fam[4]] = spread(rng, (fam[4].size, dim), 90, 110)
        rows[fam[5]] = rng.standard_normal((fam[5].size, dim))
        rows[fam[5][::7]] = 0.0
    return as_bf16_bits(rows.astype(np.float32))


def mla_queries(rng, count, dim):
    fam = np.array_split(np.arange(count), 5)
    q = np.empty((count, dim))
    q[fam[0]] = rng.standard_normal((fam[0].size, dim))
    q[fam[1]] = spread(rng, (fam[1].size, dim), -30, 30)
    q[fam[2]] = paired(rng, (fam[2].size, dim))
    q[fam[3]] = spread(rng, (fam[3].size, dim), -100, -90)
    q[fam[4]] = spread(rng, (fam[4].size, dim), 20, 30)
    return q.astype(np.float32)


@pytest.mark.parametrize("adversarial", [False, True])
@pytest.mark.parametrize("query_dtype", ["bf16", "f32"])
@pytest.mark.parametrize("count", [80, 256])  # 256: the full-pass screen (queries in registers)
def test_mla_batched_screen_obeys_its_bound(hip_lib, adversarial, query_dtype, count):
    rng = np.random.default_rng(17 + adversarial)
    n, dim = 2048, 288
    bits = mla_rows(rng, n, dim, adversarial)
    rows = bf16_bits_to_f32(bits)
    qf = mla_queries(rng, count, dim)
    if query_dtype == "bf16":
        qf = bf16_bits_to_f32(as_bf16_bits(qf))  # the values the law sees
    with MlaNodeBank(bits, np.arange(n, dtype=np.uint64), dtype="bf16") as bank:
        vals, bounds, ids = bank.probe_screen(qf, query_dtype=query_dtype)
    assert vals.shape == (count, n)
    np.testing.assert_array_equal(ids, np.arange(n, dtype=np.uint64))
    score = oracle.mla_scores(rows, qf)
    norms = oracle.mla_row_norms(rows).astype(np.float64)
    nmax = norms[np.isfinite(norms)].max()
    qn = np.array([oracle.mla_qnorm(q) for q in qf])
    big = qn * nmax
    # B is established exactly where ||q|| * max norm < 2^125
    assert np.all(np.isfinite(bounds[big < 2.0 ** 124]))
    assert np.all(np.isinf(bounds[big > 2.0 ** 126]))
    fin = np.isfinite(bounds)
    assert fin.sum() >= 48
    err = np.abs(vals[fin].astype(np.float64) - score[fin].astype(np.float64))
    ratio = err / bounds[fin, None]
    assert np.all(ratio <= 1.0), f"worst |s~ - score| / B = {ratio.max():.3g}"
    if not adversarial:
        # the bound is not vacuous on ordinary data (Gaussian and paired
        # queries; tiny queries make the law's 1e-8 term dominate B): well
        # under the score scale, and not far above the errors seen
        ordinary = np.r_[0:16, 32:48]
        assert np.all(bounds[ordinary] < 2.0 ** -6)
        assert ratio.max() > 1e-3


# ------------------------------------------------------------------- GQA

def gqa_bank(rng, kind, n, kv, hd):
    lens = rng.integers(1, 7, size=n).astype(np.uint64)
    lens[::3] = 1  # single-token nodes: the maximum is the pair itself
    offs = np.zeros(n + 1, np.uint64)
    offs[1:] = np.cumsum(lens)
    fam = np.arange(n) % 6
    blocks = []
    # fp32 banks are screened through an fp16 copy: their wide, tiny and
    # huge families straddle its normal range, subnormals and maximum
    wide = {"bf16": (-60, 60), "f32": (-20, 20)}.get(kind, (-12, 12))
    tiny = {"bf16": (-133, -120), "f32": (-30, -16)}.get(kind, (-24, -14))
    huge = {"bf16": (100, 118), "f32": (14, 18)}.get(kind, (10, 14))
    for i in range(n):
        shape = (kv, int(lens[i]), hd)
        f = fam[i]
        if f == 0:
            b = rng.standard_normal(shape)
        elif f == 1:
            b = spread(rng, shape, *wide)
        elif f == 2:
            b = cancelling(rng, shape, 2.0 ** -10)
        elif f == 3:
            b = spread(rng, shape, *tiny)
        elif f == 4:
            b = spread(rng, shape, *huge)
        else:
            b = rng.standard_normal(shape)
            b[:, ::2] = 0.0
        blocks.append(b.reshape(-1))
    vals = np.concatenate(blocks).astype(np.float32)
    if kind == "bf16":
        bits = as_bf16_bits(vals)
        return dict(keys=bits, law=bf16_bits_to_f32(bits), code=oracle.BF16), offs
    if kind == "f16":
        h = vals.astype(np.float16)
        return dict(keys=h.view(np.uint16), law=h.astype(np.float32), code=oracle.F16), offs
    if kind == "f32":
        return dict(keys=vals, law=vals, code=oracle.F32), offs
    codes, scales = oracle.quantize_int8(vals.reshape(-1, hd), hd, "f16")
    law = oracle.dequantize_int8(codes, scales, hd, "f16").reshape(-1)
    return dict(keys=codes, scales=scales, law=law, code=oracle.I8), offs


def gqa_query(rng, H, Qt, hd, kind):
    fam = np.arange(H) % 5
    q = np.empty((H, Qt, hd))
    hi = 100 if kind == "bf16" else 10
    for h in range(H):
        f = fam[h]
        if f == 0:
            q[h] = rng.standard_normal((Qt, hd))
        elif f == 1:
            q[h] = spread(rng, (Qt, hd), -30, 30)
        elif f == 2:
            q[h] = paired(rng, (Qt, hd))
        elif f == 3:
            q[h] = spread(rng, (Qt, hd), -100, -90)
        else:
            q[h] = spread(rng, (Qt, hd), hi - 8, hi)
    return bf16_bits_to_f32(as_bf16_bits(q.astype(np.float32))).reshape(H, Qt, hd)


def open_bank(bank, offs, kv, hd):
    kw = dict(kv_heads=kv, head_dim=hd, node_ids=np.arange(offs.size - 1, dtype=np.uint64))
    if bank["code"] == oracle.I8:
        return GqaNodeBank(bank["keys"], offs, dtype="i8", scales=bank["scales"],
                           scale_dtype="f16", group_size=hd, **kw)
    if bank["code"] == oracle.F32:
        return GqaNodeBank(bank["keys"], offs, **kw)
    return GqaNodeBank(bank["keys"], offs, dtype="bf16" if bank["code"] == oracle.BF16 else "f16",
                       **kw)


@pytest.mark.parametrize("kind", ["bf16", "f16", "i8", "f32"])
def test_gqa_screen_obeys_its_bound(hip_lib, kind):
    rng = np.random.default_rng({"bf16": 5, "f16": 6, "i8": 7, "f32": 8}[kind])
    n, kv, hd, H, Qt = 360, 2, 128, 8, 3
    R = H // kv
    bank, offs = gqa_bank(rng, kind, n, kv, hd)
    q = gqa_query(rng, H, Qt, hd, kind)
    with open_bank(bank, offs, kv, hd) as b:
        maxima, colinfo, K, ids = b.probe_screen(q, query_dtype="bf16")
    np.testing.assert_array_equal(ids[:n], np.arange(n, dtype=np.uint64))
    law = bank["law"].astype(np.float64)
    checked = capped = 0
    worst = 0.0
    for i in range(n):
        L = int(offs[i + 1] - offs[i])
        keys = law[int(offs[i]) * kv * hd:int(offs[i + 1]) * kv * hd].reshape(kv, L, hd)
        for g in range(kv):
            cols = q[g * R:(g + 1) * R].reshape(R * Qt, hd).astype(np.float64)
            exact = np.abs(cols @ keys[g].T).max(axis=1)  # [R*Qt]
            coef, eabs, scale, kcap = (colinfo[g, :, j].astype(np.float64) for j in range(4))
            ok = K[i] < kcap
            capped += int((~ok).sum())
            e = coef * K[i] + eabs
            d = np.abs(maxima[i, g].astype(np.float64) - scale * exact)
            assert np.all(d[ok] <= e[ok]), (i, g, np.max(d[ok] / e[ok]))
            checked += int(ok.sum())
            if ok.any():
                worst = max(worst, float(np.max(d[ok] / e[ok])))
    assert checked > n * kv * R * Qt // 2
    if kind in ("bf16", "f32"):
        assert capped > 0  # the overflow cap (fp32: the fp16 copy's range) is exercised
    assert worst <= 1.0


@pytest.mark.parametrize("kind", ["bf16", "f16", "i8", "f32"])
@pytest.mark.parametrize("mode", ["sr", "bv", "exact"])
def test_gqa_stress_banks_route_like_the_law(hip_lib, monkeypatch, kind, mode):
    monkeypatch.setenv("GRM_HIP_GQA_SCREEN", "0" if mode == "exact" else "1")
    monkeypatch.setenv("GRM_HIP_GQA_BOUND", "1" if mode == "bv" else "0")
    rng = np.random.default_rng({"bf16": 5, "f16": 6, "i8": 7, "f32": 8}[kind])
    n, kv, hd, H, Qt = 360, 2, 128, 8, 3
    bank, offs = gqa_bank(rng, kind, n, kv, hd)
    qs = np.stack([gqa_query(rng, H, Qt, hd, kind) for _ in range(3)])
    with open_bank(bank, offs, kv, hd) as b:
        res = b.route(qs, 8)
    kw = {}
    if kind == "i8":
        kw = dict(scales=bank["scales"], scale_dtype="f16", group_size=hd)
    want, sc, _ = oracle.gqa_route(bank["keys"], bank["code"], offs, kv, hd, qs, 8, **kw)
    np.testing.assert_array_equal(res.ids, want)
    filled = want != NO_ID
    np.testing.assert_array_equal(res.scores[filled].view(np.uint32), sc[filled].view(np.uint32))


def fp32_query(rng, H, Qt, hd):
    """Queries in fp32 proper (not bf16-representable): Gaussian, wide,
    paired and tiny families, so both parts of a split query matter."""
    fam = np.arange(H) % 4
    q = np.empty((H, Qt, hd))
    for h in range(H):
        f = fam[h]
        if f == 0:
            q[h] = rng.standard_normal((Qt, hd))
        elif f == 1:
            q[h] = spread(rng, (Qt, hd), -12, 12)
        elif f == 2:
            q[h] = paired(rng, (Qt, hd)) * (1.0 + 2.0 ** -9 * rng.standard_normal((Qt, hd)))
        else:
            q[h] = spread(rng, (Qt, hd), -40, -20)
    return q.astype(np.float32)


@pytest.mark.parametrize("kind", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("Qt", [1, 2])
@pytest.mark.parametrize("split", ["1", "0"])
def test_gqa_fp32_query_split_routes_like_the_law(hip_lib, monkeypatch, kind, Qt, split):
    """One fp32 query over at most 8 columns per kv head takes the screen
    with each column's remainder in an idle column slot (split) or rounded
    once (GRM_HIP_GQA_SPLIT=0); both must route like the law."""
    monkeypatch.setenv("GRM_HIP_GQA_SCREEN", "1")
    monkeypatch.setenv("GRM_HIP_GQA_BOUND", "0")
    monkeypatch.setenv("GRM_HIP_GQA_SPLIT", split)
    rng = np.random.default_rng({"bf16": 15, "f16": 16, "f32": 18}[kind] + 3 * Qt)
    n, kv, hd, H = 360, 2, 128, 8
    bank, offs = gqa_bank(rng, kind, n, kv, hd)
    qs = [fp32_query(rng, H, Qt, hd)[None] for _ in range(3)]
    with open_bank(bank, offs, kv, hd) as b:
        got = [b.route(q, 8) for q in qs]
        stats = b.route_stats()
    assert stats["screen_refine"] >= 3
    for q, res in zip(qs, got):
        want, sc, _ = oracle.gqa_route(bank["keys"], bank["code"], offs, kv, hd, q, 8)
        np.testing.assert_array_equal(res.ids, want)
        filled = want != NO_ID
        np.testing.assert_array_equal(res.scores[filled].view(np.uint32),
                                      sc[filled].view(np.uint32))
