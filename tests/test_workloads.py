"""The synthetic INT8 bank generator (CPU only: a host function of the
library, no device call).

Its keys are restated here in numpy (a splitmix64 counter stream indexing
the normal-quantile table) and quantised by the oracle's packed-format
quantiser with fp16 row scales (oracle.quantize_int8, core/graft_quant.py:
93-131); the library's codes and scale bits must equal that, at an offset
row and on any thread count.  The table itself is checked against the
normal law (symmetry, moments, and the quantiles' defining CDF values).
"""

import math

import numpy as np

import oracle
from graftrepository_amd import _lib, workloads as wl

M64 = (1 << 64) - 1


def splitmix_words(key: int, start: int, count: int) -> np.ndarray:
    idx = np.arange(start, start + count, dtype=np.uint64)
    z = idx * np.uint64(0x9E3779B97F4A7C15) + np.uint64(key)
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def test_splitmix_restatement_known_values():
    # splitmix64's published first outputs for state 0: the finaliser of
    # 0x9E3779B97F4A7C15 * (i + 1)
    w = splitmix_words(0x9E3779B97F4A7C15, 0, 3)
    assert [int(x) for x in w] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4,
                                   0x06C45D188009454F]


def test_normal_table_is_the_normal_quantiles():
    t = wl._normal_table().astype(np.float64)
    assert t.size == 65536 and np.all(np.diff(t) > 0)
    np.testing.assert_array_equal(t, -t[::-1])            # symmetric
    assert abs(t.mean()) < 1e-12 and abs(t.std() - 1.0) < 2e-4
    for u in (0, 1, 1000, 32767, 40000, 65535):
        p = 0.5 * (1.0 + math.erf(t[u] / math.sqrt(2.0)))
        assert abs(p - (u + 0.5) / 65536) < 1e-6 * max(1.0, 65536 * p * 1e-3)


def test_synth_rows_match_numpy_restatement_and_oracle_quantiser():
    lib = _lib.load()
    hd, row0, rows, seed = 128, 123_457, 3000, 9
    key = wl.int8_stream_key(seed)
    table = wl._normal_table()
    codes = np.empty(rows * hd, dtype=np.int8)
    scales = np.empty(rows, dtype=np.uint16)
    _lib.check(lib.grm_hip_synth_int8_rows(key, row0, rows, hd, table.ctypes.data, 5,
                                           codes.ctypes.data, scales.ctypes.data), "synth")
    words = splitmix_words(key, row0 * hd // 4, rows * hd // 4)
    x = table[words.view(np.uint16)].reshape(rows, hd)
    want_c, want_s = oracle.quantize_int8(x, hd, "f16")
    np.testing.assert_array_equal(codes.reshape(rows, hd), want_c)
    np.testing.assert_array_equal(scales, want_s.reshape(-1))
    c2, s2 = wl.quantize_rows_i8(x)
    np.testing.assert_array_equal(c2, want_c)
    np.testing.assert_array_equal(s2, want_s.reshape(-1))
    # every row reaches the grid's edge; codes look like a quantised normal
    assert np.all(np.abs(want_c.astype(np.int32)).max(axis=1) >= 127)
    assert 40 < codes.astype(np.float64).std() < 50


def test_bank_independent_of_worker_count():
    lens = wl.gqa_lengths(40, 3, kind="lognormal")
    a = wl.gqa_int8_bank(lens, 8, 64, seed=4, workers=1)
    b = wl.gqa_int8_bank(lens, 8, 64, seed=4, workers=7)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)
    assert a[0].size == int(lens.sum()) * 8 * 64 and a[1].size == int(lens.sum()) * 8
    c = wl.gqa_int8_bank(lens, 8, 64, seed=5, workers=3)
    assert not np.array_equal(a[0], c[0])
