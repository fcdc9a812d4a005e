"""The reported CPU baseline (oracle/cpu_baseline.c) against the oracle.

cpu_baseline.c restates the reference's SIMD dispatch (simd.rs:23-84): AVX2
and AVX-512 kernels for every codec and the VPOPCNTDQ Hamming. The bar for
those kernels is the reference's own SIMD-vs-scalar tolerance,
|simd - scalar| <= 1e-3 * (1 + |scalar|) (simd.rs tests, tests.rs:923), here
against the oracle's scalar restatement of tile.rs:267-281 on the same tiles.
bench.py times this library, so a fast but wrong baseline fails here.
"""
import ctypes

import numpy as np
import pytest

import oracle_ffi as o

TOL = 1e-3
lib = ctypes.CDLL(str(o.BASELINE_SO))
lib.cpu_score_tiles_isa.restype = ctypes.c_int
lib.cpu_score_tiles_isa.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                    ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
lib.cpu_score_rows.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_void_p,
                               ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int]
lib.cpu_baseline_isa.restype = ctypes.c_int
lib.cpu_baseline_vpopcntdq.restype = ctypes.c_int
ISA = lib.cpu_baseline_isa()
ISAS = [i for i in (0, 1, 2) if i <= ISA]


def _p(a):
    return a.ctypes.data


def baseline(tiles, q, qs, isa):
    t = np.ascontiguousarray(tiles, o.TILE_DTYPE)
    out = np.empty(len(t), np.float32)
    rc = lib.cpu_score_tiles_isa(_p(t), len(t), _p(o.f32(q)), _p(np.ascontiguousarray(qs, np.uint64)),
                                 _p(out), isa)
    assert rc == 0
    return out


def assert_tol(got, ref):
    bad = np.abs(got.astype(np.float64) - ref) > TOL * (1 + np.abs(ref.astype(np.float64)))
    assert not bad.any(), (np.argwhere(bad)[:5], got[bad][:5], ref[bad][:5])


def encoded(codec, n, seed, kind="gauss"):
    r = o.Rng(seed)
    k = r.gaussian(n * 128).reshape(n, 128).astype(np.float32)
    if kind == "student":  # C3 keys: Student-t(4) with four x20 outlier channels
        zz = r.gaussian(n * 4 * 128).reshape(n, 128, 4)
        k = (k / np.sqrt((zz ** 2).mean(-1))).astype(np.float32)
        k[:, [3, 17, 64, 100]] *= np.float32(20.0)
    z = o.projection(seed + 1)
    return o.encode(k, codec, 1, z)


def test_dispatch_levels_reported():
    assert ISA in (0, 1, 2)
    assert lib.cpu_baseline_vpopcntdq() in (0, 1)
    # the ISA levels above the host's are refused, not emulated
    t = encoded(0, 4, 1)
    out = np.empty(4, np.float32)
    q = np.zeros(128, np.float32)
    qs = np.zeros(4, np.uint64)
    assert lib.cpu_score_tiles_isa(_p(t), 4, _p(q), _p(qs), _p(out), 3) == -1


@pytest.mark.parametrize("isa", ISAS)
@pytest.mark.parametrize("codec", range(6))
@pytest.mark.parametrize("kind", ["gauss", "student"])
def test_every_codec_within_the_reference_tolerance(isa, codec, kind):
    # HOT, WARM (page_out) and, for TQ3/MIX3, NOCORR (drop_correction) tiles
    tiles = encoded(codec, 300, 10 + codec, kind)
    variants = [tiles, np.array([o.page_out(t) for t in tiles], o.TILE_DTYPE)]
    if codec in (4, 5):
        variants.append(np.array([o.drop_correction(t)[0] for t in tiles], o.TILE_DTYPE))
    r = np.random.default_rng(codec)
    for v in variants:
        for _ in range(3):
            q = r.normal(size=128).astype(np.float32)
            qs = r.integers(0, 2**63, 4, dtype=np.uint64) * 2 + r.integers(0, 2, 4, dtype=np.uint64)
            ref, _ = o.score(v, q, qs)
            assert_tol(baseline(v, q, qs, isa), ref)


def test_scalar_level_is_the_oracle():
    # level 0 is the scalar path itself: bit-identical to the oracle
    tiles = encoded(1, 200, 3)
    q = np.random.default_rng(0).normal(size=128).astype(np.float32)
    qs = np.arange(4, dtype=np.uint64) * 0x0123456789ABCDEF
    ref, _ = o.score(tiles, q, qs)
    assert np.array_equal(baseline(tiles, q, qs, 0).view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("isa", ISAS)
def test_hamming_term_exact(isa):
    # lambda = 1 and a zero latent: the score is exactly 256 - 2 * Hamming,
    # whichever popcount the host uses
    t = encoded(0, 64, 5)
    t["latent_kv"] = 0x88  # every nibble 8: level 0
    t["dynamic_lambda"] = 1.0
    t["flags"] = 0
    r = np.random.default_rng(7)
    t["residual_bitmap"] = r.integers(0, 2**63, (64, 4), dtype=np.uint64)
    qs = r.integers(0, 2**63, 4, dtype=np.uint64)
    got = baseline(t, np.zeros(128, np.float32), qs, isa)
    ham = np.array([sum(bin(int(a) ^ int(b)).count("1") for a, b in zip(row, qs))
                    for row in t["residual_bitmap"]])
    assert np.array_equal(got, (256 - 2 * ham).astype(np.float32))


def test_threaded_rows_equal_per_tile_scores():
    # cpu_score_rows (what bench.py times) scores the GQA layout of
    # slha_gpu_score: scores[r * group + j][t] against tiles[r][t]; any thread
    # count gives the per-tile results bit for bit
    n_rows, n_tok, group = 3, 257, 4
    tiles = encoded(2, n_rows * n_tok, 9).reshape(n_rows, n_tok)
    r = np.random.default_rng(1)
    q = r.normal(size=(n_rows * group, 128)).astype(np.float32)
    qs = r.integers(0, 2**63, (n_rows * group, 4), dtype=np.uint64)
    want = np.stack([baseline(tiles[i // group], q[i], qs[i], ISA) for i in range(n_rows * group)])
    for threads in (1, 3, 8):
        out = np.empty((n_rows * group, n_tok), np.float32)
        lib.cpu_score_rows(_p(np.ascontiguousarray(tiles)), n_rows, n_tok, _p(q), _p(qs), group,
                           _p(out), threads)
        assert np.array_equal(out.view(np.uint32), want.view(np.uint32)), threads
