"""Exact replacements in the encode kernels' codec arithmetic, checked on the CPU.

The quantisers in slhav2_amd/csrc/slha_kernels.hip replace three per-dim
steps of the reference's scalar code with cheaper ones that must give the
same bits:
- `x / eff` (int4.rs:52-60, nf4.rs:44-54, tq3.rs:31-46, mixed.rs:38-55) by
  Markstein's correction from y = RN(1 / eff), for 2^-71 <= eff <= 2^96;
- `x.round() as i32` by `v_cvt_i32_f32(x + copysign(0.5 - 2^-25, x))`;
- NF4's 16-level nearest scan (nf4.rs:7-18) by a count of 15 f32 thresholds,
  read here from the kernel source and checked against the oracle's scan.
The GPU parity tests check the kernels' tiles; these tests check the
identities themselves on sampled and boundary inputs (exhaustive runs over
all inputs take minutes and are not part of the suite).
"""
import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

import oracle_ffi as o

KERNELS = Path(__file__).resolve().parents[1] / "slhav2_amd" / "csrc" / "slha_kernels.hip"

C_SRC = r"""
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <limits.h>
static uint64_t st;
static uint64_t rnd(void) { st ^= st << 13; st ^= st >> 7; st ^= st << 17; return st; }
static float fu(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t uf(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static int32_t rs_i32(float f) {
    if (isnan(f)) return 0;
    if (f >= 2147483648.0f) return INT_MAX;
    if (f <= -2147483648.0f) return INT_MIN;
    return (int32_t)f;
}
/* kernel form: q0 = x y, r = fma(-q0, b, x), q = fma(r, y, q0) */
static float quot_fast(float x, float b, float y) {
    volatile float q0 = x * y;
    float r = fmaf(-q0, b, x);
    return fmaf(r, y, q0);
}
long check_round(long n, uint64_t seed) {
    st = seed; long bad = 0;
    const float c = 0x1.fffffep-2f;
    for (long i = 0; i < n; ++i) {
        float x;
        if (i & 1) x = fu((uint32_t)rnd());
        else {  /* k + 1/2 and its neighbours */
            int32_t k = (int32_t)(rnd() % 4194304) - 2097152;
            x = fu(uf((float)k + 0.5f) + (int32_t)(rnd() % 5) - 2);
        }
        volatile float s = x + copysignf(c, x);
        if (rs_i32(s) != rs_i32(roundf(x))) ++bad;
    }
    return bad;
}
/* quotients from 2^qlo to 2^qhi, divisors from 2^-71 to 2^96 */
long check_quot(long n, uint64_t seed, int qlo, int qhi) {
    st = seed; long bad = 0;
    for (long i = 0; i < n; ++i) {
        float b;
        switch (i & 3) {
            case 0: b = ldexpf(1.0f + (float)(rnd() % 8388608) / 8388608.0f, (int)(rnd() % 168) - 71); break;
            case 1: b = ldexpf(1.99999988f, (int)(rnd() % 167) - 71); break;
            case 2: { float g = ldexpf(1.0f + (float)(rnd() % 8388608) / 8388608.0f, (int)(rnd() % 8) - 4);
                      b = g * ((float)(1 + rnd() % 255) / 255.0f); break; }
            default: b = ldexpf(1.0f + (float)((rnd() % 256) << 15) / 8388608.0f, (int)(rnd() % 168) - 71);
        }
        if (!(b >= 0x1p-71f && b <= 0x1p96f)) continue;
        const float y = 1.0f / b;
        float x;
        if ((i & 7) == 3) {  /* x near (k + 1/2) b: the rounding ties */
            int32_t k = (int32_t)(rnd() % 64) - 32;
            x = fu(uf(((float)k + 0.5f) * b) + (int32_t)(rnd() % 7) - 3);
        } else {
            int e = qlo + (int)(rnd() % (uint64_t)(qhi - qlo + 1));
            x = ldexpf(1.0f + (float)(rnd() % 8388608) / 8388608.0f, e) * b;
            if (rnd() & 1) x = -x;
        }
        if (!isfinite(x)) continue;
        const float ref = x / b, got = quot_fast(x, b, y);
        if (uf(ref) != uf(got) && !(ref == 0.0f && got == 0.0f)) ++bad;
    }
    return bad;
}
"""


@pytest.fixture(scope="module")
def arith(tmp_path_factory):
    d = tmp_path_factory.mktemp("codec_arith")
    src, so = d / "arith.c", d / "libarith.so"
    src.write_text(C_SRC)
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fPIC", "-shared", str(src), "-o", str(so), "-lm"],
                   check=True)
    lib = ctypes.CDLL(str(so))
    lib.check_round.restype = ctypes.c_long
    lib.check_round.argtypes = [ctypes.c_long, ctypes.c_uint64]
    lib.check_quot.restype = ctypes.c_long
    lib.check_quot.argtypes = [ctypes.c_long, ctypes.c_uint64, ctypes.c_int, ctypes.c_int]
    return lib


def test_round_half_away_by_biased_add(arith):
    assert arith.check_round(4_000_000, 12345) == 0


@pytest.mark.parametrize("qlo,qhi", [(-32, -6), (-6, 13)])
def test_markstein_quotient_is_correctly_rounded(arith, qlo, qhi):
    assert arith.check_quot(3_000_000, 777 + qlo, qlo, qhi) == 0


def test_markstein_quotient_planted_mistakes_fail(arith):
    """The check above sees a dropped correction: q0 = RN(x y) alone is often an ulp off."""
    rng = np.random.default_rng(5)
    b = np.float32(rng.uniform(0.1, 3.0, 20000))
    x = np.float32(rng.uniform(-8, 8, 20000)) * b
    y = np.float32(1.0) / b
    assert np.count_nonzero(np.float32(x * y) != np.float32(x / b)) > 100


def _kernel_thresholds() -> np.ndarray:
    text = KERNELS.read_text()
    m = re.search(r"constexpr float kT\[15\] = \{([^}]*)\}", text)
    assert m, "NF4 threshold table not found in slha_kernels.hip"
    vals = [float.fromhex(t.strip().rstrip("f")) for t in m.group(1).split(",")]
    assert len(vals) == 15
    return np.array(vals, dtype=np.float32)


def _count(t: np.ndarray, thr: np.ndarray) -> np.ndarray:
    return (t[:, None] >= thr[None, :]).sum(axis=1)


def test_nf4_threshold_count_equals_the_oracle_scan():
    thr = _kernel_thresholds()
    assert np.all(np.diff(thr) > 0)
    bits = thr.view(np.uint32).astype(np.int64)
    near = []
    for b in bits:  # every f32 within 300 ulps of each threshold, both sides
        near.append(np.arange(b - 300, b + 301))
    cand = np.concatenate(near)
    vals = np.concatenate([
        cand.astype(np.uint32).view(np.float32),
        np.random.default_rng(3).uniform(-1, 1, 60000).astype(np.float32),
        np.array([-1.0, 1.0, 0.0, -0.0, 1e-30, -1e-30, 2.0**-29, -2.0**-29, np.nan], np.float32),
    ])
    vals = vals[np.isnan(vals) | ((vals >= -1) & (vals <= 1))]
    got = _count(vals, thr)
    ref = np.array([o.lib.orc_nf4_nearest(ctypes.c_float(float(v))) for v in vals])
    assert np.array_equal(got, ref)


def test_nf4_planted_threshold_error_fails():
    """Moving one threshold by a single ulp changes the index of some input."""
    thr = _kernel_thresholds()
    bad = thr.copy()
    bad[7] = np.nextafter(bad[7], np.float32(1))
    t = np.array([thr[7]], np.float32)
    ref = o.lib.orc_nf4_nearest(ctypes.c_float(float(t[0])))
    assert _count(t, thr)[0] == ref and _count(t, bad)[0] != ref


def test_round_planted_bias_of_one_half_fails():
    """With a bias of exactly 1/2 the largest float below 1/2 would round up."""
    x = np.nextafter(np.float32(0.5), np.float32(0))
    assert np.trunc(np.float32(x + np.float32(0.5))) == 1.0
    assert np.trunc(np.float32(x + np.float32(float.fromhex("0x1.fffffep-2")))) == 0.0
