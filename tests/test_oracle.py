"""Pins the CPU oracle before it is trusted as the GPU checker.

Each test names the reference file it pins against. Checks are chosen so that a
plausible restatement mistake (wrong group boundary, /7 vs /3.5, a dropped
correction term, a transposed Z, a wrong sign convention, round-half-even
instead of half-away) fails at least one of them:
  * known answers held by the reference's own examples/tests
    (basic_usage.rs, slhav2-vram codec.rs / tests/cpu.rs, NF4 literals);
  * published SplitMix64 outputs;
  * closed forms in float64 (Hadamard matrix, dot products, rms);
  * brute-force searches (nearest quantisation level, per-bit Hamming);
  * the reference's invariants (tests.rs, properties.rs, tests/slha.rs).
"""
import numpy as np
import pytest

import oracle_ffi as o

GOLDEN = 0x9E3779B97F4A7C15


def ramp():
    return ((np.arange(128, dtype=np.float32) - 64.0) / 16.0).astype(np.float32)


def round_half_away(x):
    x = np.asarray(x, np.float64)
    return np.sign(x) * np.floor(np.abs(x) + 0.5)


# --- rng.rs ---------------------------------------------------------------

def test_splitmix64_published_vectors():
    # Rng::new(seed) starts from seed ^ GOLDEN, so seed = GOLDEN is the raw
    # SplitMix64 stream from state 0, whose first outputs are published.
    r = o.Rng(GOLDEN)
    assert [r.next_u64() for _ in range(3)] == [
        0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_next_unit_is_top_24_bits():
    a, b = o.Rng(1234), o.Rng(1234)
    for _ in range(1000):
        u = a.next_u64()
        assert b.next_unit() == np.float32((u >> 40) / float(1 << 24))


def test_gaussian_moments_and_determinism():
    g = o.Rng(5).gaussian(200000)
    assert abs(g.mean()) < 0.01 and abs(g.std() - 1.0) < 0.01
    assert np.array_equal(g[:100], o.Rng(5).gaussian(100))


def _box_muller_f64(u1, u2, variant="ref"):
    """rng.rs:39-44 in float64 from the pinned next_unit draws:
    sqrt(-2 ln max(u1, 1e-7)) * cos(2 pi u2). The variants plant the plausible
    slips (sin for cos, u1 and u2 swapped) to show the check rejects them."""
    a = np.maximum(u1.astype(np.float64), 1e-7)
    b = u2.astype(np.float64)
    if variant == "swap_u":
        a, b = np.maximum(b, 1e-7), a
    trig = np.sin if variant == "sin" else np.cos
    return np.sqrt(-2.0 * np.log(a)) * trig(2.0 * np.pi * b)


def _box_muller_close(got, want):
    # f32 evaluation error: ln, sqrt and the f32 product 2*pi*u2 (the angle is
    # off by at most ~6e-7 rad, so the cosine by ~6e-7 absolute) give
    # |got - want| <= r * 1.5e-6 + 4 ulp(|want|). r = sqrt(-2 ln u1) <= 5.7.
    r = np.sqrt(-2.0 * np.log(1e-7))
    tol = r * 1.5e-6 + 4 * np.spacing(np.abs(want).astype(np.float32)).astype(np.float64)
    return np.abs(got.astype(np.float64) - want) <= tol


def test_gaussian_is_box_muller_closed_form():
    # rng.rs:39-44: u1 = next_unit().max(1e-7), u2 = next_unit(),
    # r = sqrt(-2 ln u1), g = r cos(2 pi u2). The uniform draws are pinned by
    # test_next_unit_is_top_24_bits, so the two-draw pairing, the max, and the
    # trigonometric branch are pinned here against float64.
    for seed in (0, 5, 2**63 + 11):
        n = 50000
        g = o.Rng(seed).gaussian(n)
        r = o.Rng(seed)
        u = np.array([r.next_unit() for _ in range(2 * n)], np.float32)
        u1, u2 = u[0::2], u[1::2]
        assert _box_muller_close(g, _box_muller_f64(u1, u2)).all()
        # A planted sin/cos or u1/u2 swap fails on most draws.
        for bad in ("sin", "swap_u"):
            assert (~_box_muller_close(g, _box_muller_f64(u1, u2, bad))).mean() > 0.9
    # u1 = 0 must take the 1e-7 floor. A seed whose first draw is 0 comes from
    # inverting the SplitMix64 finaliser (rng.rs:22-28) on an output whose top
    # 24 bits are zero.
    m64 = 2**64 - 1

    def unshift(x, s):
        y = x
        for _ in range(64 // s + 1):
            y = x ^ (y >> s)
        return y & m64

    z = 0x0000001234567890
    z = unshift(z, 31)
    z = unshift((z * pow(0x94D049BB133111EB, -1, 2**64)) & m64, 27)
    z = unshift((z * pow(0xBF58476D1CE4E5B9, -1, 2**64)) & m64, 30)
    seed = ((z - GOLDEN) & m64) ^ GOLDEN
    r = o.Rng(seed)
    assert r.next_unit() == 0.0
    u2 = np.float32(r.next_unit())
    g = o.Rng(seed).gaussian(1)
    want = np.sqrt(-2.0 * np.log(1e-7)) * np.cos(2.0 * np.pi * np.float64(u2))
    assert abs(float(g[0]) - want) <= 1e-5 and abs(want) > 0.1


# --- KATs -----------------------------------------------------------------

def test_basic_usage_known_answer():
    # scirust/examples/basic_usage.rs:9-45 + README.md:98-102: score -8,
    # dequant[0..4] = [-4, -4, -4, -4].
    lat, scale, _ = o.quantize(0, ramp())
    t = o.make_tile(lat, scale, [255] * 8, lam=0.5)
    dq = o.dequant(t)
    assert np.array_equal(dq[:4], np.full(4, -4.0, np.float32))
    q = np.zeros(128, np.float32)
    q[:2] = 1.0
    s, h = o.score(t, q, [0x123456789ABCDEF0] * 4)
    assert h[0] == 128 and s[0] == np.float32(-8.0)


@pytest.mark.parametrize("nib,level", [(0x0, -8.0), (0x8, 0.0), (0xF, 7.0)])
def test_decode_int4_known_answer(nib, level):
    # slhav2-vram/src/codec.rs:325-329
    t = o.make_tile([nib | (nib << 4)] * 64, 1.0, [255] * 8)
    assert np.all(o.dequant(t) == np.float32(level))


def test_effective_scale_known_answer():
    # slhav2-vram/src/codec.rs:363-366: effective_scale(2.0, 128) ~ 1.0039216
    t = o.make_tile([0x98] * 64, 2.0, [128] * 8)  # low nibble 8 -> 0, high 9 -> 1
    dq = o.dequant(t)
    assert dq[0] == 0.0 and abs(dq[1] - 1.0039216) < 1e-6


@pytest.mark.parametrize("byte,expected", [(0x88, 0.0), (0x00, -1024.0), (0xFF, 896.0)])
def test_zero_point_tiles(byte, expected):
    # slhav2-vram/tests/cpu.rs:54-115 (q = 1, scale 1, gs 255, residual 0, lambda 0)
    t = o.make_tile([byte] * 64, 1.0, [255] * 8)
    s, _ = o.score(t, np.ones(128, np.float32), [0] * 4)
    assert s[0] == np.float32(expected)


def test_nf4_codebook_literals():
    # constants.rs:138-141 (also slha_score.cu:33-38, codec.rs:333-336)
    cb = [-1.0, -0.7075, -0.5421, -0.4165, -0.3108, -0.2158, -0.1272, -0.0421,
          0.0421, 0.1272, 0.2158, 0.3108, 0.4165, 0.5421, 0.7075, 1.0]
    lat = [i | (i << 4) for i in range(16)] * 4
    t = o.make_tile(lat, 1.0, [255] * 8, flags=o.lib and 2)
    dq = o.dequant(t)
    assert np.array_equal(dq[0:32:2], np.asarray(cb, np.float32))


# --- quantisers: bounds + brute-force nearest levels ----------------------

def gauss_inputs(seed, n=50):
    r = o.Rng(seed)
    out = []
    for _ in range(n):
        amp = r.next_unit() * 5.0 + 0.1
        out.append((r.gaussian(128) * np.float32(amp)).astype(np.float32))
    return out


def steep(seed):
    # tests.rs:133-141
    g = o.Rng(seed).gaussian(128)
    amp = (37.0 * np.power(np.arange(1, 129, dtype=np.float32), np.float32(-0.9))).astype(np.float32)
    return (amp * g).astype(np.float32)


def nibbles(lat):
    lat = np.asarray(lat, np.uint8)
    return np.stack([lat & 15, lat >> 4], 1).reshape(-1).astype(np.int64)


def expected_gs(steps):
    steps = np.asarray(steps, np.float32)
    glob = np.float32(steps.max()) if steps.max() > 0 else np.float32(1.0)
    r = round_half_away((steps / glob * np.float32(255.0)).astype(np.float32))
    return glob, np.clip(r, 1, 255).astype(np.uint8)


def test_int4_single_is_nearest_level():
    # int4.rs:9-24; tests.rs:46-70 (round trip within one step, negatives kept)
    for v in gauss_inputs(1) + [ramp()]:
        lat, scale, _ = o.quantize(0, v)
        assert np.float32(scale) == np.float32(np.abs(v).max() / np.float32(7.0))
        lev = nibbles(lat) - 8
        want = np.clip(round_half_away((v / np.float32(scale)).astype(np.float32)), -8, 7)
        assert np.array_equal(lev, want)
        dq = o.dequant(o.make_tile(lat, scale, [255] * 8))
        assert np.all(np.abs(dq - v) <= scale + 1e-6)


def test_int4_grouped_bytes_and_levels():
    # int4.rs:34-63; properties.rs:138-165 (error <= eff)
    for v in gauss_inputs(2):
        lat, glob, gs = o.quantize(1, v)
        steps = np.abs(v).reshape(8, 16).max(1).astype(np.float32) / np.float32(7.0)
        g2, gs2 = expected_gs(steps)
        assert glob == g2 and np.array_equal(gs, gs2)
        eff = (np.float32(glob) * (gs.astype(np.float32) / np.float32(255.0))).repeat(16)
        lev = nibbles(lat) - 8
        cand = np.arange(-8, 8)[None, :] * eff[:, None].astype(np.float64)
        err = np.abs(cand - v[:, None].astype(np.float64))
        best = err.min(1)
        assert np.all(np.abs(lev * eff.astype(np.float64) - v) <= best + 1e-6 * eff)
        dq = o.dequant(o.make_tile(lat, glob, gs))
        assert np.all(np.abs(dq - v) <= eff + 1e-5)


def test_nf4_bruteforce_argmin_and_bound():
    # nf4.rs:7-57 (strict '<' -> lowest index on ties); properties.rs:167-180
    cb = np.asarray([-1.0, -0.7075, -0.5421, -0.4165, -0.3108, -0.2158, -0.1272, -0.0421,
                     0.0421, 0.1272, 0.2158, 0.3108, 0.4165, 0.5421, 0.7075, 1.0], np.float32)
    for v in gauss_inputs(3):
        lat, glob, gs = o.quantize(2, v)
        steps = np.abs(v).reshape(8, 16).max(1).astype(np.float32)
        g2, gs2 = expected_gs(steps)
        assert glob == g2 and np.array_equal(gs, gs2)
        eff = (np.float32(glob) * (gs.astype(np.float32) / np.float32(255.0))).repeat(16)
        t = np.clip((v / eff).astype(np.float32), -1, 1)
        want = np.argmin(np.abs(t[:, None] - cb[None, :]), axis=1)  # first minimum = lowest index
        assert np.array_equal(nibbles(lat), want)
        dq = o.dequant(o.make_tile(lat, glob, gs, flags=2))
        assert np.all(np.abs(dq - v) <= 0.16 * eff + 1e-5)
    # exact midpoint tie between levels 7 and 8 (+-0.0421) -> lower index 7
    assert o.lib.orc_nf4_nearest(0.0) == 7


def tq3_expect(v, eff):
    t = (v / eff).astype(np.float32)
    code = np.clip(round_half_away((t + np.float32(3.5)).astype(np.float32)), 0, 7).astype(np.int64)
    corr = (t - (code.astype(np.float32) - np.float32(3.5))) > 0
    return code, corr


def unpack3(lat, bit0, n):
    bits = np.unpackbits(np.asarray(lat, np.uint8), bitorder="little")
    return np.array([bits[bit0 + 3 * i] | (bits[bit0 + 3 * i + 1] << 1) | (bits[bit0 + 3 * i + 2] << 2)
                     for i in range(n)], np.int64)


def unpack1(lat, bit0, n):
    return np.unpackbits(np.asarray(lat, np.uint8), bitorder="little")[bit0:bit0 + n].astype(bool)


def test_tq3_codes_corr_and_bounds():
    # tq3.rs:10-49; tests.rs:223-347
    for v in gauss_inputs(4) + [steep(19)]:
        lat, glob, gs = o.quantize(4, v)
        steps = np.abs(v).reshape(8, 16).max(1).astype(np.float32) / np.float32(3.5)
        g2, gs2 = expected_gs(steps)
        assert glob == g2 and np.array_equal(gs, gs2)
        eff = (np.float32(glob) * (gs.astype(np.float32) / np.float32(255.0))).repeat(16)
        code, corr = tq3_expect(v, eff)
        assert np.array_equal(unpack3(lat, 0, 128), code)
        assert np.array_equal(unpack1(lat, 384, 128), corr)
        dq = o.dequant(o.make_tile(lat, glob, gs, flags=8))
        assert np.all(np.abs(dq - v) <= eff + 1e-5)
    # equal-spread groups: quarter-step bound (tests.rs:223-247)
    pat = o.Rng(17).gaussian(16)
    v = np.tile(pat, 8)
    lat, glob, gs = o.quantize(4, v)
    assert np.all(gs == 255)
    dq = o.dequant(o.make_tile(lat, glob, gs, flags=8))
    assert np.all(np.abs(dq - v) <= 0.25 * glob + 1e-5)
    # NOCORR with the plane zeroed: half-step bound (tests.rs:321-347)
    v = steep(29)
    lat, glob, gs = o.quantize(4, v)
    t = o.make_tile(lat, glob, gs, flags=8)
    t_nc, reclaimed = o.drop_correction(t)
    assert reclaimed == 1 and np.all(t_nc["latent_kv"][0][48:] == 0)
    eff = (np.float32(glob) * (gs.astype(np.float32) / np.float32(255.0))).repeat(16)
    dq_nc = o.dequant(t_nc)
    assert np.all(np.abs(dq_nc - v) <= 0.5 * eff + 1e-5)
    assert ((o.dequant(t) - v) ** 2).sum() < ((dq_nc - v) ** 2).sum()


def test_mixed_layout_and_bounds():
    # mixed.rs:13-57; tests.rs:142-171
    for seed in range(11, 19):
        v = steep(seed)
        lat, glob, gs = o.quantize(3, v)
        steps = np.concatenate([[np.abs(v[:8]).max() / np.float32(127.0)],
                                np.abs(v[8:120]).reshape(7, 16).max(1) / np.float32(7.0)]).astype(np.float32)
        g2, gs2 = expected_gs(steps)
        assert glob == g2 and np.array_equal(gs, gs2)
        eff_hi = np.float32(glob) * (np.float32(gs[0]) / np.float32(255.0))
        head = lat[:8].astype(np.int64) - 128
        want = np.clip(round_half_away((v[:8] / eff_hi).astype(np.float32)), -128, 127)
        assert np.array_equal(head, want)
        dq = o.dequant(o.make_tile(lat, glob, gs, flags=4))
        assert np.all(dq[120:] == 0.0)
        # gs[0] is a rounded byte, so the head step can sit just below
        # max|v|/127 and the extreme dim clamps at +-127: the one-step bound
        # of tests.rs:149-157 holds on the dims that do not clamp.
        inside = np.abs(v[:8] / eff_hi) <= 127.0
        assert np.all(np.abs(dq[:8] - v[:8])[inside] <= eff_hi + 1e-6)
        assert np.all(np.abs(head[~inside]) >= 127)
        eff = (np.float32(glob) * (gs[1:].astype(np.float32) / np.float32(255.0))).repeat(16)
        inside = np.abs(v[8:120] / eff) <= 7.0
        assert np.all(np.abs(dq[8:120] - v[8:120])[inside] <= eff[inside] + 1e-6)


def test_mix3_layout_and_bounds():
    # mix3.rs:11-62; tests.rs:404-500
    for seed in range(41, 49):
        v = steep(seed)
        lat, glob, gs = o.quantize(5, v)
        eff = (np.float32(glob) * (gs[1:].astype(np.float32) / np.float32(255.0))).repeat(16)
        code, corr = tq3_expect(v[8:120], eff)
        assert np.array_equal(unpack3(lat, 64, 112), code)
        assert np.array_equal(unpack1(lat, 400, 112), corr)
        dq = o.dequant(o.make_tile(lat, glob, gs, flags=32))
        assert np.all(dq[120:] == 0.0)
        inside = np.abs(v[8:120] / eff) <= 3.5
        assert np.all(np.abs(dq[8:120] - v[8:120])[inside] <= eff[inside] + 1e-6)
        t_nc, r = o.drop_correction(o.make_tile(lat, glob, gs, flags=32))
        assert r == 1 and np.all(t_nc["latent_kv"][0][50:] == 0)
        assert np.array_equal(o.dequant(t_nc)[:8], dq[:8])  # head untouched


# --- Hamming / eq. 2.3 ----------------------------------------------------

def test_hamming_bruteforce():
    # tests.rs:977-997, tests/slha.rs:17-46
    r = o.Rng(0x4D31)
    for _ in range(500):
        a = np.array([r.next_u64() for _ in range(4)], np.uint64)
        b = np.array([r.next_u64() for _ in range(4)], np.uint64)
        bits = np.unpackbits((a ^ b).view(np.uint8))
        t = o.make_tile([0x88] * 64, 1.0, [255] * 8, lam=1.0, residual=b)
        _, h = o.score(t, np.zeros(128, np.float32), a)
        assert h[0] == bits.sum()
        sa = 1 - 2 * np.unpackbits(a.view(np.uint8), bitorder="little").astype(np.int64)
        sb = 1 - 2 * np.unpackbits(b.view(np.uint8), bitorder="little").astype(np.int64)
        assert 256 - 2 * int(h[0]) == int((sa * sb).sum())


def rand_tile(r, codec_flags=0, warm=False):
    lat = np.array([r.next_u64() & 0xFF for _ in range(64)], np.uint8)
    gs = np.array([(r.next_u64() & 0xFF) | 1 for _ in range(8)], np.uint8)
    res = np.array([r.next_u64() for _ in range(4)], np.uint64)
    flags = codec_flags | (1 if warm else 0)
    return o.make_tile(lat, r.next_unit() * 2.0 + 0.01, gs, flags=flags,
                       lam=abs(float(r.gaussian(1)[0])) * 0.1, sigma=r.next_unit(), residual=res)


@pytest.mark.parametrize("flags", [0, 2, 4, 8, 8 | 16, 32, 32 | 16])
def test_score_matches_equation_2_3(flags):
    # tests/slha.rs:51-67 (hand formula), properties.rs:101-115 (WARM), :224-237 (bound)
    r = o.Rng(100 + flags)
    for it in range(100):
        t = rand_tile(r, flags)
        q = r.gaussian(128)
        qs = np.array([r.next_u64() for _ in range(4)], np.uint64)
        s, h = o.score(t, q, qs)
        k = o.dequant(t).astype(np.float64)
        lam = float(t["dynamic_lambda"][0])
        manual = float((q.astype(np.float64) * k).sum()) + lam * (256 - 2 * int(h[0]))
        assert abs(s[0] - manual) <= 1e-4 * (1 + abs(manual))
        w = t.copy()
        w["flags"] |= 1
        sw, _ = o.score(w, q, qs)
        assert abs(sw[0] - float((q.astype(np.float64) * k).sum())) <= 1e-4 * (1 + abs(sw[0]))
        assert abs(s[0] - sw[0]) <= lam * 256 + 1e-3


# --- sign-LSH, RHT, rms, lambda -------------------------------------------

def test_sign_bits_against_float64_and_negation():
    # scenario.rs:66-83; properties.rs:203-221
    z = o.projection(2)
    r = o.Rng(3)
    zn = np.linalg.norm(z.astype(np.float64), axis=1)
    for _ in range(50):
        v = r.gaussian(128)
        bits = np.unpackbits(o.sign_bits(z, v).view(np.uint8), bitorder="little")
        dot = z.astype(np.float64) @ v.astype(np.float64)
        clear = np.abs(dot) > 1e-4 * zn * np.linalg.norm(v)
        assert np.array_equal(bits[clear], (dot[clear] < 0).astype(np.uint8))
        nb = np.unpackbits(o.sign_bits(z, -v).view(np.uint8), bitorder="little")
        assert np.all(bits ^ nb)


def test_projection_is_row_major_gaussian_stream():
    # scenario.rs:59-64: Z = fill_gaussian over D_S*D_K in row-major order
    z = o.projection(9)
    assert np.array_equal(z.reshape(-1)[:300], o.Rng(9).gaussian(300))


def hadamard(n):
    i = np.arange(n)
    pc = np.vectorize(lambda x: bin(x).count("1"))(i[:, None] & i[None, :])
    return np.where(pc % 2 == 0, 1.0, -1.0) / np.sqrt(n)


def test_rht_closed_form_and_orthogonality():
    # incoherence.rs:45-126, :135-208
    diag = o.rht_diag(0x1234 ^ 0xA2A2A2A2A2A2A2A2)
    rr = o.Rng(0x1234 ^ 0xA2A2A2A2A2A2A2A2)
    assert np.array_equal(diag, np.array([-1.0 if rr.next_unit() < 0.5 else 1.0
                                          for _ in range(128)], np.float32))
    H = hadamard(128)
    r = o.Rng(11)
    for _ in range(20):
        v = r.gaussian(128)
        got = o.rht(diag, v).astype(np.float64)
        want = H @ (diag.astype(np.float64) * v)
        assert np.max(np.abs(got - want)) < 1e-5
        assert abs(np.linalg.norm(got) - np.linalg.norm(v)) <= 1e-4 * np.linalg.norm(v)
        twice = o.fwht(o.fwht(v))
        assert np.all(np.abs(twice - v) <= 1e-4 * (1 + np.abs(v)))
    assert o.lib.orc_next_pow2(160) == 256 and o.lib.orc_next_pow2(128) == 128


def test_rms_and_lambda_constant():
    # metrics.rs:207-226; scenario.rs:30-32
    r = o.Rng(21)
    for _ in range(50):
        v = (r.gaussian(128) * np.float32(r.next_unit() * 3)).astype(np.float32)
        want = np.float32(np.sqrt(np.mean(v.astype(np.float64) ** 2)))
        assert o.rms(v) == want
    assert np.isnan(o.rms(np.array([1.0, np.inf], np.float32)))
    assert o.lib.orc_analytic_lambda_c() == np.float32(np.sqrt(np.float32(np.pi) / np.float32(512)))
    assert abs(o.lib.orc_analytic_lambda_c() - 0.0783) < 1e-4


# --- encode composition (mode R / Z) ---------------------------------------

@pytest.mark.parametrize("codec", range(6))
@pytest.mark.parametrize("use_rht", [False, True])
def test_encode_mode_r_composition(codec, use_rht):
    z = o.projection(77)
    diag = o.rht_diag(77 ^ 0xA2A2A2A2A2A2A2A2) if use_rht else None
    keys = o.Rng(5 + codec).gaussian(16 * 128).reshape(16, 128)
    tiles = o.encode(keys, codec, 1, z, diag, pos0=10, head=3)
    flags = [0, 0, 2, 4, 8, 32][codec]
    for i, t in enumerate(tiles):
        lat, sc, gs = o.quantize(codec, keys[i])
        assert np.array_equal(t["latent_kv"], lat) and t["scale"] == np.float32(sc)
        assert np.array_equal(t["group_scales"], gs)
        assert t["flags"] == flags and t["position"] == 10 + i and t["token_id"] == 10 + i
        assert t["head_id"] == 3
        e = (keys[i] - o.dequant(t)).astype(np.float32)
        assert t["residual_sigma"] == np.float32(o.rms(e))
        assert t["dynamic_lambda"] == np.float32(np.float32(o.rms(e)) * o.lib.orc_analytic_lambda_c())
        src = o.rht(diag, e) if use_rht else e
        assert np.array_equal(t["residual_bitmap"], o.sign_bits(z, src))
        assert o.validate(t) == 0
    zt = o.encode(keys, codec, 0, z, diag)
    assert np.all(zt["residual_bitmap"] == 0) and np.all(zt["dynamic_lambda"] == 0)
    assert np.array_equal(zt["latent_kv"], tiles["latent_kv"])


def test_mode_r_score_estimates_true_dot():
    # Mode R's lambda*(256-2h) estimates <q, e>, so the score tracks <q, k>.
    z = o.projection(3)
    r = o.Rng(8)
    keys = r.gaussian(2000 * 128).reshape(2000, 128)
    q = r.gaussian(128)
    tiles = o.encode(keys, 1, 1, z)
    s, _ = o.score(tiles, q, o.query_sign(q, z))
    coarse, _ = o.score(o.encode(keys, 1, 0, z), q, [0] * 4)
    true = keys.astype(np.float64) @ q
    assert np.mean((s - true) ** 2) < np.mean((coarse - true) ** 2)


# --- validation / CCOS / top-k ---------------------------------------------

def test_validate_tile_contract():
    # slha-c/src/lib.rs:244-286
    ok = o.make_tile([0x88] * 64, 1.0, [255] * 8)
    assert o.validate(ok) == 0
    for flags, code in [(0x40, -6), (2 | 4, -6), (16, -6), (16 | 8, 0), (16 | 32, 0), (1, 0)]:
        assert o.validate(o.make_tile([0] * 64, 1.0, [255] * 8, flags=flags)) == code
    assert o.validate(o.make_tile([0] * 64, np.nan, [255] * 8)) == -5
    assert o.validate(o.make_tile([0] * 64, 1.0, [255] * 8, lam=np.inf)) == -5
    assert o.validate(o.make_tile([0] * 64, -1.0, [255] * 8)) == -6
    assert o.validate(o.make_tile([0] * 64, 1.0, [255] * 8, sigma=-0.5)) == -6


def test_page_out_effects():
    # ccos.rs:369-378
    r = o.Rng(4)
    t = rand_tile(r)
    w = o.page_out(t)
    assert np.all(w["residual_bitmap"] == 0) and w["dynamic_lambda"] == 0 and w["flags"] & 1
    assert np.array_equal(w["latent_kv"], t["latent_kv"])
    q = r.gaussian(128)
    s_hot0 = t.copy()
    s_hot0["dynamic_lambda"] = 0
    assert o.score(w, q, [7] * 4)[0][0] == o.score(s_hot0, q, [7] * 4)[0][0]
    assert o.drop_correction(t)[1] == 0  # INT4: no separable plane


def test_topk_order_and_ties():
    s = np.array([1.0, 3.0, 3.0, -2.0, 3.0, 0.5, 1.0], np.float32)
    idx, val = o.topk(s, 5)
    assert list(idx) == [1, 2, 4, 0, 6]
    assert list(val) == [3.0, 3.0, 3.0, 1.0, 1.0]
    idx, _ = o.topk(s, 9)
    assert list(idx[7:]) == [0xFFFFFFFF, 0xFFFFFFFF]
    r = np.random.default_rng(0)
    x = r.integers(-5, 5, 1000).astype(np.float32)
    idx, _ = o.topk(x, 64)
    want = np.lexsort((np.arange(1000), -x))[:64]
    assert np.array_equal(idx, want)
