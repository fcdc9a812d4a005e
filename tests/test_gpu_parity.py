"""GPU parity: every HIP entry point against the CPU oracle on identical inputs.

Bars (from the reference's own tests and BASELINE.json):
  * tile bytes (codes, residual bits, sigma, lambda, metadata): bit-exact;
  * Hamming distances: bit-exact;
  * SCORE_EXACT scores: bit-identical to tile.rs's scalar path;
  * SCORE_FAST scores: |gpu - ref| <= 1e-3 * (1 + |ref|)
    (scirust/src/attention/slha_v2/tests.rs:923, scirust/tests/properties.rs:73);
  * top-k indices: exact, ties to the lower token index.
"""
import json

import numpy as np
import pytest

import oracle_ffi as o

pytestmark = pytest.mark.gpu

TOL = 1e-3
FLAG_SETS = [0, 1, 2, 3, 4, 5, 8, 9, 8 | 16, 8 | 16 | 1, 32, 33, 32 | 16]


@pytest.fixture(scope="module")
def s(torch_cuda):
    import slhav2_amd

    return slhav2_amd


@pytest.fixture(scope="module")
def torch(torch_cuda):
    return torch_cuda


def dev(torch, a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.cuda()


def tiles_np(t):
    return t.cpu().numpy().reshape(-1, 128).copy().view(o.TILE_DTYPE).reshape(-1)


def random_tiles(n, seed, flag_sets=FLAG_SETS):
    r = np.random.default_rng(seed)
    t = np.zeros(n, o.TILE_DTYPE)
    t["latent_kv"] = r.integers(0, 256, (n, 64), dtype=np.uint8)
    t["residual_bitmap"] = r.integers(0, 2**63, (n, 4), dtype=np.uint64) * 2 + r.integers(0, 2, (n, 4), dtype=np.uint64)
    t["scale"] = (r.random(n) * 2 + 0.01).astype(np.float32)
    t["dynamic_lambda"] = np.abs(r.normal(size=n) * 0.1).astype(np.float32)
    t["residual_sigma"] = r.random(n).astype(np.float32)
    t["group_scales"] = r.integers(1, 256, (n, 8), dtype=np.uint8)
    t["flags"] = np.asarray(flag_sets, np.uint16)[r.integers(0, len(flag_sets), n)]
    t["position"] = np.arange(n, dtype=np.uint32)
    return t


def keys_for(seed, n, kind="gauss"):
    r = o.Rng(seed)
    k = r.gaussian(n * 128).reshape(n, 128)
    if kind == "scaled":  # C4: per-token scale log-uniform in [0.1, 10]
        u = np.array([r.next_unit() for _ in range(n)], np.float32)
        k = (k * (np.float32(0.1) * np.float32(100.0) ** u)[:, None]).astype(np.float32)
    if kind == "student":  # C3: Student-t(4) with 4 outlier channels x20
        z = r.gaussian(n * 4 * 128).reshape(n, 128, 4)
        k = (k / np.sqrt((z ** 2).mean(-1))).astype(np.float32)
        k[:, [3, 17, 64, 100]] *= np.float32(20.0)
    k[0] = 0.0
    k[1] = ((np.arange(128) - 64) / 16.0).astype(np.float32)
    return k.astype(np.float32)


def assert_tol(got, ref):
    bad = np.abs(got.astype(np.float64) - ref) > TOL * (1 + np.abs(ref.astype(np.float64)))
    assert not bad.any(), (np.argwhere(bad)[:5], got[bad][:5], ref[bad][:5])


def test_audit_known_answer(s):
    rep = json.loads(s.audit())
    assert rep["ok"] is True and rep["kat_basic_usage"] == -8.0 and rep["tile_size"] == 128
    assert "gfx950" in rep["arch"]


@pytest.mark.parametrize("codec", range(6))
@pytest.mark.parametrize("rht", [False, True])
@pytest.mark.parametrize("kind", ["gauss", "scaled", "student"])
def test_encode_bit_exact(s, torch, codec, rht, kind):
    n_rows, n_tok, n_kv = 2, 193, 2
    keys = keys_for(1000 + codec, n_rows * n_tok, kind)
    with s.Model(seed=31 + codec, rht=rht) as m:
        z, diag = m.projection()
        for dtype in (torch.float32, torch.bfloat16):
            kin = keys if dtype == torch.float32 else o.bf16_round(keys)
            kd = dev(torch, kin.reshape(n_rows, n_tok, 128), dtype)
            tiles = tiles_np(s.gpu_encode(m, kd, codec, n_kv_heads=n_kv, pos0=5))
            for r in range(n_rows):
                ref = o.encode(kin[r * n_tok:(r + 1) * n_tok], codec, 1, z, diag if rht else None,
                               pos0=5, head=r % n_kv)
                got = tiles[r * n_tok:(r + 1) * n_tok]
                assert got.tobytes() == ref.tobytes(), (codec, rht, kind, dtype, r)


def near_orthogonal_keys(z, diag, n, seed):
    """INT4-single keys whose residual e is two dims (a, b) with
    w[a] e_a + w[b] e_b ~ 0, where w = z[s] (no RHT) or D H z[s] (RHT, so that
    RHT(e) . z[s] = e . w) for s = key index mod 256: projection s is within
    rounding of zero, so its sign bit cannot be certified from the MFMA value
    and goes through the sequential fallback."""
    import scipy.linalg

    w_all = z.astype(np.float64)
    if diag is not None:
        h = scipy.linalg.hadamard(128) / np.sqrt(128.0)
        w_all = (w_all @ h.T) * diag.astype(np.float64)[None, :]
    r = np.random.default_rng(seed)
    k = r.integers(-6, 7, (n, 128)).astype(np.float32)
    k[:, 0] = 7.0  # max |k| = 7: scale 1, integer dims are exact
    for i in range(n):
        w = w_all[i % 256]
        a, b = sorted(r.choice(np.arange(1, 128), 2, replace=False), key=lambda d: abs(w[d]))
        ea = r.uniform(0.05, 0.2)
        k[i, a] += np.float32(ea)
        k[i, b] += np.float32(-w[a] * ea / w[b])
    return k


@pytest.mark.parametrize("rht", [False, True])
def test_encode_sign_fallback_paths(s, torch, rht):
    """The MFMA sign sketch recomputes uncertain bits sequentially. Keys that
    force each path (per-bit queue, queue overflow to whole-key recompute,
    non-finite and out-of-range residuals, zero residuals) match the oracle
    byte for byte."""
    with s.Model(seed=77, rht=rht) as m:
        z, diag = m.projection()
        d = diag if rht else None
        r = np.random.default_rng(5)
        blocks = [
            near_orthogonal_keys(z, d, 512, 6),                    # queue, ~1+ entry per key
            (r.normal(size=(300, 128)) * 1e-36).astype(np.float32),  # tiny: every bit uncertain
            (r.normal(size=(64, 128)) * 1e-41).astype(np.float32),   # subnormal keys
            (r.normal(size=(64, 128)) * 1e37).astype(np.float32),    # |v| beyond 2^100
            np.zeros((70, 128), np.float32),                        # zero residual
            np.tile(np.arange(-7, 9, dtype=np.float32), 8)[None].repeat(40, 0),  # exact: e = 0
            r.normal(size=(200, 128)).astype(np.float32),
        ]
        bad = r.normal(size=(64, 128)).astype(np.float32)
        bad[::3, 5] = np.inf
        bad[1::3, 77] = np.nan
        blocks.append(bad)
        keys = np.concatenate(blocks)
        for codec in (0, 1, 4, 5):
            got = tiles_np(s.gpu_encode(m, dev(torch, keys), codec))
            ref = o.encode(keys, codec, 1, z, d)
            if got.tobytes() != ref.tobytes():
                diff = np.nonzero((got.view(np.uint8).reshape(-1, 128) != ref.view(np.uint8).reshape(-1, 128)).any(1))[0]
                raise AssertionError((codec, rht, diff[:10]))


def test_encode_small_quotient_boundaries(s, torch):
    """Quotients x / eff next to the codecs' decisions nearest to 0: NF4
    chooses between its levels -0.0421 and +0.0421 at t = 2^-29, and TQ3's
    code flips at t = -2^-23. Each 16-dim group's maximum fixes eff at 1
    (NF4 step = max, TQ3 step = max / 3.5), then the keys are scaled by
    powers of two so that eff is 2^-60 (inside the range of the reciprocal
    quotient) and 2^-80 (outside it: the division). Tile bytes equal the
    oracle's."""
    print("encode small quotients", flush=True)
    r = np.random.default_rng(41)

    def keys_near(t0, top, n):
        ulps = r.integers(-3, 4, size=(n, 128))
        base = np.full((n, 128), np.float32(t0))
        k = base.view(np.int32) + ulps.astype(np.int32)
        k = k.view(np.float32) * np.where(r.random((n, 128)) < 0.5, 1, -1).astype(np.float32)
        k[:, ::16] = np.float32(top)  # each group's maximum
        k[r.random((n, 128)) < 0.1] = 0.0
        k[:, ::16] = np.float32(top)
        return k.astype(np.float32)

    with s.Model(seed=43, rht=False) as m:
        z, _ = m.projection()
        for codec, t0, top in ((2, 2.0 ** -29, 1.0), (4, -(2.0 ** -23), 3.5), (2, 2.0 ** -32, 1.0),
                               (4, 2.0 ** -30, 3.5)):
            base = keys_near(t0, top, 192)
            for scale in (1.0, 2.0 ** -60, 2.0 ** -80):
                keys = (base * np.float32(scale)).astype(np.float32)
                got = tiles_np(s.gpu_encode(m, dev(torch, keys), codec))
                ref = o.encode(keys, codec, 1, z, None)
                if got.tobytes() != ref.tobytes():
                    g = got.view(np.uint8).reshape(-1, 128)
                    rr = ref.view(np.uint8).reshape(-1, 128)
                    raise AssertionError((codec, t0, scale, np.nonzero((g != rr).any(1))[0][:10]))


def boundary_keys(n, seed):
    """Keys whose elements sit on, or one or two ulps from, the codecs'
    rounding boundaries: with max |k| = 7 (INT4 step 1) every half-integer
    is a roundf tie; with group maxima of 3.5 (TQ3 step 1) the elements are
    on or next to t + 3.5 = k + 1/2 and to the correction levels k - 3.5."""
    r = np.random.default_rng(seed)
    half = np.arange(-7, 7, dtype=np.float32) + np.float32(0.5)   # INT4 ties
    tq3 = np.concatenate([np.arange(-4, 4, dtype=np.float32),        # t + 3.5 half-integers
                          np.arange(0, 8, dtype=np.float32) - np.float32(3.5)])  # levels
    base = np.concatenate([half, tq3]).astype(np.float32)
    keys = r.choice(base, size=(n, 128)).astype(np.float32)
    nudge = r.integers(-2, 3, size=(n, 128))
    keys = np.nextafter(keys, np.where(nudge > 0, np.inf, -np.inf).astype(np.float32))
    keys = np.where(nudge == 0, r.choice(base, size=(n, 128)), keys).astype(np.float32)
    keys[:, 0] = 7.0                 # fix the INT4 step at 1
    keys[:, 16::16] = 3.5            # and each TQ3 group's step at 1
    keys[n // 2:] *= np.float32(0.37)  # non-unit steps too
    return keys


@pytest.mark.parametrize("rht", [False, True])
def test_encode_rounding_boundaries_bit_exact(s, torch, rht):
    """Codes (roundf ties to the larger magnitude, TQ3 correction bits at
    their levels) equal the oracle's for keys built on and around every
    rounding boundary."""
    keys = boundary_keys(512, 9)
    with s.Model(seed=78, rht=rht) as m:
        z, diag = m.projection()
        d = diag if rht else None
        for codec in (0, 1, 4):
            print(f"boundary keys codec={codec} rht={rht}", flush=True)
            got = tiles_np(s.gpu_encode(m, dev(torch, keys), codec))
            ref = o.encode(keys, codec, 1, z, d)
            assert got.tobytes() == ref.tobytes(), codec


def test_encode_c4_size_bit_exact(s, torch):
    # C4-like keys (N(0,1) x log-uniform scale, bf16), TQ3 + RHT, 131072 keys:
    # every tile byte against the oracle.
    keys = o.bf16_round(keys_for(4242, 131072, "scaled"))
    with s.Model(seed=0xC4, rht=True) as m:
        z, diag = m.projection()
        got = tiles_np(s.gpu_encode(m, dev(torch, keys, torch.bfloat16), s.CODEC_TQ3))
    ref = o.encode(keys, s.CODEC_TQ3, 1, z, diag)
    assert got.tobytes() == ref.tobytes()


@pytest.mark.parametrize("codec", [0, 2, 4])
def test_encode_mode_z_and_warm(s, torch, codec):
    keys = keys_for(7, 300)
    with s.Model(seed=5, rht=False, residual_mode=s.RESIDUAL_Z) as m:
        z, _ = m.projection()
        t = tiles_np(s.gpu_encode(m, dev(torch, keys), codec, warm=True))
    ref = o.encode(keys, codec, 0, z)
    ref["flags"] |= 1
    assert t.tobytes() == ref.tobytes()


@pytest.mark.parametrize("rht", [False, True])
def test_prepare_queries_bit_exact(s, torch, rht):
    q = keys_for(11, 97, "scaled")
    with s.Model(seed=12, rht=rht) as m:
        z, diag = m.projection()
        for dtype in (torch.float32, torch.bfloat16):
            qin = q if dtype == torch.float32 else o.bf16_round(q)
            qc, qs = s.gpu_prepare_queries(m, dev(torch, qin, dtype))
            qs = qs.cpu().numpy().view(np.uint64)
            assert np.array_equal(qc.cpu().numpy(), qin)
            for i in range(len(q)):
                assert np.array_equal(qs[i], o.query_sign(qin[i], z, diag if rht else None))


@pytest.mark.parametrize("group", [1, 4, 5, 8])
def test_score_exact_bit_identical_and_hamming(s, torch, group):
    n_rows, n_tok = 3, 777
    tiles = random_tiles(n_rows * n_tok, 40 + group)
    r = np.random.default_rng(group)
    q = r.normal(size=(n_rows * group, 128)).astype(np.float32)
    qs = r.integers(0, 2**63, (n_rows * group, 4), dtype=np.uint64)
    td = dev(torch, tiles.view(np.uint8).reshape(n_rows, n_tok, 128))
    qd, qsd = dev(torch, q), dev(torch, qs.view(np.int64))
    exact, ham = s.gpu_score(td, qd, qsd, group=group, mode=s.SCORE_EXACT, hamming=True)
    fast = s.gpu_score(td, qd, qsd, group=group, mode=s.SCORE_FAST)
    exact, ham, fast = exact.cpu().numpy(), ham.cpu().numpy(), fast.cpu().numpy()
    for row in range(n_rows):
        for j in range(group):
            qi = row * group + j
            ref, href = o.score(tiles[row * n_tok:(row + 1) * n_tok], q[qi], qs[qi])
            assert np.array_equal(exact[qi].view(np.uint32), ref.view(np.uint32))
            assert np.array_equal(ham[qi].astype(np.uint32), href)
            assert_tol(fast[qi], ref)


@pytest.mark.parametrize("group,codec", [(4, 0), (8, 2), (20, 4), (5, None), (24, 0), (64, 1),
                                         (33, None), (40, "tq3_nocorr"), (17, 2), (32, 0),
                                         (64, "tq3_mix"), (48, "tq3_mix"), (64, 4)])
def test_score_fast_streaming_ragged(s, torch, group, codec):
    # Many workgroups per row, a ragged last wave per row (n_tok not a
    # multiple of 64) and waves entirely past the end of the row. Groups
    # past 16 take the wide kernel (INT4 and TQ3 with and without the
    # correction plane on 32x32 MFMA; 32 and 64 queries fill whole query
    # blocks, 17..31, 33..63 leave rows of the last block unstored). codec
    # None: random mixed-codec tiles, so waves fall back to the per-lane
    # path. tq3_mix: TQ3 waves whose tiles mix corrected, NOCORR and WARM.
    n_rows, n_tok = 8, 50_001
    r = np.random.default_rng(1000 + group)
    if codec is None:
        td = dev(torch, random_tiles(n_rows * n_tok, 7).view(np.uint8).reshape(n_rows, n_tok, 128))
    else:
        g = torch.Generator(device="cuda").manual_seed(group)
        keys = torch.randn((n_rows, n_tok, 128), device="cuda", generator=g)
        with s.Model(seed=group) as m:
            td = s.gpu_encode(m, keys, s.CODEC_TQ3 if codec in ("tq3_nocorr", "tq3_mix") else codec,
                              n_kv_heads=n_rows)
        if codec == "tq3_nocorr":
            slots = torch.arange(n_rows * n_tok, dtype=torch.int32, device="cuda")
            s.gpu_ccos_apply(td, slots, 1)
        if codec == "tq3_mix":
            pick = np.random.default_rng(7).random(n_rows * n_tok)
            for op, sel in ((1, pick < 0.5), (0, (pick > 0.4) & (pick < 0.7))):
                slots = dev(torch, np.nonzero(sel)[0].astype(np.int32))
                s.gpu_ccos_apply(td, slots, op)
    q = r.normal(size=(n_rows * group, 128)).astype(np.float32)
    qs = r.integers(0, 2**63, (n_rows * group, 4), dtype=np.uint64)
    qd, qsd = dev(torch, q), dev(torch, qs.view(np.int64))
    fast = s.gpu_score(td, qd, qsd, group=group).cpu().numpy()
    exact = s.gpu_score(td, qd, qsd, group=group, mode=s.SCORE_EXACT).cpu().numpy()
    assert_tol(fast, exact)
    tn = tiles_np(td)
    for row in (0, n_rows - 1):
        idx = np.r_[0:70, n_tok - 70:n_tok]
        qi = row * group + group - 1
        ref, _ = o.score(tn[row * n_tok + idx], q[qi], qs[qi])
        assert np.array_equal(exact[qi, idx].view(np.uint32), ref.view(np.uint32))
        assert_tol(fast[qi, idx], ref)


@pytest.mark.parametrize("group", [1, 2, 3, 4])
def test_score_int4_hint_integer_path(s, torch, group):
    # slha_gpu_score_codec with the INT4 hint: the pipelined integer path
    # (group <= 4). Ragged rows (n_tok % 64 != 0 and % 16 != 0, waves past the
    # end), ~30 % WARM tiles, mode R keys; against SCORE_EXACT on every pair
    # and the oracle on sampled tokens of every row.
    n_rows, n_tok = 3, 5_003
    g = torch.Generator(device="cuda").manual_seed(77 + group)
    keys = torch.randn((n_rows, n_tok, 128), device="cuda", generator=g).to(torch.bfloat16)
    r = np.random.default_rng(group)
    q = r.normal(size=(n_rows * group, 128)).astype(np.float32)
    # Tiny and huge queries keep their relative precision: scores of a query
    # scaled by S are compared after dividing by S, so the tolerance's floor
    # of 1e-3 sits at the query's own scale (cancellation in a score is
    # relative to |q| |k|, as in the reference's SIMD-vs-scalar bar).
    qscale = np.ones(n_rows * group)
    qscale[0], qscale[-1] = 1e-30, 1e30
    q = (q * qscale[:, None]).astype(np.float32)
    if group > 1:
        # limb edges of the four-byte split of q 2^30 (max |q| = 1 sets the
        # prescale): values next to multiples of 2^8, 2^16, 2^24 and +-2^30
        # that f32 holds exactly
        cand = np.array([k * 2**sh + d for sh in (8, 16, 24) for k in (-64, -3, -1, 1, 2, 63)
                         for d in (-129, -128, -127, -1, 1, 127, 128)]
                        + [2**30, -(2**30), 2**30 - 128, -(2**30) + 128], np.float64)
        cand = cand[(np.abs(cand) <= 2**30) & (cand.astype(np.float32) == cand)]
        qe = np.resize(cand, 128)
        qe[1::2] = -qe[1::2]
        q[1] = (qe / 2**30).astype(np.float32)
        q[1, 0] = 1.0
    with s.Model(seed=5 + group) as m:
        td = s.gpu_encode(m, keys, s.CODEC_INT4_SINGLE, n_kv_heads=n_rows)
        warm = np.flatnonzero(r.random(n_rows * n_tok) < 0.3).astype(np.int32)
        s.gpu_ccos_apply(td, dev(torch, warm), 0)
        qc, qs = s.gpu_prepare_queries(m, dev(torch, q))
    hinted = s.gpu_score(td, qc, qs, group=group, codec_hint=s.CODEC_INT4_SINGLE).cpu().numpy()
    plain = s.gpu_score(td, qc, qs, group=group).cpu().numpy()
    exact = s.gpu_score(td, qc, qs, group=group, mode=s.SCORE_EXACT).cpu().numpy()
    qsc = qscale[:, None]
    assert_tol(hinted / qsc, exact / qsc)
    assert_tol(plain / qsc, exact / qsc)
    tn = tiles_np(td)
    qn, qsn = qc.cpu().numpy(), qs.cpu().numpy().view(np.uint64)
    idx = np.r_[0:80, 2_000:2_064, n_tok - 80:n_tok]
    for row in range(n_rows):
        for j in range(group):
            qi = row * group + j
            ref, _ = o.score(tn[row * n_tok + idx], qn[qi], qsn[qi])
            assert np.array_equal(exact[qi, idx].view(np.uint32), ref.view(np.uint32))
            assert_tol(hinted[qi, idx] / qscale[qi], ref / qscale[qi])


@pytest.mark.parametrize("group", [1, 2, 3, 4])
def test_score_nf4_hint_path(s, torch, group):
    # slha_gpu_score_codec with the NF4 hint: the f16 NF4 path (group <= 4),
    # levels as f16 hi + lo pairs. Keys with four x20 outlier channels (as
    # C3's), ragged rows, ~30 % WARM tiles, tiny and huge queries compared
    # at their own scale; against SCORE_EXACT on every pair and the oracle on
    # sampled tokens of every row.
    n_rows, n_tok = 3, 5_003
    g = torch.Generator(device="cuda").manual_seed(91 + group)
    keys = torch.randn((n_rows, n_tok, 128), device="cuda", generator=g)
    keys[..., [3, 17, 64, 100]] *= 20.0
    keys = keys.to(torch.bfloat16)
    r = np.random.default_rng(10 + group)
    q = r.normal(size=(n_rows * group, 128)).astype(np.float32)
    qscale = np.ones(n_rows * group)
    qscale[0], qscale[-1] = 1e-30, 1e30
    q = (q * qscale[:, None]).astype(np.float32)
    with s.Model(seed=15 + group) as m:
        td = s.gpu_encode(m, keys, s.CODEC_NF4, n_kv_heads=n_rows)
        warm = np.flatnonzero(r.random(n_rows * n_tok) < 0.3).astype(np.int32)
        s.gpu_ccos_apply(td, dev(torch, warm), 0)
        qc, qs = s.gpu_prepare_queries(m, dev(torch, q))
    hinted = s.gpu_score(td, qc, qs, group=group, codec_hint=s.CODEC_NF4).cpu().numpy()
    plain = s.gpu_score(td, qc, qs, group=group).cpu().numpy()
    exact = s.gpu_score(td, qc, qs, group=group, mode=s.SCORE_EXACT).cpu().numpy()
    qsc = qscale[:, None]
    assert_tol(hinted / qsc, exact / qsc)
    assert_tol(plain / qsc, exact / qsc)
    tn = tiles_np(td)
    qn, qsn = qc.cpu().numpy(), qs.cpu().numpy().view(np.uint64)
    idx = np.r_[0:80, 2_000:2_064, n_tok - 80:n_tok]
    for row in range(n_rows):
        for j in range(group):
            qi = row * group + j
            ref, _ = o.score(tn[row * n_tok + idx], qn[qi], qsn[qi])
            assert np.array_equal(exact[qi, idx].view(np.uint32), ref.view(np.uint32))
            assert_tol(hinted[qi, idx] / qscale[qi], ref / qscale[qi])


@pytest.mark.parametrize("case", ["mixed_codecs", "int4_tiles", "one_int4_tile"])
def test_score_nf4_hint_fallback(s, torch, case):
    # The NF4 hint on tiles that are not all NF4: such waves score on the
    # paths of the unhinted kernel; results match SCORE_EXACT either way.
    n_rows, n_tok, group = 2, 4_100, 4
    r = np.random.default_rng(hash(case) % 1000)
    if case == "mixed_codecs":
        td = dev(torch, random_tiles(n_rows * n_tok, 12).view(np.uint8).reshape(n_rows, n_tok, 128))
    else:
        g = torch.Generator(device="cuda").manual_seed(4)
        keys = torch.randn((n_rows, n_tok, 128), device="cuda", generator=g)
        codec = s.CODEC_INT4_GROUPED if case == "int4_tiles" else s.CODEC_NF4
        with s.Model(seed=10) as m:
            td = s.gpu_encode(m, keys, codec, n_kv_heads=n_rows)
        if case == "one_int4_tile":  # tile 33 of wave 1 loses its NF4 flag
            tn = td.cpu().numpy().reshape(-1, 128).copy()
            tn[64 + 33, 118] &= 0xFD
            td = dev(torch, tn.reshape(n_rows, n_tok, 128))
    q = r.normal(size=(n_rows * group, 128)).astype(np.float32)
    qs = r.integers(0, 2**63, (n_rows * group, 4), dtype=np.uint64)
    qd, qsd = dev(torch, q), dev(torch, qs.view(np.int64))
    hinted = s.gpu_score(td, qd, qsd, group=group, codec_hint=s.CODEC_NF4).cpu().numpy()
    exact = s.gpu_score(td, qd, qsd, group=group, mode=s.SCORE_EXACT).cpu().numpy()
    assert np.isfinite(hinted).all()
    assert_tol(hinted, exact)


@pytest.mark.parametrize("case", ["mx_int4", "mixed_codecs", "one_nf4_tile", "one_tile_gs", "nan_query"])
def test_score_int4_hint_fallback(s, torch, case):
    # The INT4 hint on tiles that do not all fit the integer path: a wave with
    # any such tile in any of its four 16-tile blocks scores on the per-lane
    # path; results match SCORE_EXACT either way. A NaN query value gives NaN
    # scores for that query, as on the other paths.
    n_rows, n_tok, group = 2, 4_100, 4
    r = np.random.default_rng(hash(case) % 1000)
    if case == "mixed_codecs":
        td = dev(torch, random_tiles(n_rows * n_tok, 11).view(np.uint8).reshape(n_rows, n_tok, 128))
    else:
        g = torch.Generator(device="cuda").manual_seed(3)
        keys = torch.randn((n_rows, n_tok, 128), device="cuda", generator=g)
        codec = s.CODEC_INT4_GROUPED if case == "mx_int4" else s.CODEC_INT4_SINGLE
        with s.Model(seed=9) as m:
            td = s.gpu_encode(m, keys, codec, n_kv_heads=n_rows)
        tn = td.cpu().numpy().reshape(-1, 128).copy()
        if case == "one_nf4_tile":  # tile 50 of wave 1 (block 3) is NF4
            tn[64 + 50, 118] |= 2
        if case == "one_tile_gs":  # tile 20 of wave 2 (block 1): unequal group scales
            tn[128 + 20, 121] = 200
        td = dev(torch, tn.reshape(n_rows, n_tok, 128))
    q = r.normal(size=(n_rows * group, 128)).astype(np.float32)
    if case == "nan_query":
        q[5, 77] = np.nan
    qs = r.integers(0, 2**63, (n_rows * group, 4), dtype=np.uint64)
    qd, qsd = dev(torch, q), dev(torch, qs.view(np.int64))
    hinted = s.gpu_score(td, qd, qsd, group=group, codec_hint=s.CODEC_INT4_SINGLE).cpu().numpy()
    exact = s.gpu_score(td, qd, qsd, group=group, mode=s.SCORE_EXACT).cpu().numpy()
    if case == "nan_query":
        assert np.isnan(hinted[5]).all() and np.isnan(exact[5]).all()
        keep = np.ones(n_rows * group, bool)
        keep[5] = False
        hinted, exact = hinted[keep], exact[keep]
    assert np.isfinite(hinted).all()
    assert_tol(hinted, exact)


def test_score_int4_hint_unaligned_output(s, torch):
    # Output rows that are not 16-byte aligned (scores buffer at an offset of
    # one float; n_tok a multiple of 4 and not) take the per-element stores.
    n_rows, group = 2, 4
    for n_tok in (4_096, 4_098):
        g = torch.Generator(device="cuda").manual_seed(n_tok)
        keys = torch.randn((n_rows, n_tok, 128), device="cuda", generator=g)
        q = torch.randn((n_rows * group, 128), device="cuda", generator=g)
        with s.Model(seed=2) as m:
            td = s.gpu_encode(m, keys, s.CODEC_INT4_SINGLE, n_kv_heads=n_rows)
            qc, qs = s.gpu_prepare_queries(m, q)
        buf = torch.full((n_rows * group * n_tok + 1,), -7.0, dtype=torch.float32, device="cuda")
        view = buf[1:].view(n_rows * group, n_tok)
        s.gpu_score(td, qc, qs, group=group, codec_hint=s.CODEC_INT4_SINGLE, out=view)
        exact = s.gpu_score(td, qc, qs, group=group, mode=s.SCORE_EXACT).cpu().numpy()
        assert buf[0].item() == -7.0
        assert_tol(view.cpu().numpy(), exact)


def test_score_codec_hint_rejects_unknown(s, torch):
    tiles = torch.zeros((1, 64, 128), dtype=torch.uint8, device="cuda")
    qc = torch.zeros((1, 128), dtype=torch.float32, device="cuda")
    qs = torch.zeros((1, 4), dtype=torch.int64, device="cuda")
    out = torch.empty((1, 64), dtype=torch.float32, device="cuda")
    vp = s.ctypes.c_void_p
    for bad in (-2, 6):
        rc = s.lib.slha_gpu_score_codec(vp(tiles.data_ptr()), 1, 64, vp(qc.data_ptr()),
                                        vp(qs.data_ptr()), 1, s.SCORE_FAST, bad,
                                        vp(out.data_ptr()), None, None)
        assert rc == s.ERR_CODEC


def test_score_fast_wide_group_c4_shape(s, torch):
    # C4 shape: one row, 64 queries per tile (TQ3 + RHT tiles).
    keys = keys_for(99, 2048, "scaled")
    with s.Model(seed=4, rht=True) as m:
        tiles = s.gpu_encode(m, dev(torch, o.bf16_round(keys)), s.CODEC_TQ3)
        q = o.bf16_round(keys_for(98, 64))
        qc, qs = s.gpu_prepare_queries(m, dev(torch, q, torch.bfloat16))
        sc = s.gpu_score(tiles, qc, qs, group=64).cpu().numpy()
    tnp = tiles_np(tiles)
    qsn = qs.cpu().numpy().view(np.uint64)
    for j in range(0, 64, 7):
        ref, _ = o.score(tnp, q[j], qsn[j])
        assert_tol(sc[j], ref)


def test_host_abi_paths(s, torch):
    with s.Model(seed=21, rht=False) as m:
        z, _ = m.projection()
        keys = keys_for(5, 40)
        for codec in range(6):
            t = s.encode_key(m, keys[3], position=9, codec=codec)
            ref = o.encode(keys[3:4], codec, 1, z, pos0=9)[0]
            assert t.tobytes() == ref.tobytes()
            assert np.array_equal(s.decode_latent(m, t), o.dequant(ref))
        qc, qs = s.prepare_query(m, keys[7])
        assert np.array_equal(qc, keys[7]) and np.array_equal(qs, o.query_sign(keys[7], z))
        tiles = o.encode(keys, 1, 1, z)
        got = s.score_tiles(m, tiles, qc, qs)
        ref, _ = o.score(tiles, qc, qs)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
        assert s.score_tile(m, tiles[4], qc, qs) == ref[4]
        assert s.process_tile(tiles[4], qc, qs) == ref[4]
        # decode_key: latent + sign-sketch estimate (learned.rs:283-321)
        dk = s.decode_key(m, tiles[2])
        sc = np.float32(tiles[2]["residual_sigma"]) * np.float32(np.sqrt(np.float32(np.pi / 2))) / np.float32(256)
        bits = np.unpackbits(tiles[2]["residual_bitmap"].view(np.uint8), bitorder="little")
        est = o.dequant(tiles[2]).astype(np.float64) + ((1 - 2 * bits.astype(np.float64)) * sc) @ z
        assert np.max(np.abs(dk - est)) < 1e-4
        # a bad tile anywhere leaves every output untouched (slha.h:193-195)
        bad = tiles.copy()
        bad[5]["flags"] = 0x40
        out = np.full(len(bad), 3.0, np.float32)
        rc = s.lib.slha_score_tiles(m.handle, bad.ctypes.data, len(bad), qc.ctypes.data,
                                    qs.ctypes.data, out.ctypes.data)
        assert rc == s.ERR_INVALID_TILE and np.all(out == 3.0)


def test_validate_kernel(s, torch):
    tiles = random_tiles(5000, 3)
    tiles[4000]["flags"] = 2 | 8
    tiles[1234]["scale"] = np.nan
    tiles[3000]["dynamic_lambda"] = -1.0
    res = s.gpu_validate_tiles(dev(torch, tiles.view(np.uint8).reshape(-1, 128)))
    first = next(i for i in range(len(tiles)) if o.validate(tiles[i]) != 0)
    assert res == (first, o.validate(tiles[first])) == (1234, -5)
    assert s.gpu_validate_tiles(dev(torch, random_tiles(100, 4).view(np.uint8).reshape(-1, 128))) is None


def test_ccos_apply(s, torch):
    tiles = random_tiles(512, 8, [0, 2, 8, 32, 8 | 16])
    td = dev(torch, tiles.view(np.uint8).reshape(-1, 128))
    slots = np.arange(0, 512, 3, dtype=np.int32)
    s.gpu_ccos_apply(td, dev(torch, slots), 1)
    s.gpu_ccos_apply(td, dev(torch, slots[::2].copy()), 0)
    want = tiles.copy()
    for i in slots:
        want[i:i + 1] = o.drop_correction(want[i])[0]
    for i in slots[::2]:
        want[i:i + 1] = o.page_out(want[i])
    assert tiles_np(td).tobytes() == want.tobytes()


def build_paged(lens, n_kv, page_tiles, seed, tiles_src):
    """Cut per-(seq, head) token streams into pages and shuffle them in one arena."""
    r = np.random.default_rng(seed)
    max_pages = max(1, max(-(-l // page_tiles) for l in lens))
    logical = []
    for si, l in enumerate(lens):
        for h in range(n_kv):
            for p in range(-(-l // page_tiles)):
                logical.append((si, h, p))
    perm = r.permutation(len(logical))
    arena = np.zeros(max(len(logical), 1) * page_tiles, o.TILE_DTYPE)
    table = np.zeros((len(lens), n_kv, max_pages), np.int32)
    for phys, li in enumerate(perm):
        si, h, p = logical[li]
        table[si, h, p] = phys
        src = tiles_src[(si, h)]
        chunk = src[p * page_tiles:(p + 1) * page_tiles]
        arena[phys * page_tiles:phys * page_tiles + len(chunk)] = chunk
    return arena, table, max_pages


# page_tiles >= 64 takes the wave-gather fast kernel, 16 the per-lane one;
# flags [0] gives uniform INT4 waves (f16 MFMA path), [0, 2] mixed waves.
@pytest.mark.parametrize("const_scores,page_tiles,flag_set,group", [
    (False, 256, (0, 2), 4), (True, 256, (0, 2), 4), (False, 64, (0,), 4),
    (False, 4096, (0,), 8), (False, 16, (0,), 4), (True, 64, (0,), 4)])
def test_paged_topk(s, torch, const_scores, page_tiles, flag_set, group):
    lens = [1, 63, 64, 1000, 5000, 300]
    n_kv, k = 2, 64
    r = np.random.default_rng(11)
    src = {}
    for si, l in enumerate(lens):
        for h in range(n_kv):
            t = random_tiles(l, 100 * si + h, list(flag_set))
            warm = r.random(l) < 0.3
            for i in np.nonzero(warm)[0]:
                t[i:i + 1] = o.page_out(t[i])
            if const_scores:  # identical tiles: every score ties, top-k = first k tokens
                t[:] = t[0]
            src[(si, h)] = t
    arena, table, max_pages = build_paged(lens, n_kv, page_tiles, 5, src)
    hq = n_kv * group
    q = r.normal(size=(len(lens) * hq, 128)).astype(np.float32)
    qs = r.integers(0, 2**63, (len(lens) * hq, 4), dtype=np.uint64)
    scores, idx, val = s.gpu_score_paged_topk(
        dev(torch, arena.view(np.uint8).reshape(-1, 128)), page_tiles, dev(torch, table),
        max_pages, dev(torch, np.asarray(lens, np.int32)), n_kv, group, dev(torch, q),
        dev(torch, qs.view(np.int64)), k)
    scores, idx, val = scores.cpu().numpy(), idx.cpu().numpy().view(np.uint32), val.cpu().numpy()
    base = 0
    for si, l in enumerate(lens):
        for qh in range(hq):
            h = qh // group
            got = scores[base + qh * l: base + (qh + 1) * l]
            ref, _ = o.score(src[(si, h)], q[si * hq + qh], qs[si * hq + qh])
            assert_tol(got, ref)
            ti, tv = o.topk(got, k)
            assert np.array_equal(idx[si, qh], ti), (si, qh)
            if const_scores:
                assert list(ti[: min(k, l)]) == list(range(min(k, l)))
            assert np.array_equal(val[si, qh][: min(k, l)], tv[: min(k, l)])
        base += hq * l


def test_paged_topk_many_sequences(s, torch):
    # Eleven ragged sequences (one token to past two segments), 30 % WARM
    # tiles, mixed INT4/NF4 waves and a tie plateau across a segment edge;
    # two calls in a row on one stream (the per-stream top-k workspace is
    # reused), each checked row by row against the oracle.
    lens = [17000, 1, 300, 40000, 64, 5000, 16384, 999, 20000, 7, 16385]
    n_kv, group, k, page_tiles = 2, 4, 64, 256
    hq = n_kv * group
    for call in range(2):
        print(f"paged many-sequence call {call}", flush=True)
        r = np.random.default_rng(31 + call)
        src = {}
        for si, l in enumerate(lens):
            for h in range(n_kv):
                t = random_tiles(l, 7000 * call + 100 * si + h, [0, 2])
                for i in np.nonzero(r.random(l) < 0.3)[0]:
                    t[i:i + 1] = o.page_out(t[i])
                src[(si, h)] = t
        # a plateau straddling the first segment edge of sequence 0, head 1
        q = r.normal(size=(len(lens) * hq, 128)).astype(np.float32)
        qs = r.integers(0, 2**63, (len(lens) * hq, 4), dtype=np.uint64)
        t = src[(0, 1)]
        t[16384 - 20:16384 + 60] = t[16384 - 20]
        arena, table, max_pages = build_paged(lens, n_kv, page_tiles, 9 + call, src)
        scores, idx, val = s.gpu_score_paged_topk(
            dev(torch, arena.view(np.uint8).reshape(-1, 128)), page_tiles, dev(torch, table),
            max_pages, dev(torch, np.asarray(lens, np.int32)), n_kv, group, dev(torch, q),
            dev(torch, qs.view(np.int64)), k)
        scores, idx, val = scores.cpu().numpy(), idx.cpu().numpy().view(np.uint32), val.cpu().numpy()
        base = 0
        for si, l in enumerate(lens):
            for qh in range(hq):
                h = qh // group
                got = scores[base + qh * l: base + (qh + 1) * l]
                ref, _ = o.score(src[(si, h)], q[si * hq + qh], qs[si * hq + qh])
                assert_tol(got, ref)
                ti, tv = o.topk(got, k)
                assert np.array_equal(idx[si, qh], ti), (call, si, qh)
                assert np.array_equal(val[si, qh].view(np.uint32), tv.view(np.uint32)), (call, si, qh)
            base += hq * l


def test_c1_cpu_reference_config(s, torch):
    # 4096 f32 N(0,1) keys, INT4, one f32 N(0,1) query.
    keys = o.Rng(0x5EED0000).gaussian(4096 * 128).reshape(4096, 128)
    q = o.Rng(0x5EED0001).gaussian(128)
    with s.Model(seed=0x5EED0002) as m:
        z, _ = m.projection()
        td = s.gpu_encode(m, dev(torch, keys), s.CODEC_INT4_SINGLE)
        qc, qs = s.gpu_prepare_queries(m, dev(torch, q[None]))
        exact, ham = s.gpu_score(td, qc, qs, mode=s.SCORE_EXACT, hamming=True)
        fast = s.gpu_score(td, qc, qs)
    ref_t = o.encode(keys, 0, 1, z)
    assert tiles_np(td).tobytes() == ref_t.tobytes()
    ref, href = o.score(ref_t, q, o.query_sign(q, z))
    assert np.array_equal(exact.cpu().numpy()[0].view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(ham.cpu().numpy()[0].astype(np.uint32), href)
    assert_tol(fast.cpu().numpy()[0], ref)


def test_c2_full_size_properties(s, torch):
    # BASELINE configs[1] at full size: 8 KV heads x 32768 bf16 keys, 32 queries.
    g = torch.Generator(device="cuda").manual_seed(0x5EED0001)
    keys = torch.randn((8, 32768, 128), device="cuda", generator=g).to(torch.bfloat16)
    q = torch.randn((32, 128), device="cuda", generator=g).to(torch.bfloat16)
    with s.Model(seed=0x5EED0002) as m:
        z, _ = m.projection()
        tiles = s.gpu_encode(m, keys, s.CODEC_INT4_SINGLE, n_kv_heads=8)
        qc, qs = s.gpu_prepare_queries(m, q)
        fast = s.gpu_score(tiles, qc, qs, group=4)
        hinted = s.gpu_score(tiles, qc, qs, group=4, codec_hint=s.CODEC_INT4_SINGLE)
        exact, ham = s.gpu_score(tiles, qc, qs, group=4, mode=s.SCORE_EXACT, hamming=True)
    fast, exact, ham = fast.cpu().numpy(), exact.cpu().numpy(), ham.cpu().numpy()
    hinted = hinted.cpu().numpy()
    assert fast.shape == (32, 32768)
    assert_tol(fast, exact)
    assert_tol(hinted, exact)
    # sampled oracle checks: tile bytes, Hamming, exact scores
    kn = keys.float().cpu().numpy()
    tn = tiles.cpu().numpy().reshape(8, 32768, 128)
    qn, qsn = q.float().cpu().numpy(), qs.cpu().numpy().view(np.uint64)
    r = np.random.default_rng(0)
    for h in range(8):
        idx = np.sort(r.choice(32768, 256, replace=False))
        ref_t = o.encode(kn[h, idx], 0, 1, z)
        ref_t["position"] = idx
        ref_t["token_id"] = idx
        ref_t["head_id"] = h
        got_t = tn[h, idx].copy().view(o.TILE_DTYPE).reshape(-1)
        assert got_t.tobytes() == ref_t.tobytes()
        for j in range(4):
            qi = 4 * h + j
            ref, href = o.score(ref_t, qn[qi], qsn[qi])
            assert np.array_equal(exact[qi, idx].view(np.uint32), ref.view(np.uint32))
            assert np.array_equal(ham[qi, idx].astype(np.uint32), href)
    # Hamming is an integer in [0, 256] with mean ~128 for independent signs
    assert ham.min() >= 0 and ham.max() <= 256 and abs(ham.mean() - 128) < 2
