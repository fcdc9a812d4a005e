"""CCOS ElasticKvCache over a device arena (scirust/src/ccos.rs,
scirust/tests/ccos.rs).

CPU tests pin the oracle's observe_scores (ccos.rs:257-300) against float64
softmax and the reference's own invalid-input cases, and check argument
errors of the C ABI. GPU tests run the reference's CCOS tests
(tests/ccos.rs:37-789) through slha_ccos_* with tiles from this build's GPU
encoder: the budget ladder, page-out and eviction orders, the TQ3 / MIX3
correction rung, H2O importance from scores observed on the GPU (compared
with the oracle), sinks, and COLD eviction to an EventLog with rehydrate.
"""
import numpy as np
import pytest

import oracle_ffi as o

HOT, WARM = 128, 96
TQ3_CORR, MIX3_CORR = 16, 14


# --------------------------------------------------------------------------
# Oracle pinning (CPU)


def test_observe_scores_oracle_against_float64():
    r = np.random.default_rng(4)
    for n, t in ((1, 1.0), (7, 0.5), (1000, 0.25), (4096, 3.0)):
        sc = (r.standard_normal(n) * 5).astype(np.float32)
        live = (r.random(n) > 0.3).astype(np.uint8)
        live[0] = 1
        imp = o.observe_scores(np.zeros(n, np.float32), sc, live, t)
        x = sc.astype(np.float64)[live == 1]
        ref = np.exp((x - x.max()) / t)
        ref /= ref.sum()
        np.testing.assert_allclose(imp[live == 1], ref, rtol=2e-5, atol=1e-9)
        assert not imp[live == 0].any()
        assert abs(float(imp.sum()) - 1.0) < 1e-4


def test_observe_scores_oracle_rejects_invalid_inputs():
    """tests/ccos.rs:243-261 and ccos.rs:266-289."""
    live = np.ones(1, np.uint8)
    for t in (0.0, -1.0, np.nan, np.inf):
        assert o.observe_scores(np.zeros(1), [1.0], live, t)[0] == 0.0
    for s in (np.nan, np.inf, -np.inf):
        assert o.observe_scores(np.zeros(1), [s], live, 1.0)[0] == 0.0
    # a COLD slot's score, even non-finite, is ignored; no live slot: no update
    imp = o.observe_scores(np.zeros(2), [0.0, np.nan], np.array([1, 0], np.uint8), 1.0)
    assert imp.tolist() == [1.0, 0.0]
    assert not o.observe_scores(np.zeros(2), [0.0, 1.0], np.zeros(2, np.uint8), 1.0).any()
    # accumulation (tests/ccos.rs:264-306)
    sc = np.array([0.0, 0.0, 10.0, 0.0], np.float32)
    imp = o.observe_scores(np.zeros(4), sc, np.ones(4, np.uint8), 0.5)
    assert imp[2] > 0.9 and imp[0] < 0.1 and abs(float(imp.sum()) - 1.0) <= 1e-4
    imp = o.observe_scores(imp, sc, np.ones(4, np.uint8), 0.5)
    assert imp[2] > 1.8


def test_ccos_argument_checks():
    import slhav2_amd as sa

    assert sa.lib.slha_ccos_new(None, 16, 0, 0, 0, 0) is None
    assert "NULL" in sa.last_error()
    assert sa.lib.slha_ccos_free(None) == sa.ERR_NULL
    assert sa.lib.slha_ccos_enforce_budget(None, None, None) == sa.ERR_NULL
    st = sa._CcosStats()
    import ctypes

    assert sa.lib.slha_ccos_stats(ctypes.c_void_p(64), ctypes.byref(st)) == sa.ERR_INVALID_HANDLE


# --------------------------------------------------------------------------
# GPU: the reference's CCOS tests through the C ABI


@pytest.fixture(scope="module")
def sa(torch_cuda):
    import slhav2_amd

    return slhav2_amd


@pytest.fixture(scope="module")
def torch(torch_cuda):
    return torch_cuda


def tiles_of(sa, torch, n, codec=0, seed=1, warm=False):
    """n tiles encoded on the GPU, positions 0..n-1 (uint8 [n, 128])."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    keys = torch.randn((1, n, 128), device="cuda", generator=g).to(torch.bfloat16)
    with sa.Model(seed=seed, rht=False) as m:
        return sa.gpu_encode(m, keys, codec, n_kv_heads=1, warm=warm).reshape(n, 128)


def with_sigma(torch, tiles, sigmas):
    t = tiles.cpu().numpy().copy().view(o.TILE_DTYPE).reshape(-1)
    t["residual_sigma"] = np.asarray(sigmas, np.float32)
    return torch.from_numpy(t.view(np.uint8).reshape(-1, 128).copy()).cuda()


def arena(torch, cap=256):
    return torch.zeros((cap, 128), dtype=torch.uint8, device="cuda")


def invariants(c, budget):
    """tests/ccos.rs:13-31."""
    assert c.live_bytes() <= budget
    h, w, _ = c.counts()
    assert h * HOT + w * WARM - c.reclaimed_correction_bytes() == c.live_bytes()


@pytest.mark.gpu
def test_enforce_budget_respects_budget_and_recycles(sa, torch):
    """tests/ccos.rs:37-76, 40 random configurations."""
    print("ccos prop", flush=True)
    pool = tiles_of(sa, torch, 48, seed=3)
    r = np.random.default_rng(0)
    for trial in range(40):
        n = 1 + int(r.integers(0, 48))
        budget = int(r.integers(0, n * HOT + 1))
        c = sa.ElasticKvCache(arena(torch, 128), budget, policy=trial % 2)
        for i in range(n):
            c.insert(pool[i:i + 1])
            if r.integers(0, 3) == 0:
                c.enforce_budget()
                invariants(c, budget)
        c.enforce_budget()
        invariants(c, budget)
        total = sum(c.counts())
        c.insert(pool[:n])
        assert sum(c.counts()) <= total + n
        c.close()


@pytest.mark.gpu
def test_page_out_masks_residual_and_falls_back_to_coarse(sa, torch):
    """tests/ccos.rs:79-100: WARM scores equal the coarse-only score."""
    t = tiles_of(sa, torch, 1, seed=2)
    c = sa.ElasticKvCache(arena(torch, 4), 1 << 60)
    slot = c.insert(t)[0]
    g = torch.Generator(device="cuda").manual_seed(9)
    with sa.Model(seed=2, rht=False) as m:
        qc, qs = sa.gpu_prepare_queries(m, torch.randn((1, 128), device="cuda", generator=g))
    _, hot, _ = c.score_all(qc, qs)
    c.page_out(slot)
    assert c.state(slot) == sa.WARM
    _, warm, _ = c.score_all(qc, qs)
    ref = o.page_out(t[0].cpu().numpy().view(o.TILE_DTYPE))
    assert c.arena[slot].cpu().numpy().tobytes() == ref.tobytes()
    warm_tile = tiles_of(sa, torch, 1, seed=2, warm=True)
    want = sa.gpu_score(warm_tile, qc, qs, mode=sa.SCORE_EXACT).item()
    assert warm[0] == np.float32(want) and hot[0] != warm[0]


@pytest.mark.gpu
def test_enforce_budget_bounds_live_bytes(sa, torch):
    c = sa.ElasticKvCache(arena(torch, 128), 50 * HOT)
    c.insert(tiles_of(sa, torch, 100, seed=42))
    assert c.live_bytes() > 50 * HOT
    c.enforce_budget()
    assert c.live_bytes() <= 50 * HOT
    _, w, cold = c.counts()
    assert w + cold > 0


@pytest.mark.gpu
def test_evict_recycles_slots(sa, torch):
    t = tiles_of(sa, torch, 4, seed=5)
    c = sa.ElasticKvCache(arena(torch, 8), 1 << 60, policy=sa.PAGE_OLDEST_FIRST)
    s0 = c.insert(t[0:1])[0]
    c.insert(t[1:2])
    assert c.evict(s0)
    assert c.state(s0) == sa.COLD
    s2 = c.insert(t[2:3])[0]
    assert s2 == s0 and c.state(s2) == sa.HOT
    assert c.arena[s2].cpu().numpy().tobytes() == t[2].cpu().numpy().tobytes()


@pytest.mark.gpu
def test_page_out_policies_differ(sa, torch):
    """tests/ccos.rs:137-163: sigma decreasing with slot order."""
    t = with_sigma(torch, tiles_of(sa, torch, 5, seed=6), [0.9, 0.7, 0.5, 0.3, 0.1])
    budget = 5 * HOT - 1
    lo = sa.ElasticKvCache(arena(torch, 8), budget, policy=sa.PAGE_LOWEST_IMPACT_FIRST)
    old = sa.ElasticKvCache(arena(torch, 8), budget, policy=sa.PAGE_OLDEST_FIRST)
    lo.insert(t)
    old.insert(t)
    lo.enforce_budget()
    old.enforce_budget()
    assert old.state(0) == sa.WARM and old.state(4) == sa.HOT
    assert lo.state(4) == sa.WARM and lo.state(0) == sa.HOT


@pytest.mark.gpu
def test_hybrid_evicts_oldest_not_lowest_impact(sa, torch):
    """tests/ccos.rs:166-192."""
    t = with_sigma(torch, tiles_of(sa, torch, 5, seed=11), [0.9, 0.7, 0.5, 0.3, 0.1])
    c = sa.ElasticKvCache(arena(torch, 8), 4 * 96)
    c.insert(t)
    c.enforce_budget()
    assert c.counts()[2] == 1
    assert c.state(0) == sa.COLD and c.state(4) == sa.WARM


@pytest.mark.gpu
def test_score_all_skips_cold_and_insert_keeps_warm(sa, torch):
    """tests/ccos.rs:195-220."""
    c = sa.ElasticKvCache(arena(torch, 8), 1 << 60, policy=sa.PAGE_OLDEST_FIRST)
    c.insert(tiles_of(sa, torch, 6, seed=8))
    c.evict(2)
    with sa.Model(seed=8, rht=False) as m:
        qc, qs = sa.gpu_prepare_queries(m, torch.ones((1, 128), device="cuda"))
    live, _, _ = c.score_all(qc, qs)
    assert len(live) == 5 and 2 not in live.tolist()
    w = sa.ElasticKvCache(arena(torch, 2), 1 << 60)
    slot = w.insert(tiles_of(sa, torch, 1, seed=9, warm=True))[0]
    assert w.state(slot) == sa.WARM and w.live_bytes() == WARM


@pytest.mark.gpu
@pytest.mark.parametrize("n,offset", [(3000, 0), (2999, 0), (3000, 1)])
def test_observe_scores_matches_oracle(sa, torch, n, offset):
    """GPU importance against the oracle's sequential f32 update, with COLD
    slots skipped; invalid inputs leave importance unchanged. (2999: a slot
    tail past the 4-slot groups; offset 1: scores not 16-byte aligned, the
    one-slot path.)"""
    print(f"ccos observe n={n} offset={offset}", flush=True)
    c = sa.ElasticKvCache(arena(torch, 4096), 1 << 60, policy=sa.PAGE_OLDEST_FIRST)
    pool = tiles_of(sa, torch, 1000, seed=12)
    c.insert(pool[:n - 2000])
    c.insert(pool)
    c.insert(pool)
    assert len(c) == n
    cold = np.random.default_rng(1).choice(n, 400, replace=False)
    for s in cold:
        c.evict(int(s))
    live = np.ones(n, np.uint8)
    live[cold] = 0
    r = np.random.default_rng(2)
    imp = np.zeros(n, np.float32)
    buf = torch.empty(n + offset, device="cuda")
    for step in range(4):
        sc = (r.standard_normal(n) * 4).astype(np.float32)
        sc[cold[:5]] = np.nan  # COLD slots never count
        buf[offset:] = torch.from_numpy(sc).cuda()
        c.observe_scores(buf[offset:], 0.7)
        imp = o.observe_scores(imp, sc, live, 0.7)
        got = c._slots()[2]
        np.testing.assert_allclose(got, imp, rtol=1e-5, atol=1e-8)
        assert not got[cold].any()
    before = c._slots()[2].copy()
    bad = np.zeros(n, np.float32)
    bad[int(np.nonzero(live)[0][-1])] = np.inf
    c.observe_scores(torch.from_numpy(bad).cuda(), 1.0)
    for t in (0.0, -1.0, float("nan"), float("inf")):
        c.observe_scores(torch.zeros(n, device="cuda"), t)
    assert (c._slots()[2] == before).all()


@pytest.mark.gpu
@pytest.mark.parametrize("t,spread", [(1e-20, 1e30), (0.7, 1e30), (1e-25, 1.0), (1e30, 1e3), (1e20, 1e-15)])
def test_observe_scores_extreme_temperatures_and_spreads(sa, torch, t, spread):
    """x / t where x yt overflows (spread / t beyond FLT_MAX: every weight but
    the maximum's is exp(-inf) = 0), temperatures outside the range of the
    reciprocal quotient (1e-25, 1e30: the division path), and quotients below
    2^-32 (1e-15 / 1e20: exp 1, uniform weights)."""
    print(f"ccos observe extreme t={t} spread={spread}", flush=True)
    n = 2000
    c = sa.ElasticKvCache(arena(torch, 2048), 1 << 60)
    c.insert(tiles_of(sa, torch, n, seed=21))
    live = np.ones(n, np.uint8)
    r = np.random.default_rng(22)
    imp = np.zeros(n, np.float32)
    for _ in range(2):
        sc = (r.standard_normal(n) * spread).astype(np.float32)
        c.observe_scores(torch.from_numpy(sc).cuda(), t)
        imp = o.observe_scores(imp, sc, live, t)
        np.testing.assert_allclose(c._slots()[2], imp, rtol=1e-5, atol=1e-8)


@pytest.mark.gpu
def test_informed_eviction_preserves_sinks_and_heavy_hitters(sa, torch):
    """tests/ccos.rs:309-394."""
    t = tiles_of(sa, torch, 8, seed=50)
    budget = 3 * WARM
    causal = sa.ElasticKvCache(arena(torch, 8), budget)
    informed = sa.ElasticKvCache.with_eviction(arena(torch, 8), budget, sink_window=2)
    causal.insert(t)
    informed.insert(t)
    sc = torch.zeros(8, device="cuda")
    sc[2] = 10.0
    for _ in range(5):
        informed.observe_scores(sc, 0.5)
    assert informed.importance(2) > 4.0
    causal.enforce_budget()
    informed.enforce_budget()
    assert causal.counts()[2] == 5 and informed.counts()[2] == 5
    assert [causal.state(s) for s in (0, 1, 2)] == [sa.COLD] * 3
    assert all(informed.state(s) != sa.COLD for s in (0, 1, 2))
    assert all(informed.state(s) == sa.COLD for s in (3, 4, 5, 6, 7))


@pytest.mark.gpu
def test_importance_eviction_with_no_sinks_is_pure_h2o(sa, torch):
    """tests/ccos.rs:397-465."""
    c = sa.ElasticKvCache.with_eviction(arena(torch, 8), 2 * WARM, sink_window=0)
    assert c.insert(tiles_of(sa, torch, 6, seed=70)) == list(range(6))
    c.observe_scores(torch.tensor([6.0 - i for i in range(6)], device="cuda"), 0.25)
    imp = [c.importance(s) for s in range(6)]
    assert abs(sum(imp) - 1.0) <= 1e-4
    assert all(imp[i] > imp[i + 1] for i in range(5))
    c.enforce_budget()
    assert c.counts()[2] == 4
    assert c.state(0) != sa.COLD and c.state(1) != sa.COLD
    assert all(c.state(s) == sa.COLD for s in range(2, 6))


@pytest.mark.gpu
@pytest.mark.parametrize("codec,corr", [(4, TQ3_CORR), (5, MIX3_CORR)])
def test_correction_rung_comes_before_paging(sa, torch, codec, corr):
    """tests/ccos.rs:485-497 (TQ3) and 569-583 (MIX3)."""
    n = 32
    budget = n * (HOT - corr)
    c = sa.ElasticKvCache(arena(torch, 32), budget)
    before = tiles_of(sa, torch, n, codec=codec, seed=7)
    c.insert(before)
    assert c.live_bytes() == n * HOT
    c.enforce_budget()
    invariants(c, budget)
    assert c.counts() == (n, 0, 0) and c.nocorr_count() == n
    assert c.reclaimed_correction_bytes() == n * corr and c.live_bytes() == budget
    t = before.cpu().numpy().view(o.TILE_DTYPE).reshape(-1)
    for s in range(n):  # the device bytes are drop_correction's
        want, _ = o.drop_correction(t[s:s + 1].copy())
        assert c.arena[s].cpu().numpy().tobytes() == want.tobytes()


@pytest.mark.gpu
def test_tq3_single_drop_and_ladder_to_warm(sa, torch):
    """tests/ccos.rs:500-529."""
    c = sa.ElasticKvCache(arena(torch, 16), 16 * HOT - TQ3_CORR)
    c.insert(tiles_of(sa, torch, 16, codec=4, seed=7))
    c.enforce_budget()
    assert c.counts() == (16, 0, 0) and c.nocorr_count() == 1
    c2 = sa.ElasticKvCache(arena(torch, 32), 32 * 96)
    c2.insert(tiles_of(sa, torch, 32, codec=4, seed=7))
    c2.enforce_budget()
    invariants(c2, 32 * 96)
    h, w, cold = c2.counts()
    assert cold == 0 and h + w == 32 and w > 0 and c2.nocorr_count() == 32


@pytest.mark.gpu
@pytest.mark.parametrize("codec", [1, 3])
def test_codecs_without_a_plane_skip_the_rung(sa, torch, codec):
    """tests/ccos.rs:532-548, 586-600 (grouped INT4, mixed)."""
    n = 16
    budget = n * 112 if codec == 1 else n * (HOT - MIX3_CORR)
    c = sa.ElasticKvCache(arena(torch, 16), budget)
    c.insert(tiles_of(sa, torch, n, codec=codec, seed=3))
    c.enforce_budget()
    invariants(c, budget)
    h, w, _ = c.counts()
    assert c.nocorr_count() == 0 and w > 0 and h + w == n


@pytest.mark.gpu
def test_tq3_ladder_is_deterministic(sa, torch):
    t = tiles_of(sa, torch, 24, codec=4, seed=7)
    a = sa.ElasticKvCache(arena(torch, 24), 24 * 100)
    b = sa.ElasticKvCache(arena(torch, 24), 24 * 100)
    a.insert(t)
    b.insert(t)
    a.enforce_budget()
    b.enforce_budget()
    assert a.live_bytes() == b.live_bytes()
    assert (a._slots()[0] == b._slots()[0]).all()
    assert a.arena.cpu().numpy().tobytes() == b.arena.cpu().numpy().tobytes()


@pytest.mark.gpu
def test_durable_eviction_persists_and_failure_keeps_tile_live(sa, torch, tmp_path):
    """tests/ccos.rs:610-686."""
    p = tmp_path / "ok"
    c = sa.ElasticKvCache(arena(torch, 4), 1 << 60)
    log = sa.EventLog.create(p)
    c.attach_durable_event_log(log)
    slot = c.insert(tiles_of(sa, torch, 1, seed=1))[0]
    assert c.evict(slot) and c.state(slot) == sa.COLD
    assert c.log_errors() == 0 and c.blocked_evictions() == 0
    with sa.EventLog.open(p) as r:
        assert len(r) == 1
    q = tmp_path / "ro"
    sa.EventLog.create(q).close()
    ro = sa.EventLog.open_read_only(q)
    c2 = sa.ElasticKvCache(arena(torch, 4), 0)
    c2.attach_durable_event_log(ro)
    t = tiles_of(sa, torch, 1, seed=2)
    slot = c2.insert(t)[0]
    assert not c2.enforce_budget()
    assert c2.state(slot) != sa.COLD and c2.live_bytes() > 0
    assert c2.log_errors() == 1 and c2.blocked_evictions() == 1
    assert c2.insert(t)[0] != slot
    with sa.EventLog.open(q) as r:
        assert len(r) == 0
    log.close()
    ro.close()


@pytest.mark.gpu
@pytest.mark.parametrize("durable", [True, False])
def test_failed_appends_evict_slot_by_slot(sa, torch, tmp_path, durable):
    """enforce_budget's eviction loop (ccos.rs:596-611) calls evict
    (ccos.rs:404-438) one slot at a time. With a log that refuses every
    append and three WARM slots (288 B) over a 200 B budget, one eviction
    would do: under RequireDurable every live slot is tried and blocked
    (3 log errors, 3 blocked, nothing evicted); best effort evicts the first
    slot after its failed append (1 log error, 0 blocked)."""
    q = tmp_path / "ro"
    sa.EventLog.create(q).close()
    ro = sa.EventLog.open_read_only(q)
    c = sa.ElasticKvCache(arena(torch, 8), 200, policy=sa.PAGE_OLDEST_FIRST)
    (c.attach_durable_event_log if durable else c.attach_event_log)(ro)
    slots = c.insert(tiles_of(sa, torch, 3, seed=31))
    within = c.enforce_budget()
    if durable:
        assert not within and c.counts() == (0, 3, 0)
        assert (c.log_errors(), c.blocked_evictions()) == (3, 3)
    else:
        assert within and c.counts() == (0, 2, 1) and c.state(slots[0]) == sa.COLD
        assert (c.log_errors(), c.blocked_evictions()) == (1, 0)
    # the device copy of the states follows every change: observe_scores
    # skips exactly the COLD slots, also after a recycled insert
    t = tiles_of(sa, torch, 2, seed=32)
    c.insert(t[:1])
    live = (c._slots()[0] != sa.COLD).astype(np.uint8)
    sc = np.array([1.0, 2.0, 3.0, 4.0][:len(c)], np.float32)
    c.observe_scores(torch.from_numpy(sc).cuda(), 1.0)
    want = o.observe_scores(np.zeros(len(c), np.float32), sc, live, 1.0)
    np.testing.assert_allclose(c._slots()[2], want, rtol=1e-5, atol=1e-8)
    with sa.EventLog.open(q) as r:
        assert len(r) == 0
    ro.close()
    c.close()


@pytest.mark.gpu
def test_evict_snapshots_to_event_log_then_rehydrates_identically(sa, torch, tmp_path):
    """tests/ccos.rs:689-747 and 750-767."""
    p = tmp_path / "rt"
    c = sa.ElasticKvCache(arena(torch, 8), 2 * HOT)
    log = sa.EventLog.create(p)
    c.attach_event_log(log)
    t = tiles_of(sa, torch, 5, seed=9)
    latents = t.cpu().numpy()[:, :64].copy()
    c.insert(t)
    c.enforce_budget()
    cold = c.counts()[2]
    assert cold >= 3 and c.log_errors() == 0
    with sa.EventLog.open(p) as r:
        recs = r.read_all()
    assert len(recs) == cold
    for rec in recs:
        assert rec["tile"][:64].tobytes() == latents[int(rec["seq"])].tobytes()
        assert rec["tile"].view(o.TILE_DTYPE)["flags"][0] & 1
    assert [int(x) for x in recs["seq"]] == list(range(cold))  # oldest first
    logged0 = recs[recs["seq"] == 0][0]["tile"].tobytes()
    slot = c.rehydrate(0)
    assert slot is not None and c.state(slot) == sa.WARM
    assert c.arena[slot].cpu().numpy().tobytes() == logged0
    assert c.importance(slot) == 0.0
    assert c.rehydrate(12345) is None
    log.close()
    d = sa.ElasticKvCache(arena(torch, 4), HOT)
    d.insert(tiles_of(sa, torch, 3, seed=2))
    d.enforce_budget()
    assert d.log_errors() == 0 and d.rehydrate(0) is None


@pytest.mark.gpu
def test_edge_cases_match_the_reference_contract(sa, torch):
    """A full arena rejects the insert before any change; evict of a COLD
    slot, page_out of a WARM slot and drop_correction on a tile without a
    correction plane change nothing (ccos.rs:369-438)."""
    c = sa.ElasticKvCache(arena(torch, 4), 1 << 60)
    t = tiles_of(sa, torch, 5, seed=21)
    c.insert(t[:4])
    with pytest.raises(sa.SlhaError) as e:
        c.insert(t[4:5])
    assert e.value.code == sa.ERR_DIMENSION and len(c) == 4
    assert c.evict(1) and not c.evict(1)
    assert c.live_bytes() == 3 * HOT
    c.page_out(0)
    before = c.arena[0].cpu().numpy().tobytes()
    c.page_out(0)
    assert c.state(0) == sa.WARM and c.arena[0].cpu().numpy().tobytes() == before
    assert not c.drop_correction(2)  # INT4: no plane
    assert c.live_bytes() == 2 * HOT + WARM
    assert c.insert(t[4:5]) == [1]  # the COLD slot is recycled
