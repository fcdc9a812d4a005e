"""Golden vectors (tests/golden/slha_golden.npz, written by make_golden.py).

CPU: the oracle still reproduces the committed vectors byte for byte, and the
vectors satisfy what the mathematics fixes independently of the oracle
(brute-force popcount, WARM = coarse, hot - warm = lambda (256 - 2 h)).
GPU: the HIP library reproduces the committed tiles and Hamming distances
bit-exactly, exact scores bit-identically and fast scores within 1e-3*(1+|s|).
"""
from pathlib import Path

import numpy as np
import pytest

import oracle_ffi as o

GOLDEN = Path(__file__).resolve().parent / "golden" / "slha_golden.npz"
SEED = 0x5EED0C0D
RHT_XOR = 0xA2A2A2A2A2A2A2A2  # learned.rs:158-165
POS0 = 100
TOL = 1e-3


@pytest.fixture(scope="module")
def g():
    with np.load(GOLDEN, allow_pickle=False) as d:
        return {k: d[k] for k in d.files}


def names(g):
    return sorted(k[len("tiles_"):] for k in g if k.startswith("tiles_"))


def tiles_of(g, name):
    return g[f"tiles_{name}"].copy().view(o.TILE_DTYPE).reshape(-1)


def rht_of(name):
    return int(name.split("_")[1][1:])


def test_fixture_inventory(g):
    ns = names(g)
    assert len(ns) == 6 * 2 * 2 + 2 * 2 + 2  # hot+warm per codec/RHT, nocorr TQ3/MIX3, modez INT4
    assert g["keys"].shape == (32, 128) and g["queries"].shape == (3, 128)


def test_oracle_reproduces_golden_vectors(g):
    z = o.projection(SEED)
    diag = o.rht_diag(SEED ^ RHT_XOR)
    assert np.array_equal(z.reshape(-1)[:8], g["z_head"])
    assert z.astype(np.float64).sum() == g["z_sum"][0]
    assert np.array_equal(diag, g["diag"])
    for r in (0, 1):
        d = diag if r else None
        qs = np.stack([o.query_sign(q, z, d) for q in g["queries"]])
        assert np.array_equal(qs, g[f"q_sign_rht{r}"])
    for name in names(g):
        c, r, v = int(name[1]), rht_of(name), name.split("_")[2]
        d = diag if r else None
        ref = o.encode(g["keys"], c, 0 if v == "modez" else 1, z, d, pos0=POS0, head=0)
        if v == "warm":
            ref = np.concatenate([o.page_out(t) for t in ref])
        if v == "nocorr":
            ref = np.concatenate([o.drop_correction(t)[0] for t in ref])
        assert ref.tobytes() == g[f"tiles_{name}"].tobytes(), name
        for j, q in enumerate(g["queries"]):
            s, h = o.score(ref, q, g[f"q_sign_rht{r}"][j])
            assert np.array_equal(s.view(np.uint32), g[f"scores_{name}"][j].view(np.uint32)), name
            assert np.array_equal(h, g[f"ham_{name}"][j]), name


def test_golden_hamming_is_brute_force_popcount(g):
    for name in names(g):
        t = tiles_of(g, name)
        qs = g[f"q_sign_rht{rht_of(name)}"]
        for j in range(3):
            x = t["residual_bitmap"] ^ qs[j][None, :]
            bits = np.unpackbits(x.view(np.uint8).reshape(len(t), -1), axis=1).sum(axis=1)
            assert np.array_equal(bits.astype(np.uint32), g[f"ham_{name}"][j]), name


def test_golden_warm_is_coarse_and_hot_adds_residual_term(g):
    for name in names(g):
        if not name.endswith("_hot"):
            continue
        warm = name[: -len("hot")] + "warm"
        t = tiles_of(g, name)
        tw = tiles_of(g, warm)
        assert (tw["flags"] & 1).all() and (tw["dynamic_lambda"] == 0).all()
        assert (tw["residual_bitmap"] == 0).all()
        for j, q in enumerate(g["queries"]):
            # WARM = coarse = sum q.dequant; check against a float64 dot product
            deq = np.stack([o.dequant(x) for x in tw]).astype(np.float64)
            coarse64 = deq @ q.astype(np.float64)
            sw = g[f"scores_{warm}"][j].astype(np.float64)
            assert np.all(np.abs(sw - coarse64) <= 1e-5 * (1 + np.abs(coarse64).max())), warm
            # hot = coarse + lambda (256 - 2 h), both rounded in f32
            lam = t["dynamic_lambda"].astype(np.float64)
            term = lam * (256.0 - 2.0 * g[f"ham_{name}"][j])
            sh = g[f"scores_{name}"][j].astype(np.float64)
            assert np.all(np.abs(sh - (sw + term)) <= 1e-5 * (1 + np.abs(sh))), name


def test_golden_mode_z_has_no_residual(g):
    for r in (0, 1):
        t = tiles_of(g, f"c0_r{r}_modez")
        hot = tiles_of(g, f"c0_r{r}_hot")
        assert (t["residual_bitmap"] == 0).all() and (t["dynamic_lambda"] == 0).all()
        assert (t["residual_sigma"] == 0).all()
        assert np.array_equal(t["latent_kv"], hot["latent_kv"])
        for j in range(3):
            # zero residual: Hamming = popcount(q_sign); score = coarse = WARM score
            expect = int(np.unpackbits(g[f"q_sign_rht{r}"][j].view(np.uint8)).sum())
            assert (g[f"ham_c0_r{r}_modez"][j] == expect).all()
            assert np.array_equal(g[f"scores_c0_r{r}_modez"][j], g[f"scores_c0_r{r}_warm"][j])


@pytest.mark.gpu
def test_gpu_reproduces_golden_vectors(g, torch_cuda):
    import slhav2_amd as s

    torch = torch_cuda
    keys = torch.from_numpy(g["keys"]).cuda()
    qd = torch.from_numpy(g["queries"]).cuda()
    for r in (0, 1):
        with s.Model(seed=SEED, rht=bool(r), residual_mode=s.RESIDUAL_R) as m, \
             s.Model(seed=SEED, rht=bool(r), residual_mode=s.RESIDUAL_Z) as mz:
            qc, qs = s.gpu_prepare_queries(m, qd)
            assert np.array_equal(qs.cpu().numpy().view(np.uint64), g[f"q_sign_rht{r}"])
            for c in range(6):
                hot = s.gpu_encode(m, keys, c, pos0=POS0)
                got = {"hot": hot}
                warm = hot.clone()
                slots = torch.arange(32, dtype=torch.int32, device="cuda")
                s.gpu_ccos_apply(warm, slots, 0)
                got["warm"] = warm
                if c in (4, 5):
                    nc = hot.clone()
                    s.gpu_ccos_apply(nc, slots, 1)
                    got["nocorr"] = nc
                if c == 0:
                    got["modez"] = s.gpu_encode(mz, keys, c, pos0=POS0)
                for v, t in got.items():
                    name = f"c{c}_r{r}_{v}"
                    assert np.array_equal(t.cpu().numpy().reshape(32, 128), g[f"tiles_{name}"]), name
                    # score the committed tiles (not the GPU's own) on the GPU
                    td = torch.from_numpy(g[f"tiles_{name}"]).cuda().reshape(1, 32, 128)
                    qsd = torch.from_numpy(g[f"q_sign_rht{r}"].view(np.int64)).cuda()
                    for j in range(3):
                        ex, hm = s.gpu_score(td, qc[j:j + 1], qsd[j:j + 1], mode=s.SCORE_EXACT,
                                             hamming=True)
                        fast = s.gpu_score(td, qc[j:j + 1], qsd[j:j + 1])
                        ref = g[f"scores_{name}"][j]
                        assert np.array_equal(ex.cpu().numpy()[0].view(np.uint32), ref.view(np.uint32)), name
                        assert np.array_equal(hm.cpu().numpy()[0].astype(np.uint32), g[f"ham_{name}"][j]), name
                        f = fast.cpu().numpy()[0].astype(np.float64)
                        assert np.all(np.abs(f - ref) <= TOL * (1 + np.abs(ref))), name
