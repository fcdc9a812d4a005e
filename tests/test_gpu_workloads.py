"""GPU parity at the shapes of BASELINE.json configs[2] (C3) and configs[4] (C5).

C5 (ccos.rs:346-355 score_all + top-k): rows longer than one 16 384-score
top-k segment go through the cross-segment merge. Rows straddle the segment
edges (16 383, 16 384, 16 385), span several segments (40 000, 131 072), and
carry score plateaus and whole constant rows whose ties cross segment edges,
so the (score desc, index asc) order is decided between segments.

C3 (codec/nf4.rs:23-57, codec/int4.rs:34-63): Student-t(4) bf16 keys with four
outlier channels x20 per KV head, NF4 and MX-INT4 tiles scored for 32 query
heads per sequence at GQA group 4; tile bytes against the oracle, fast against
exact on every pair, exact scores and Hamming bit-identical to the oracle on
sampled tokens of every row.
"""
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import oracle_ffi as o
from test_gpu_parity import assert_tol, build_paged, dev, random_tiles, tiles_np

pytestmark = pytest.mark.gpu

SEG = 16384  # scores per top-k segment of the paged path


@pytest.fixture(scope="module")
def s(torch_cuda):
    import slhav2_amd

    return slhav2_amd


@pytest.fixture(scope="module")
def torch(torch_cuda):
    return torch_cuda


def page_out_where(t, mask):
    """HOT -> WARM through the oracle's page_out (ccos.rs:369-382) for the
    tiles selected by `mask`."""
    for i in np.nonzero(mask)[0]:
        t[i:i + 1] = o.page_out(t[i])


def plateau_tile(base, q_sign, lam):
    """A HOT INT4 tile with a zero latent (every nibble 8) and residual =
    q_sign: for that query its score is exactly 256*lam (Hamming 0), above
    every random tile's."""
    t = np.array(base, o.TILE_DTYPE).reshape(1)
    t["latent_kv"] = 0x88
    t["residual_bitmap"] = q_sign
    t["dynamic_lambda"] = np.float32(lam)
    t["flags"] = 0
    return t


@pytest.mark.parametrize("group", [4, 8])
def test_c5_multi_segment_topk(s, torch, group):
    lens = [SEG - 1, SEG, SEG + 1, 40000, 131072]
    n_kv, k, page_tiles = 2, 64, 4096
    hq = n_kv * group
    r = np.random.default_rng(21 + group)
    q = r.normal(size=(len(lens) * hq, 128)).astype(np.float32)
    qs = r.integers(0, 2**63, (len(lens) * hq, 4), dtype=np.uint64)
    src = {}
    # (seq, head) -> plateaus (start, length, lambda); each straddles a segment
    # edge, so a tie group is cut by k across two segments.
    plateaus = {
        (2, 0): [(SEG - 30, 100, 100.0)],
        (3, 1): [(SEG - 10, 40, 100.0), (2 * SEG - 10, 100, 99.0)],
        (4, 0): [(5 * SEG - 20, 50, 100.0), (7 * SEG - 5, 30, 99.5)],
    }
    const_rows = {(1, 1), (2, 1), (4, 1)}  # every score ties: top-k = first k tokens
    for si, l in enumerate(lens):
        for h in range(n_kv):
            t = random_tiles(l, 1000 * si + h, [0])
            page_out_where(t, r.random(l) < 0.3)
            if (si, h) in const_rows:
                t[:] = t[0]
            for start, n, lam in plateaus.get((si, h), []):
                t[start:start + n] = plateau_tile(t[start], qs[si * hq + h * group], lam)
            src[(si, h)] = t
    arena, table, max_pages = build_paged(lens, n_kv, page_tiles, 7, src)
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
            assert np.array_equal(idx[si, qh], ti), (si, qh, idx[si, qh][:8], ti[:8])
            assert np.array_equal(val[si, qh].view(np.uint32), tv.view(np.uint32)), (si, qh)
            if (si, h) in const_rows:
                assert list(ti) == list(range(k))
            pl = plateaus.get((si, h), [])
            if pl and qh % group == 0:
                # the plateaus (clipped at the row end) hold the top scores,
                # highest lambda first; the top k cross a segment edge
                want = []
                for start, n, lam in sorted(pl, key=lambda p: -p[2]):
                    want += list(range(start, min(start + n, l)))
                m = min(k, len(want))
                assert list(ti[:m]) == want[:m], (si, qh)
                assert len({int(i) // SEG for i in ti[:m]}) > 1
        base += hq * l


def student_keys(rows, n_tok, n_kv, seed):
    """bf16 Student-t(4) keys z0 / sqrt(mean(z1..z4 ^ 2)), four distinct
    outlier channels per KV head scaled x20 before the bf16 rounding
    (BASELINE configs[2])."""
    r = np.random.default_rng(seed)
    chans = [r.permutation(128)[:4] for _ in range(n_kv)]
    out = np.empty((rows, n_tok, 128), np.float32)
    for row in range(rows):
        z0 = r.standard_normal((n_tok, 128), dtype=np.float32)
        chi = (r.standard_normal((4, n_tok, 128), dtype=np.float32) ** 2).mean(0)
        t = z0 / np.sqrt(chi)
        t[:, chans[row % n_kv]] *= np.float32(20.0)
        out[row] = o.bf16_round(t).reshape(n_tok, 128)
    return out


@pytest.mark.parametrize("codec", [2, 1])  # NF4, MX-INT4 (grouped INT4)
def test_c3_student_t_scoring(s, torch, codec):
    n_seq, n_kv, n_tok, group = 2, 8, 20000, 4
    rows, n_q = n_seq * n_kv, n_seq * n_kv * group
    keys = student_keys(rows, n_tok, n_kv, 0xC3 + codec)
    q = o.bf16_round(np.random.default_rng(5).standard_normal((n_q, 128), dtype=np.float32))
    with s.Model(seed=0x5EED0004) as m:
        z, _ = m.projection()
        td = s.gpu_encode(m, dev(torch, keys, torch.bfloat16), codec, n_kv_heads=n_kv)
        qc, qsd = s.gpu_prepare_queries(m, dev(torch, q, torch.bfloat16))
        fast = s.gpu_score(td, qc, qsd, group=group)
        exact, ham = s.gpu_score(td, qc, qsd, group=group, mode=s.SCORE_EXACT, hamming=True)
    tn = td.cpu().numpy()
    fast, exact, ham = fast.cpu().numpy(), exact.cpu().numpy(), ham.cpu().numpy()
    qsn = qsd.cpu().numpy().view(np.uint64)

    def enc(row):
        t = o.encode(keys[row], codec, 1, z, head=row % n_kv)
        return row, t

    with ThreadPoolExecutor(8) as ex:
        ref_tiles = dict(ex.map(enc, range(rows)))
    for row in range(rows):
        assert tn[row].tobytes() == ref_tiles[row].tobytes(), row
    # the outlier channels make the group scales differ across groups
    gs = ref_tiles[0]["group_scales"]
    assert (gs.min(1) < gs.max(1)).mean() > 0.5
    assert_tol(fast, exact)
    r = np.random.default_rng(9)
    for row in range(rows):
        idx = np.sort(r.choice(n_tok, 512, replace=False))
        for j in range(group):
            qi = row * group + j
            assert np.array_equal(qsn[qi], o.query_sign(q[qi], z))
            ref, href = o.score(ref_tiles[row][idx], q[qi], qsn[qi])
            assert np.array_equal(exact[qi, idx].view(np.uint32), ref.view(np.uint32)), (row, j)
            assert np.array_equal(ham[qi, idx].astype(np.uint32), href), (row, j)
