"""slha_gpu_score_paged_topk_noalloc against slha_gpu_score_paged_topk, both
through the C ABI on the same device inputs: scores, top-k indices and top-k
values bit-identical.

Two calls in a row on one GPU share the static scratch array, so the second,
smaller call runs over the first call's leftover candidate lists:
  1. one sequence, group 256, k = 256, 524 288 tokens: 256 query rows x 32
     segments x 256 candidates x 8 B = 16 MiB, exactly the array's size;
  2. four ragged sequences at group 4, k = 64, with score plateaus that
     straddle the 16 384-score segment edges.
A call needing more than the array is rejected before any device work and
leaves its outputs untouched.
"""
import numpy as np
import pytest

import oracle_ffi as o
from test_gpu_parity import build_paged, dev, random_tiles

pytestmark = pytest.mark.gpu

SEG = 16384


@pytest.fixture(scope="module")
def s(torch_cuda):
    import slhav2_amd

    return slhav2_amd


@pytest.fixture(scope="module")
def torch(torch_cuda):
    return torch_cuda


def paged_inputs(torch, lens, n_kv, group, page_tiles, seed, plateau=False):
    r = np.random.default_rng(seed)
    hq = n_kv * group
    q = r.normal(size=(len(lens) * hq, 128)).astype(np.float32)
    qs = r.integers(0, 2**63, (len(lens) * hq, 4), dtype=np.uint64)
    src = {}
    for si, l in enumerate(lens):
        for h in range(n_kv):
            t = random_tiles(l, seed * 100 + 10 * si + h, [0, 2])
            if plateau and l > SEG:  # ties across the first segment edge
                t[SEG - 20:SEG + 20] = t[SEG - 20]
            src[(si, h)] = t
    arena, table, max_pages = build_paged(lens, n_kv, page_tiles, seed, src)
    return (dev(torch, arena.view(np.uint8).reshape(-1, 128)), dev(torch, table), max_pages,
            dev(torch, np.asarray(lens, np.int32)), dev(torch, q), dev(torch, qs.view(np.int64)))


def both(s, torch, lens, n_kv, group, k, page_tiles, seed, plateau=False):
    arena, table, max_pages, seq_len, q, qs = paged_inputs(torch, lens, n_kv, group, page_tiles, seed,
                                                           plateau)
    print(f"noalloc paged top-k lens={lens[:4]} group={group} k={k}", flush=True)
    na = s.gpu_score_paged_topk(arena, page_tiles, table, max_pages, seq_len, n_kv, group, q, qs, k,
                                noalloc=True)
    torch.cuda.synchronize()
    ref = s.gpu_score_paged_topk(arena, page_tiles, table, max_pages, seq_len, n_kv, group, q, qs, k)
    torch.cuda.synchronize()
    for a, b in zip(na, ref):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    return na


def test_noalloc_paged_topk_matches_the_allocating_entry_point(s, torch):
    # 1: the whole 16 MiB array (n_seq * n_kv * group * ceil(len / 16384) * k * 8)
    n_tok, group, k = 32 * SEG, 256, 256
    assert 1 * 1 * group * (n_tok // SEG) * k * 8 == 16 << 20
    scores, idx, val = both(s, torch, [n_tok], 1, group, k, 4096, 41)
    sc = scores.cpu().numpy()
    for qh in (0, 255):  # indices against the oracle's top-k on the same scores
        ti, tv = o.topk(sc[qh * n_tok:(qh + 1) * n_tok], k)
        assert np.array_equal(idx[0, qh].cpu().numpy().view(np.uint32), ti)
        assert np.array_equal(val[0, qh].cpu().numpy().view(np.uint32), tv.view(np.uint32))
    # 2: a smaller call over the leftover lists of call 1
    lens = [40000, 1000, 70001, 16385]
    scores, idx, val = both(s, torch, lens, 2, 4, 64, 4096, 42, plateau=True)
    sc, ix = scores.cpu().numpy(), idx.cpu().numpy().view(np.uint32)
    base = 0
    for si, l in enumerate(lens):
        for qh in range(8):
            ti, _ = o.topk(sc[base + qh * l: base + (qh + 1) * l], 64)
            assert np.array_equal(ix[si, qh], ti), (si, qh)
        base += 8 * l


def test_noalloc_rejects_more_than_its_scratch(s, torch):
    # group 256, 8 KV heads, 32 segments, k = 64: 2048 * 32 * 64 * 8 B = 32 MiB
    seq_len = dev(torch, np.array([32 * SEG], np.int32))
    base = torch.zeros(1, dtype=torch.int64, device="cuda")
    dummy = torch.zeros(16, dtype=torch.int64, device="cuda")
    idx = torch.full((2048 * 64,), 7, dtype=torch.int32, device="cuda")
    val = torch.full((2048 * 64,), 7.0, device="cuda")
    f = s.lib.slha_gpu_score_paged_topk_noalloc
    rc = f(dummy.data_ptr(), 4096, dummy.data_ptr(), 128, seq_len.data_ptr(), base.data_ptr(), 1,
           32 * SEG, 8, 256, dummy.data_ptr(), dummy.data_ptr(), dummy.data_ptr(), 64, idx.data_ptr(),
           val.data_ptr(), None)
    assert rc == s.ERR_DIMENSION and "no-allocation" in s.last_error()
    torch.cuda.synchronize()
    assert (idx == 7).all() and (val == 7.0).all()
