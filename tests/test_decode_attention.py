"""Decode attention over compressed keys (scirust/examples/benchmark_decode.rs:
29-90): softmax(scores * scale) . V with the eq. 2.3 scores of the tiles.

CPU tests pin the oracle's softmax_into (metrics.rs:338-409) with the
reference's own cases (metrics.rs:330-337 doc test, :440-540) and with float64
closed forms, and aggregate_v with a float64 product. GPU tests compare
slha_gpu_decode_attention through the C ABI with the oracle:
  * against the oracle run on the GPU's own fast-mode scores (isolates the
    softmax . V kernels): |gpu - ref| <= 2e-5 * max|V|;
  * against the oracle run end to end on exact scores: the fast scores are
    within 1e-3 * (1 + |s|) of the exact ones (tests.rs:923), which moves the
    output by at most about scale * max|ds| * max|V|; measured differences
    are far below the 2e-4 * max|V| used here.
"""
import numpy as np
import pytest

import oracle_ffi as o

SCALE = np.float32(1.0 / np.sqrt(128.0))  # benchmark_decode.rs:51


# --------------------------------------------------------------------------
# Oracle pinning (CPU)

def test_softmax_reference_cases():
    w = o.softmax([0.0, 0.0, 0.0], 1.0)                       # metrics.rs:332-336
    assert abs(float(w.sum()) - 1.0) < 1e-6 and abs(w[0] - 1 / 3) < 1e-6
    assert o.softmax([np.float32(-np.inf)] * 4, 1.0).tolist() == [0.0] * 4   # :447-449
    assert o.softmax([0.0, np.nan], 1.0).tolist() == [0.0, 0.0]             # :485-486
    assert o.softmax([0.0, 1.0], np.inf).tolist() == [0.0, 0.0]             # :488-489
    inf = np.float32(np.inf)
    assert o.softmax([1.0, inf, inf, -inf], 1.0).tolist() == [0.0, 0.5, 0.5, 0.0]  # :519-523
    w = o.softmax([0.0, -inf, 1.0, -inf], 1.0)                # :526-534
    assert w[0] > 0 and w[1] == 0 and w[2] > w[0] and w[3] == 0
    assert abs(float(w.sum()) - 1.0) < 1e-6
    w = o.softmax([1.0, 2.0, 3.0, 4.0], 0.0)                  # :537-538
    assert np.all(np.abs(w - 0.25) < 1e-6)


def test_softmax_and_aggregate_against_float64():
    r = np.random.default_rng(1)
    for n in (1, 7, 513, 4000):
        sc = (r.standard_normal(n) * 20).astype(np.float32)
        lg = sc.astype(np.float64) * np.float64(SCALE)
        ref = np.exp(lg - lg.max())
        ref /= ref.sum()
        w = o.softmax(sc, float(SCALE))
        np.testing.assert_allclose(w, ref, rtol=2e-6, atol=1e-12)
        v = r.standard_normal((n, 64)).astype(np.float32)
        np.testing.assert_allclose(o.aggregate(w, v), w.astype(np.float64) @ v, atol=1e-5)


# --------------------------------------------------------------------------
# GPU parity through the C ABI

@pytest.fixture(scope="module")
def s(torch_cuda):
    import slhav2_amd

    return slhav2_amd


@pytest.fixture(scope="module")
def torch(torch_cuda):
    return torch_cuda


def _setup(s, torch, n_rows, n_tok, group, seed, codec=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    m = s.Model(seed=seed, rht=False)
    keys = torch.randn((n_rows, n_tok, 128), device="cuda", generator=g).to(torch.bfloat16)
    tiles = s.gpu_encode(m, keys, codec, n_kv_heads=n_rows)
    q = torch.randn((n_rows * group, 128), device="cuda", generator=g).to(torch.bfloat16)
    qc, qs = s.gpu_prepare_queries(m, q)
    m.release()
    return tiles, qc, qs


@pytest.mark.gpu
@pytest.mark.parametrize("n_rows,n_tok,group,d_v,vdt", [
    (2, 3000, 4, 128, "f32"),
    (2, 3000, 4, 128, "bf16"),
    (1, 512, 1, 128, "f32"),
    (3, 1025, 3, 64, "bf16"),
    (2, 300, 8, 32, "f32"),
    (1, 700, 16, 256, "f32"),
    (1, 5, 2, 128, "f32"),
    (2, 2000, 8, 128, "bf16"),
    (1, 777, 6, 64, "f32"),
    (1, 300, 16, 128, "bf16"),
    # more than 16 x 8 = 128 segments of 256 tokens: the combine's loops past
    # its first 128 segments, and a partial last segment
    (1, 65537, 4, 128, "bf16"),
    (2, 65537, 8, 64, "f32"),
    (1, 40000, 16, 64, "bf16"),
])
def test_gpu_decode_attention(s, torch, n_rows, n_tok, group, d_v, vdt):
    print(f"decode attention rows={n_rows} tok={n_tok} group={group} d_v={d_v} {vdt}", flush=True)
    tiles, qc, qs = _setup(s, torch, n_rows, n_tok, group, 1000 + n_tok)
    g = torch.Generator(device="cuda").manual_seed(n_tok)
    vals = torch.randn((n_rows, n_tok, d_v), device="cuda", generator=g)
    if vdt == "bf16":
        vals = vals.to(torch.bfloat16)
    out = s.gpu_decode_attention(tiles, vals, qc, qs, group=group, scale=float(SCALE)).cpu().numpy()
    fast = s.gpu_score(tiles, qc, qs, group=group).cpu().numpy()
    t_np = tiles.cpu().numpy().reshape(n_rows, n_tok, 128).copy().view(o.TILE_DTYPE)
    v_np = vals.float().cpu().numpy()
    qc_np, qs_np = qc.cpu().numpy(), qs.cpu().numpy().view(np.uint64)
    vmax = float(np.abs(v_np).max())
    for qh in range(n_rows * group):
        r = qh // group
        on_fast = o.aggregate(o.softmax(fast[qh], float(SCALE)), v_np[r])
        assert np.abs(out[qh] - on_fast).max() <= 2e-5 * vmax, qh
        exact = o.decode_attention(t_np[r].reshape(-1), v_np[r], qc_np[qh], qs_np[qh], float(SCALE))
        assert np.abs(out[qh] - exact).max() <= 2e-4 * vmax, qh


def test_decode_attention_argument_checks():
    """Bad arguments are rejected before any device work (no GPU needed)."""
    import slhav2_amd as sa

    f = sa.lib.slha_gpu_decode_attention
    assert f(None, None, 0, 1, 64, 100, None, None, 2, 1.0, None, None) == sa.ERR_DIMENSION
    assert "d_v" in sa.last_error()
    assert f(None, None, 0, 1, 64, 128, None, None, 17, 1.0, None, None) == sa.ERR_DIMENSION
    assert "group" in sa.last_error()
    assert f(None, None, 7, 1, 64, 128, None, None, 2, 1.0, None, None) == sa.ERR_DIMENSION
    assert f(None, None, 0, 1, 64, 128, None, None, 2, 1.0, None, None) == sa.ERR_NULL


@pytest.mark.gpu
def test_gpu_decode_attention_degenerate(s, torch):
    """softmax_into's contract: a non-finite scale or no token gives zero
    weights, hence a zero output."""
    tiles, qc, qs = _setup(s, torch, 1, 64, 2, 7)
    vals = torch.ones((1, 64, 128), device="cuda")
    for sc in (float("inf"), float("nan")):
        out = s.gpu_decode_attention(tiles, vals, qc, qs, group=2, scale=sc)
        assert (out == 0).all()
    empty = torch.empty((1, 0, 128), dtype=torch.uint8, device="cuda")
    out = s.gpu_decode_attention(empty, torch.empty((1, 0, 128), device="cuda"), qc, qs, group=2)
    assert (out == 0).all()


@pytest.mark.gpu
@pytest.mark.parametrize("group,d_v", [(4, 128), (8, 64), (16, 64)])
@pytest.mark.parametrize("scale", [1e38, -1e38, 3e30, -0.5])
def test_gpu_decode_attention_extreme_scale(s, torch, group, d_v, scale):
    """softmax_into forms logits in f64 (metrics.rs:351-358), so a huge finite
    scale still gives finite logits: the weights go one-hot to the top score
    (the lowest for a negative scale), shared equally between tied tokens."""
    print(f"decode attention scale={scale} group={group} d_v={d_v}", flush=True)
    n_rows, n_tok = 2, 1500
    tiles, qc, qs = _setup(s, torch, n_rows, n_tok, group, 77)
    # ties: tokens 1000.. repeat token 0's tile, so the extreme score may be shared
    tiles[:, 1000:1100] = tiles[:, :1].clone()
    g = torch.Generator(device="cuda").manual_seed(3)
    vals = torch.randn((n_rows, n_tok, d_v), device="cuda", generator=g)
    out = s.gpu_decode_attention(tiles, vals, qc, qs, group=group, scale=scale).cpu().numpy()
    fast = s.gpu_score(tiles, qc, qs, group=group).cpu().numpy()
    v_np = vals.cpu().numpy()
    vmax = float(np.abs(v_np).max())
    assert np.isfinite(out).all()
    for qh in range(n_rows * group):
        w = o.softmax(fast[qh], scale)
        assert abs(float(w.sum()) - 1.0) < 1e-5
        ref = o.aggregate(w, v_np[qh // group])
        assert np.abs(out[qh] - ref).max() <= 2e-5 * vmax, qh
