"""Learned (d > 128) models: the .slhw loader and the LearnedModel encode /
query / decode path (scirust/src/weights.rs, scirust/src/learned.rs:257-408).

CPU tests pin the loader's checks (mirroring weights.rs:351-540) and the
oracle's learned functions against closed forms and float64 arithmetic. GPU
tests compare the product through the C ABI with the oracle on identical
inputs: tiles, q_coarse / q_sign and reconstructions bit-exact (every sum
keeps the reference's sequential f32 order), scores within 1e-3 * (1 + |s|)
in fast mode and bit-identical in exact mode.
"""
import os
import struct

import numpy as np
import pytest

import oracle_ffi as o

DEV_CASES = [(192, False), (576, True), (1024, False), (1000, True), (333, False), (258, True)]


@pytest.fixture(scope="module")
def s():
    import slhav2_amd

    return slhav2_amd


def low_rank_keys(n, d, seed, rank=24):
    """Keys with a dominant low-rank part plus noise, and a matching P whose
    rows span most of it (so residuals are small but non-zero)."""
    r = np.random.default_rng(seed)
    basis, _ = np.linalg.qr(r.standard_normal((d, 128)))
    p = basis.T.astype(np.float32)  # [128, d], orthonormal rows
    coef = r.standard_normal((n, rank)) * np.linspace(3.0, 0.3, rank)
    keys = coef @ p[:rank] + 0.2 * r.standard_normal((n, d))
    return p, keys.astype(np.float32)


def write(tmp_path, name, data: bytes):
    f = tmp_path / name
    f.write_bytes(data)
    return f


# --------------------------------------------------------------------------
# Loader (CPU: slha_weights_load parses and registers without touching a GPU)

def test_fnv1a_published_vectors(s):
    # FNV-1a 32-bit test vectors (Fowler/Noll/Vo reference table)
    assert s._fnv1a(b"") == 0x811C9DC5
    assert s._fnv1a(b"a") == 0xE40C292C
    assert s._fnv1a(b"foobar") == 0xBF9CF968


@pytest.mark.parametrize("version", [1, 2])
@pytest.mark.parametrize("d,rht", [(129, False), (129, True), (300, True), (512, False)])
def test_slhw_roundtrip(s, tmp_path, version, d, rht):
    p = np.random.default_rng(d).standard_normal((128, d)).astype(np.float32)
    f = write(tmp_path, "m.slhw", s.slhw_bytes(p, 0xDEADBEEF12345678, rht, version=version))
    with s.Model.load(f) as m:  # legacy_version_one_remains_readable (weights.rs:421)
        assert m.dim == d
        assert m.pad_dim == (o.lib.orc_next_pow2(d) if rht else d)
        np.testing.assert_array_equal(m.latent_projection(), p)


def test_slhw_z_and_diag_from_seed(s, tmp_path):
    """Z [256][d_pad] from SplitMix64(seed), the diagonal from seed ^ 0xA2..A2
    (learned.rs:233-245, incoherence.rs:89-98), as the oracle generates them."""
    seed, d = 0x5EED, 300
    p = np.ones((128, d), np.float32)
    with s.Model.load(write(tmp_path, "m.slhw", s.slhw_bytes(p, seed, True))) as m:
        z, diag = m.projection()
        np.testing.assert_array_equal(z, o.projection(seed, 512))
        np.testing.assert_array_equal(diag, o.rht_diag(seed ^ 0xA2A2A2A2A2A2A2A2, 512))
    with s.Model.load(write(tmp_path, "n.slhw", s.slhw_bytes(p, seed, False))) as m:
        z, diag = m.projection()
        np.testing.assert_array_equal(z, o.projection(seed, d))
        assert (diag == 1.0).all()


def _hdr(version=2, d=130, seed=1, rht=0, pad=b"\0\0\0"):
    return struct.pack("<IIIQB", 0x534C4857, version, d, seed, rht) + pad


@pytest.mark.parametrize("case,fragment", [
    ("truncated", "weights: truncated header"),
    ("magic", "weights: bad magic (not an SLHW file)"),
    ("version", "weights: unsupported version 3 (supported: 1 and 2)"),
    ("dim", "weights: invalid dimension 128 (must be greater than D_C=128)"),
    ("rht", "weights: invalid RHT flag 2 (expected 0 or 1)"),
    ("reserved", "weights: non-zero reserved header bytes"),
    ("size", "weights: size mismatch (got 66589, expected 66588)"),
    ("payload", "weights: checksum mismatch"),
    ("header", "weights: checksum mismatch"),
    ("nonfinite", "weights: non-finite projection value at index 1000"),
])
def test_slhw_rejects(s, tmp_path, case, fragment):
    """weights.rs:388-540 (corruption, header coverage, invalid dimension,
    RHT flag and reserved bytes, non-finite values, malformed files)."""
    p = np.random.default_rng(1).standard_normal((128, 130)).astype(np.float32)
    good = bytearray(s.slhw_bytes(p, 1, False))
    if case == "truncated":
        data = bytes(good[:10])
    elif case == "magic":
        data = b"XXXX" + bytes(good[4:])
    elif case == "version":
        data = bytes(good[:4]) + struct.pack("<I", 3) + bytes(good[8:])
    elif case == "dim":
        data = _hdr(version=1, d=128) + bytes(128 * 128 * 4)
    elif case == "rht":
        data = _hdr(version=1, rht=2) + p.tobytes()
    elif case == "reserved":
        data = _hdr(version=1, pad=b"\0\1\0") + p.tobytes()
    elif case == "size":
        data = bytes(good) + b"\0"
    elif case == "payload":
        good[28 + 77] ^= 0x10
        data = bytes(good)
    elif case == "header":
        good[12] ^= 1  # seed byte: the checksum covers the header too
        data = bytes(good)
    else:
        q = p.copy()
        q.reshape(-1)[1000] = np.nan
        data = _hdr(version=1) + q.tobytes()
    f = write(tmp_path, "bad.slhw", data)
    with pytest.raises(s.SlhaError) as e:
        s.Model.load(f)
    assert e.value.code == s.ERR_IO
    assert fragment in str(e.value)


def test_slhw_rejects_paths(s, tmp_path):
    with pytest.raises(s.SlhaError, match="weights: cannot stat"):
        s.Model.load(tmp_path / "missing.slhw")
    with pytest.raises(s.SlhaError, match="is not a regular file"):
        s.Model.load(tmp_path)


def test_slhw_gpu_limit(s, tmp_path):
    d = 16385  # d_pad = d without RHT: one above the kernels' LDS limit
    p = np.zeros((128, d), np.float32)
    with pytest.raises(s.SlhaError, match="exceeds this build's GPU limit"):
        s.Model.load(write(tmp_path, "big.slhw", s.slhw_bytes(p, 1, False, version=1)))


# --------------------------------------------------------------------------
# Oracle pinning (closed forms and float64 references)

def test_oracle_learned_identity_projection():
    """P = [I | 0]: h = key[:128] exactly, the reconstruction is [h, 0], and the
    residual is e = [0, key[128:]]: its sign sketch, sigma (sequential f32
    sum of squares / d) and lambda follow from e alone."""
    d = 200
    p = np.zeros((128, d), np.float32)
    p[:, :128] = np.eye(128, dtype=np.float32)
    z = o.projection(7, d)
    m = o.Learned(p, z)
    key = np.random.default_rng(3).standard_normal(d).astype(np.float32)
    np.testing.assert_array_equal(m.latent(key), key[:128])
    rec = m.reconstruct(key[:128])
    np.testing.assert_array_equal(rec[:128], key[:128])
    assert (rec[128:] == 0).all()
    t = m.encode(key, 1, pos0=9)[0]  # grouped INT4
    e = np.concatenate([np.zeros(128, np.float32), key[128:]])
    np.testing.assert_array_equal(t["residual_bitmap"], o.sign_bits(z, e))
    acc = np.float32(0)
    for x in e:
        acc = np.float32(acc + np.float32(x * x))
    sigma = np.float32(np.sqrt(np.float32(acc / np.float32(d))))
    assert t["residual_sigma"] == sigma
    assert t["dynamic_lambda"] == np.float32(sigma * np.float32(o.lib.orc_analytic_lambda_c()))
    assert t["token_id"] == 9 and t["position"] == 9 and t["head_id"] == 0
    ref, _, gs = o.quantize(1, key[:128])
    np.testing.assert_array_equal(t["latent_kv"], ref)


@pytest.mark.parametrize("d,rht", [(300, False), (300, True)])
def test_oracle_learned_against_float64(d, rht):
    r = np.random.default_rng(d + rht)
    p = (r.standard_normal((128, d)) / np.sqrt(d)).astype(np.float32)
    d_pad = o.lib.orc_next_pow2(d) if rht else d
    z = o.projection(11, d_pad)
    diag = o.rht_diag(13, d_pad) if rht else None
    m = o.Learned(p, z, diag)
    q = r.standard_normal(d).astype(np.float32)
    qc, qs = m.query(q)
    np.testing.assert_allclose(qc, p.astype(np.float64) @ q, rtol=0, atol=1e-4)
    # sign bits: float64 Z @ (H D pad(q)) / sqrt(d_pad), checked where the
    # margin exceeds the f32 rounding of a length-d_pad sum
    v = np.zeros(d_pad)
    v[:d] = q
    if rht:
        n = d_pad
        hmat = np.array([[(-1) ** bin(i & j).count("1") for j in range(n)] for i in range(n)])
        v = hmat @ (diag * v) / np.sqrt(n)
    proj = z.astype(np.float64) @ v
    bits = np.array([(int(qs[s >> 6]) >> (s & 63)) & 1 for s in range(256)])
    sure = np.abs(proj) > 1e-3 * np.abs(z).sum(1) * np.abs(v).max()
    assert sure.sum() > 200
    np.testing.assert_array_equal(bits[sure], (proj[sure] < 0).astype(int))
    # reconstruction and the residual estimate of decode_key
    key = r.standard_normal(d).astype(np.float32)
    t = m.encode(key, 0)
    h = o.dequant(t)
    np.testing.assert_allclose(m.decode(t, False)[0], p.T.astype(np.float64) @ h, atol=1e-4)
    if not rht:
        sgn = np.array([-1.0 if (int(t["residual_bitmap"][0][s >> 6]) >> (s & 63)) & 1 else 1.0
                        for s in range(256)])
        est = p.T.astype(np.float64) @ h + float(t["residual_sigma"][0]) * np.sqrt(np.pi / 2) / 256 * (
            sgn @ z.astype(np.float64))
        np.testing.assert_allclose(m.decode(t, True)[0], est, atol=1e-4)
    else:  # RHT models return the coarse reconstruction only (learned.rs:294-298)
        np.testing.assert_array_equal(m.decode(t, True), m.decode(t, False))


# --------------------------------------------------------------------------
# GPU parity through the C ABI

@pytest.fixture(scope="module")
def torch(torch_cuda):
    return torch_cuda


def _model(s, tmp_path, d, rht, seed):
    p, keys = low_rank_keys(70, d, seed)
    f = tmp_path / f"m{d}{int(rht)}.slhw"
    s.save_weights(f, p, seed, rht)
    m = s.Model.load(f)
    z, diag = m.projection()
    return m, o.Learned(p, z, diag if rht else None), keys


def _tiles(t):
    return t.cpu().numpy().reshape(-1, 128).copy().view(o.TILE_DTYPE).reshape(-1)


@pytest.mark.gpu
@pytest.mark.parametrize("d,rht", DEV_CASES)
def test_gpu_learned_encode_bit_exact(s, torch, tmp_path, d, rht):
    m, ref, keys = _model(s, tmp_path, d, rht, 100 + d)
    try:
        for codec in range(6):
            print(f"learned encode d={d} rht={rht} codec={codec}", flush=True)
            got = _tiles(s.gpu_encode(m, torch.from_numpy(keys).cuda(), codec, pos0=5))
            want = ref.encode(keys, codec, pos0=5)
            assert got.tobytes() == want.tobytes(), f"codec {codec}"
            host = s.encode_key(m, keys[3], 8, codec)
            assert host.tobytes() == want[3].tobytes()
        # bf16 keys widen exactly before both paths see them
        kb = torch.from_numpy(keys).cuda().to(torch.bfloat16)
        got = _tiles(s.gpu_encode(m, kb.reshape(2, 35, d), 1, n_kv_heads=2))
        want = ref.encode(kb.float().cpu().numpy(), 1)
        want["position"] = want["token_id"] = np.tile(np.arange(35, dtype=np.uint32), 2)
        want["head_id"] = np.repeat(np.arange(2, dtype=np.uint16), 35)
        assert got.tobytes() == want.tobytes()
    finally:
        m.release()


@pytest.mark.gpu
@pytest.mark.parametrize("d,rht", DEV_CASES)
def test_gpu_learned_query_and_decode_bit_exact(s, torch, tmp_path, d, rht):
    m, ref, keys = _model(s, tmp_path, d, rht, 200 + d)
    try:
        print(f"learned query/decode d={d} rht={rht}", flush=True)
        q = np.random.default_rng(d).standard_normal((9, d)).astype(np.float32)
        qc, qs = s.gpu_prepare_queries(m, torch.from_numpy(q).cuda())
        qc, qs = qc.cpu().numpy(), qs.cpu().numpy().view(np.uint64)
        for i in range(len(q)):
            wc, ws = ref.query(q[i])
            np.testing.assert_array_equal(qc[i], wc)
            np.testing.assert_array_equal(qs[i], ws)
        hc, hs = s.prepare_query(m, q[0])
        np.testing.assert_array_equal(hc, qc[0])
        np.testing.assert_array_equal(hs, qs[0])
        for codec in (0, 2, 4, 5):
            tiles = ref.encode(keys[:24], codec)
            td = torch.from_numpy(tiles.view(np.uint8).reshape(-1, 128)).cuda()
            for res in (False, True):
                got = s.gpu_decode(m, td, with_residual=res).cpu().numpy()
                np.testing.assert_array_equal(got, ref.decode(tiles, res))
            np.testing.assert_array_equal(s.decode_latent(m, tiles[1]), ref.decode(tiles[1:2], False)[0])
            np.testing.assert_array_equal(s.decode_key(m, tiles[2]), ref.decode(tiles[2:3], True)[0])
            # scores of learned tiles: exact mode bit-identical, fast within 1e-3
            ex = s.gpu_score(td, torch.from_numpy(qc[:1]).cuda(),
                             torch.from_numpy(qs[:1].view(np.int64)).cuda(), mode=s.SCORE_EXACT)
            want, _ = o.score(tiles, qc[0], qs[0])
            np.testing.assert_array_equal(ex.cpu().numpy()[0], want)
            fa = s.score_tiles(m, tiles, qc[0], qs[0])
            assert (np.abs(fa - want) <= 1e-3 * (1 + np.abs(want))).all()
    finally:
        m.release()
