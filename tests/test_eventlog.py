"""EventLog for COLD eviction and rehydrate (scirust/src/eventlog.rs,
ccos.rs:404-466).

CPU tests pin the oracle's record bytes (FNV-1a published vectors, the tile
serialisation against the tile byte map, single-byte sensitivity of the
checksum) and run the library's file side through the C ABI with the cases of
the reference's own tests (eventlog.rs:520-830, same sample tiles). GPU tests
compare slha_gpu_eventlog_pack with the oracle's records byte for byte and
check slha_gpu_eventlog_unpack's checked scatter, then run evict -> log ->
reopen -> rehydrate end to end.
"""
import struct

import numpy as np
import pytest

import oracle_ffi as o

FLAG_TQ3 = 0x08
HEADER, RECORD = 16, 144


def sample_tile(seed: int) -> np.ndarray:
    """eventlog.rs:497-514."""
    t = np.zeros(1, o.TILE_DTYPE)
    t["latent_kv"][0] = [(i * seed + 3) & 0xFF for i in range(64)]
    t["residual_bitmap"][0] = [0x0123456789ABCDEF ^ seed, 1, 2, 3]
    t["scale"] = np.float32(0.5) * np.float32(seed) + np.float32(0.125)
    t["dynamic_lambda"] = np.float32(0.37)
    t["residual_sigma"] = np.float32(1.5)
    t["token_id"] = 42 + seed
    t["position"] = 7 + seed
    t["head_id"] = 2
    t["flags"] = FLAG_TQ3
    t["group_scales"][0] = [seed, 254, 3, 4, 5, 6, 7, 8]
    return t


def rec(seq: int, slot: int, tile, version: int = 2) -> np.ndarray:
    return o.eventlog_records(tile, [0], [seq], version)[0:1].copy().view(np.uint8).reshape(-1)


def recs(*items, version: int = 2) -> np.ndarray:
    """items: (seq, slot, tile); the slot is the record's slot field."""
    out = []
    for seq, slot, tile in items:
        r = rec(seq, 0, tile, version)
        r[8:12] = np.frombuffer(struct.pack("<I", slot), np.uint8)
        ck = o.lib.orc_record_checksum(seq, slot, o._p(np.ascontiguousarray(r[16:]))) if version == 2 else 0
        r[12:16] = np.frombuffer(struct.pack("<I", ck), np.uint8)
        out.append(r)
    return np.concatenate(out)


@pytest.fixture(scope="module")
def sa():
    import slhav2_amd

    return slhav2_amd


# --------------------------------------------------------------------------
# Oracle pinning


def test_fnv1a_published_vectors():
    # FNV-1a 32-bit test vectors of the FNV reference suite.
    assert o.fnv1a(b"") == 0x811C9DC5
    assert o.fnv1a(b"a") == 0xE40C292C
    assert o.fnv1a(b"foobar") == 0xBF9CF968


def test_tile_bytes_follow_the_byte_map():
    """tile_to_bytes writes the fields at the tile's byte map offsets
    (tile.rs:52-77), so a tile's memory is its serialisation."""
    for s in range(16):  # eventlog.rs:520-531
        t = sample_tile(s)
        b = o.tile_to_bytes(t)
        assert b == t.tobytes()
        assert b[96:100] == struct.pack("<f", float(t["scale"][0]))
        assert b[118:120] == struct.pack("<H", FLAG_TQ3)
        assert b[64:72] == struct.pack("<Q", 0x0123456789ABCDEF ^ s)
    r = np.random.default_rng(3)
    raw = r.integers(0, 256, (64, 128), dtype=np.uint8)
    tiles = raw.copy().view(o.TILE_DTYPE).reshape(-1)
    for i in range(64):
        assert o.tile_to_bytes(tiles[i:i + 1]) == raw[i].tobytes()


def test_record_layout_and_checksum_coverage():
    t = sample_tile(9)
    r = rec(7, 0, t)
    assert struct.unpack("<QII", r[:16].tobytes())[:2] == (7, 0)
    assert r[16:].tobytes() == t.tobytes()
    # All-zero record: FNV-1a of 140 zero bytes.
    z = np.zeros(1, o.TILE_DTYPE)
    assert struct.unpack("<I", rec(0, 0, z)[12:16].tobytes())[0] == o.fnv1a(bytes(140))
    # Every byte of seq, slot and tile is covered (an FNV-1a step is a
    # bijection of the state, so one changed byte always changes the hash);
    # the checksum field is not.
    base = rec(0x1122334455667788, 0, t)
    ck0 = struct.unpack("<I", base[12:16].tobytes())[0]
    for pos in list(range(12)) + list(range(16, 144)):
        m = base.copy()
        m[pos] ^= 0x5A
        ck = o.lib.orc_record_checksum(struct.unpack("<Q", m[:8].tobytes())[0],
                                       struct.unpack("<I", m[8:12].tobytes())[0],
                                       o._p(np.ascontiguousarray(m[16:])))
        assert ck != ck0, pos
    # Version 1 stores zero.
    assert rec(7, 0, t, version=1)[12:16].tobytes() == bytes(4)


# --------------------------------------------------------------------------
# Host file side through the C ABI (eventlog.rs:539-830)


def test_append_read_reopen_round_trip(sa, tmp_path):
    p = tmp_path / "rw.sllg"
    with sa.EventLog.create(p) as log:
        log.append(recs(*[(s * 10, s, sample_tile(s)) for s in range(5)]))
        assert len(log) == 5
        log.sync()
    with sa.EventLog.open(p) as log:
        assert len(log) == 5 and log.version == 2
        rs = log.read_all()
        for s, r in enumerate(rs):
            assert r["seq"] == s * 10 and r["slot"] == s
            assert r["tile"].tobytes() == sample_tile(s).tobytes()


def test_identical_runs_are_byte_identical(sa, tmp_path):
    files = []
    for name in ("det1", "det2"):
        p = tmp_path / name
        with sa.EventLog.create(p) as log:
            for s in range(7):
                log.append(recs((s, s * 2, sample_tile(s))))
            log.sync()
        files.append(p.read_bytes())
    assert files[0] == files[1]
    assert len(files[0]) == HEADER + 7 * RECORD
    assert files[0][:16] == struct.pack("<IIII", 0x534C4C47, 2, 128, 0)
    assert files[0][16:] == recs(*[(s, s * 2, sample_tile(s)) for s in range(7)]).tobytes()


def test_fetch_helpers_find_latest(sa, tmp_path):
    with sa.EventLog.create(tmp_path / "fetch") as log:
        log.append(recs((100, 0, sample_tile(1))))
        log.append(recs((100, 0, sample_tile(2))))
        log.append(recs((200, 1, sample_tile(3))))
        assert log.fetch_by_seq(100)["tile"].tobytes() == sample_tile(2).tobytes()
        assert log.fetch_last_for_slot(0)["tile"].tobytes() == sample_tile(2).tobytes()
        assert log.fetch_last_for_slot(1)["seq"] == 200
        assert log.fetch_by_seq(999) is None


def test_append_durable_round_trips_after_reopen(sa, tmp_path):
    p = tmp_path / "durable"
    with sa.EventLog.create(p) as log:
        log.append_durable(recs((77, 4, sample_tile(7))))
        assert len(log) == 1
    with sa.EventLog.open(p) as log:
        r = log.read_all()
        assert len(r) == 1 and r[0]["seq"] == 77 and r[0]["slot"] == 4
        assert r[0]["tile"].tobytes() == sample_tile(7).tobytes()


def test_read_only_log_allows_reads_but_rejects_appends(sa, tmp_path):
    p = tmp_path / "ro"
    with sa.EventLog.create(p) as log:
        log.append_durable(recs((1, 2, sample_tile(3))))
    with sa.EventLog.open_read_only(p) as log:
        assert len(log.read_all()) == 1
        with pytest.raises(sa.SlhaError) as e:
            log.append(recs((2, 3, sample_tile(4))))
        assert e.value.code == sa.ERR_IO and "read-only" in e.value.message
        assert len(log) == 1


def test_create_new_refuses_to_overwrite_existing_log(sa, tmp_path):
    p = tmp_path / "new"
    sa.EventLog.create_new(p).close()
    with pytest.raises(sa.SlhaError) as e:
        sa.EventLog.create_new(p)
    assert "exists" in e.value.message
    assert p.stat().st_size == HEADER


def test_version_two_detects_record_corruption(sa, tmp_path):
    p = tmp_path / "ck"
    with sa.EventLog.create(p) as log:
        log.append(recs((7, 3, sample_tile(9))))
    b = bytearray(p.read_bytes())
    b[HEADER + 16 + 5] ^= 0x80
    p.write_bytes(bytes(b))
    with pytest.raises(sa.SlhaError) as e:
        sa.EventLog.open(p)
    assert "checksum" in e.value.message


def test_open_recover_discards_only_the_partial_tail(sa, tmp_path):
    p = tmp_path / "recover"
    with sa.EventLog.create(p) as log:
        log.append(recs((10, 1, sample_tile(1)), (20, 2, sample_tile(2))))
    p.write_bytes(p.read_bytes()[:-17])
    with pytest.raises(sa.SlhaError) as e:
        sa.EventLog.open(p)
    assert "truncated record" in e.value.message
    with sa.EventLog.open_recover(p) as log:
        assert len(log) == 1
        r = log.read_all()
        assert r[0]["seq"] == 10 and r[0]["tile"].tobytes() == sample_tile(1).tobytes()
        log.append(recs((30, 3, sample_tile(3))))
    with sa.EventLog.open(p) as log:
        assert [int(x) for x in log.read_all()["seq"]] == [10, 30]
    assert p.stat().st_size == HEADER + 2 * RECORD


def test_legacy_version_one_remains_readable_and_appendable(sa, tmp_path):
    p = tmp_path / "v1"
    with sa.EventLog.create(p) as log:
        log.append(recs((1, 4, sample_tile(4))))
    b = bytearray(p.read_bytes())
    b[4:8] = struct.pack("<I", 1)
    b[HEADER + 12:HEADER + 16] = bytes(4)
    p.write_bytes(bytes(b))
    with sa.EventLog.open(p) as log:
        assert log.version == 1 and len(log) == 1
        assert log.read_all()[0]["tile"].tobytes() == sample_tile(4).tobytes()
        # A version-1 log takes version-1 records (checksum 0) only.
        with pytest.raises(sa.SlhaError) as e:
            log.append(recs((2, 5, sample_tile(5))))
        assert e.value.code == sa.ERR_INVALID_TILE
        log.append(recs((2, 5, sample_tile(5)), version=1))
    with sa.EventLog.open(p) as log:
        assert len(log) == 2 and len(log.read_all()) == 2


def test_rejects_bad_header_and_truncation(sa, tmp_path):
    p = tmp_path / "bad"
    p.write_bytes(bytes(HEADER))
    with pytest.raises(sa.SlhaError, match="bad magic"):
        sa.EventLog.open(p)
    p.write_bytes(struct.pack("<IIII", 0x534C4C47, 3, 128, 0))
    with pytest.raises(sa.SlhaError, match="unsupported version"):
        sa.EventLog.open(p)
    p.write_bytes(struct.pack("<IIII", 0x534C4C47, 2, 64, 0))
    with pytest.raises(sa.SlhaError, match="tile-size mismatch"):
        sa.EventLog.open(p)
    p.write_bytes(bytes(10))
    with pytest.raises(sa.SlhaError, match="shorter than header"):
        sa.EventLog.open(p)
    p2 = tmp_path / "trunc"
    with sa.EventLog.create(p2) as log:
        log.append(recs((1, 0, sample_tile(1))))
    p2.write_bytes(p2.read_bytes()[:-10])
    with pytest.raises(sa.SlhaError, match="truncated record"):
        sa.EventLog.open(p2)


def test_append_rejects_a_bad_checksum_and_writes_nothing(sa, tmp_path):
    p = tmp_path / "badck"
    with sa.EventLog.create(p) as log:
        good = recs((1, 1, sample_tile(1)), (2, 2, sample_tile(2)))
        bad = good.copy()
        bad[RECORD + 40] ^= 1  # tile byte of the second record
        with pytest.raises(sa.SlhaError) as e:
            log.append(bad)
        assert e.value.code == sa.ERR_INVALID_TILE and "record 1" in e.value.message
        assert len(log) == 0
        log.append(good)
        assert len(log) == 2
    assert p.stat().st_size == HEADER + 2 * RECORD


def test_read_range_and_handles(sa, tmp_path):
    with sa.EventLog.create(tmp_path / "rng") as log:
        log.append(recs(*[(s, s, sample_tile(s)) for s in range(4)]))
        assert [int(x) for x in log.read(1, 2)["seq"]] == [1, 2]
        with pytest.raises(sa.SlhaError) as e:
            log.read(3, 2)
        assert e.value.code == sa.ERR_DIMENSION
        h = log._h
    # closed handle
    assert sa.lib.slha_eventlog_close(h) == sa.ERR_INVALID_HANDLE
    assert sa.lib.slha_eventlog_append(None, None, 0, 0) == sa.ERR_NULL
    assert sa.lib.slha_eventlog_open(None, 0) is None
    assert sa.lib.slha_eventlog_open(str(tmp_path / "missing").encode(), 0) is None
    assert "EventLog: open" in sa.last_error()


def test_device_entry_points_check_arguments(sa):
    """Argument errors come back before any device work (no GPU needed)."""
    f = sa.lib.slha_gpu_eventlog_pack
    assert f(None, None, None, 4, 3, None, None) == sa.ERR_DIMENSION
    assert f(None, None, None, 0, 2, None, None) == sa.OK
    assert f(None, None, None, 4, 2, None, None) == sa.ERR_NULL
    g = sa.lib.slha_gpu_eventlog_unpack
    assert g(None, 4, 0, None, None, None, None) == sa.ERR_DIMENSION
    assert g(None, 4, 2, None, None, None, None) == sa.ERR_NULL


# --------------------------------------------------------------------------
# GPU: pack / unpack through the C ABI


@pytest.fixture(scope="module")
def torch(torch_cuda):
    return torch_cuda


def _arena(torch, n_slots: int, seed: int):
    g = np.random.default_rng(seed)
    raw = g.integers(0, 256, (n_slots, 128), dtype=np.uint8)
    return raw, torch.from_numpy(raw.copy()).cuda()


@pytest.mark.gpu
@pytest.mark.parametrize("n", [1, 255, 256, 257, 5000])
@pytest.mark.parametrize("version", [1, 2])
def test_gpu_pack_matches_oracle(sa, torch, n, version):
    print(f"eventlog pack n={n} v{version}", flush=True)
    raw, arena = _arena(torch, 6000, n)
    g = np.random.default_rng(n + 7)
    slots = g.permutation(6000)[:n].astype(np.int32)
    seqs = g.integers(0, 2**63, n, dtype=np.int64)
    got = sa.gpu_eventlog_pack(arena, torch.from_numpy(slots).cuda(), torch.from_numpy(seqs).cuda(),
                               version).cpu().numpy()
    ref = o.eventlog_records(raw.view(o.TILE_DTYPE).reshape(-1), slots, seqs.view(np.uint64), version)
    assert got.tobytes() == ref.tobytes()


@pytest.mark.gpu
def test_gpu_unpack_scatters_checked_records(sa, torch):
    print("eventlog unpack", flush=True)
    raw, arena = _arena(torch, 3000, 11)
    g = np.random.default_rng(12)
    n = 1000
    src = g.permutation(3000)[:n].astype(np.int32)
    seqs = g.integers(0, 2**40, n, dtype=np.int64)
    rec_t = sa.gpu_eventlog_pack(arena, torch.from_numpy(src).cuda(), torch.from_numpy(seqs).cuda())
    rec_np = rec_t.cpu().numpy()
    bad = np.sort(g.choice(n, 37, replace=False))
    for k, i in enumerate(bad):  # one flipped byte in seq, slot, checksum or tile
        pos = [0, 9, 13, 16, 100, 143][k % 6]
        rec_np[i, pos] ^= 0x10
    dst = g.permutation(3000)[:n].astype(np.int32)
    target = torch.zeros((3000, 128), dtype=torch.uint8, device="cuda")
    status = sa.gpu_eventlog_unpack(torch.from_numpy(rec_np).cuda(), torch.from_numpy(dst).cuda(),
                                    target).cpu().numpy()
    expect_bad = np.zeros(n, bool)
    expect_bad[bad] = True
    assert (status == expect_bad.astype(np.int32)).all()
    out = target.cpu().numpy()
    for i in range(n):
        want = bytes(128) if expect_bad[i] else raw[src[i]].tobytes()
        assert out[dst[i]].tobytes() == want, i
    untouched = np.setdiff1d(np.arange(3000), dst)
    assert not out[untouched].any()
    # Version 1 does not check: every record lands.
    target.zero_()
    st1 = sa.gpu_eventlog_unpack(torch.from_numpy(rec_np).cuda(), torch.from_numpy(dst).cuda(), target,
                                 version=1).cpu().numpy()
    assert not st1.any()
    assert target.cpu().numpy()[dst].tobytes() == rec_np[:, 16:].tobytes()


@pytest.mark.gpu
def test_gpu_evict_log_rehydrate_end_to_end(sa, torch, tmp_path):
    """ElasticKvCache::evict then rehydrate (ccos.rs:404-466) over real
    encoded tiles: pack -> D2H -> append -> reopen -> fetch -> H2D -> unpack."""
    print("eventlog end to end", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(5)
    m = sa.Model(seed=5, rht=True)
    keys = torch.randn((1, 512, 128), device="cuda", generator=gen).to(torch.bfloat16)
    arena = sa.gpu_encode(m, keys, sa.CODEC_TQ3, n_kv_heads=1).reshape(512, 128)
    m.release()
    evict = torch.tensor([3, 77, 500, 12], dtype=torch.int32, device="cuda")
    seqs = torch.tensor([1003, 1077, 1500, 1012], dtype=torch.int64, device="cuda")
    before = arena.cpu().numpy().copy()
    records = sa.gpu_eventlog_pack(arena, evict, seqs).cpu().numpy()
    p = tmp_path / "cold.sllg"
    with sa.EventLog.create(p) as log:
        log.append_durable(records)
    with sa.EventLog.open(p) as log:
        r = log.fetch_by_seq(1500)
        assert r is not None and r["slot"] == 500
        got = log.read_all()
    fresh = torch.zeros((8, 128), dtype=torch.uint8, device="cuda")
    dst = torch.tensor([7, 0, 5, 2], dtype=torch.int32, device="cuda")
    st = sa.gpu_eventlog_unpack(torch.from_numpy(got.view(np.uint8).reshape(-1, 144).copy()).cuda(), dst,
                                fresh)
    assert not st.cpu().numpy().any()
    out = fresh.cpu().numpy()
    for s, d in zip([3, 77, 500, 12], [7, 0, 5, 2]):
        assert out[d].tobytes() == before[s].tobytes()


def test_empty_log_reads_and_lookups(sa, tmp_path):
    """A log holding only its header: len 0, read_all empty, lookups find
    nothing, and it reopens in every mode."""
    p = tmp_path / "empty"
    with sa.EventLog.create(p) as log:
        assert len(log) == 0 and log.version == 2
        assert len(log.read_all()) == 0
        assert log.fetch_by_seq(0) is None and log.fetch_last_for_slot(0) is None
        log.sync()
    for mode in (sa.EVENTLOG_OPEN_STRICT, sa.EVENTLOG_OPEN_RECOVER, sa.EVENTLOG_OPEN_READ_ONLY):
        with sa.EventLog.open(p, mode) as log:
            assert len(log) == 0
            log.sync()
    assert p.read_bytes() == struct.pack("<IIII", 0x534C4C47, 2, 128, 0)
