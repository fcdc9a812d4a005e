"""Malformed inputs to the host parsers: the .slhw loader (weights.rs:159-311)
and the EventLog file side (eventlog.rs:179-486).

Both read files a caller did not write. Each case mutates a valid file (byte
flips biased to the headers, truncations, extensions, a forged record
count) and opens it in every mode; the call must either succeed or raise the
library's error with a message, never crash, and a successful open must read
back only whole, checksum-valid records (version 2) or the file's records
(version 1). Run under the host sanitizers by tests/run_sanitized.sh, an
out-of-bounds read or undefined behaviour in these paths aborts the run.
"""
import struct

import numpy as np
import pytest

import oracle_ffi as o
import slhav2_amd as s

N_CASES = 150
HEADER, RECORD = 16, 144


def valid_slhw(version: int) -> bytes:
    p = np.random.default_rng(version).normal(size=(128, 136)).astype(np.float32)
    return s.slhw_bytes(p, 0x1234, rht=True, version=version)


def checksum(seq: int, slot: int, tile) -> int:
    return int(o.lib.orc_record_checksum(seq, slot, o._p(np.ascontiguousarray(tile, np.uint8))))


def valid_log(tmp_path, version: int) -> bytes:
    """Five records; version 1 is the same file with the version-1 header and
    zero checksums (the legacy layout, eventlog.rs:25-36)."""
    path = tmp_path / f"seed_v{version}.sllg"
    tiles = np.zeros(5, o.TILE_DTYPE)
    tiles.view(np.uint8).reshape(5, 128)[:] = np.random.default_rng(3).integers(0, 256, (5, 128), dtype=np.uint8)
    rec = o.eventlog_records(tiles, np.arange(5), np.arange(5) + 10, 2)
    with s.EventLog.create(path) as log:
        log.append(rec)
    b = bytearray(path.read_bytes())
    if version == 1:
        b[4:8] = struct.pack("<I", 1)
        for i in range(5):
            b[HEADER + RECORD * i + 12:HEADER + RECORD * i + 16] = bytes(4)
    return bytes(b)


def mutations(data: bytes, seed: int):
    r = np.random.default_rng(seed)
    for i in range(N_CASES):
        b = bytearray(data)
        kind = i % 5
        if kind == 0:  # flip bytes, mostly in the first 64
            for _ in range(int(r.integers(1, 4))):
                pos = int(r.integers(0, 64)) if r.random() < 0.7 else int(r.integers(0, len(b)))
                b[pos % len(b)] ^= int(r.integers(1, 256))
        elif kind == 1:  # truncate
            del b[int(r.integers(0, len(b))):]
        elif kind == 2:  # extend with junk
            b += bytes(r.integers(0, 256, int(r.integers(1, 300)), dtype=np.uint8))
        elif kind == 3:  # overwrite a 4- or 8-byte header field with an extreme value
            pos = int(r.integers(0, 24))
            val = [0, 1, 0xFFFFFFFF, 0x7FFFFFFF, 0x80000000][int(r.integers(0, 5))]
            b[pos:pos + 4] = int(val).to_bytes(4, "little")[: len(b[pos:pos + 4])]
        else:  # flip one byte anywhere
            pos = int(r.integers(0, len(b)))
            b[pos] ^= 1 << int(r.integers(0, 8))
        yield bytes(b)


@pytest.mark.parametrize("version", [1, 2])
def test_slhw_loader_survives_malformed_files(tmp_path, version):
    f = tmp_path / "m.slhw"
    ok = 0
    for i, data in enumerate(mutations(valid_slhw(version), 100 + version)):
        f.write_bytes(data)
        try:
            with s.Model.load(f) as m:
                assert m.dim > 128
                ok += 1
        except s.SlhaError as e:
            assert e.message, i
    assert ok < N_CASES  # most mutations are rejected


@pytest.mark.parametrize("version", [1, 2])
@pytest.mark.parametrize("mode", [s.EVENTLOG_OPEN_STRICT, s.EVENTLOG_OPEN_RECOVER,
                                  s.EVENTLOG_OPEN_READ_ONLY])
def test_eventlog_open_survives_malformed_files(tmp_path, version, mode):
    f = tmp_path / "l.sllg"
    for i, data in enumerate(mutations(valid_log(tmp_path, version), 200 + 10 * version + mode)):
        f.write_bytes(data)
        try:
            log = s.EventLog.open(f, mode)
        except s.SlhaError as e:
            assert e.message, i
            continue
        with log:
            n = len(log)
            assert n <= (len(data) - 16) // 144 + 1
            recs = log.read_all()
            assert len(recs) == n
            if log.version == 2:  # every record read back passes its checksum
                for r in recs:
                    assert int(r["checksum"]) == checksum(int(r["seq"]), int(r["slot"]), r["tile"])
            if n:
                log.fetch_by_seq(int(recs[-1]["seq"]))
                log.fetch_last_for_slot(int(recs[0]["slot"]))
