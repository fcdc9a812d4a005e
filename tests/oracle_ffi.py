"""ctypes binding of the CPU oracle (oracle/liboracle_slha.so) for the tests.

Test infrastructure only: the oracle is the checker, never the thing checked.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
ORACLE_DIR = ROOT / "oracle"
ORACLE_SO = ORACLE_DIR / "liboracle_slha.so"
BASELINE_SO = ORACLE_DIR / "libcpu_baseline.so"

TILE_DTYPE = np.dtype(
    {
        "names": ["latent_kv", "residual_bitmap", "scale", "dynamic_lambda", "residual_sigma",
                  "token_id", "position", "head_id", "flags", "group_scales"],
        "formats": [("u1", 64), ("<u8", 4), "<f4", "<f4", "<f4", "<u4", "<u4", "<u2", "<u2",
                    ("u1", 8)],
        "offsets": [0, 64, 96, 100, 104, 108, 112, 116, 118, 120],
        "itemsize": 128,
    }
)


def _ensure_built() -> None:
    srcs = [ORACLE_DIR / "slha_oracle.c", ORACLE_DIR / "cpu_baseline.c"]
    newest = max(p.stat().st_mtime for p in srcs)
    if ORACLE_SO.exists() and BASELINE_SO.exists() and min(
        ORACLE_SO.stat().st_mtime, BASELINE_SO.stat().st_mtime
    ) >= newest:
        return
    subprocess.run(["python3", str(ROOT / "slhav2_amd" / "build.py"), "oracle"], check=True,
                   capture_output=True)


_ensure_built()
lib = ctypes.CDLL(str(ORACLE_SO))

_P = ctypes.c_void_p
_SZ = ctypes.c_size_t
_F = ctypes.c_float
for name, res, args in [
    ("orc_rng_next_u64", ctypes.c_uint64, [_P]),
    ("orc_rng_next_unit", _F, [_P]),
    ("orc_rng_next_gaussian", _F, [_P]),
    ("orc_rng_fill_gaussian", None, [_P, _P, _SZ]),
    ("orc_rng_init", None, [_P, ctypes.c_uint64]),
    ("orc_quantize_latent", None, [_P, _P, _P]),
    ("orc_quantize_latent_grouped", None, [_P, _P, _P, _P]),
    ("orc_quantize_latent_nf4", None, [_P, _P, _P, _P]),
    ("orc_quantize_latent_mixed", None, [_P, _P, _P, _P]),
    ("orc_quantize_latent_tq3", None, [_P, _P, _P, _P]),
    ("orc_quantize_latent_mix3", None, [_P, _P, _P, _P]),
    ("orc_nf4_nearest", ctypes.c_uint8, [_F]),
    ("orc_dequant_at", _F, [_P, ctypes.c_int]),
    ("orc_dequant_latent", None, [_P, _P]),
    ("orc_hamming", ctypes.c_uint32, [_P, _P]),
    ("orc_compute_score_scalar", _F, [_P, _P, _P]),
    ("orc_projection_fill", None, [_P, _SZ, ctypes.c_uint64]),
    ("orc_sign_bits", None, [_P, _SZ, _P, _P]),
    ("orc_next_pow2", _SZ, [_SZ]),
    ("orc_fwht_inplace", None, [_P, _SZ]),
    ("orc_rht_diag", None, [_P, _SZ, ctypes.c_uint64]),
    ("orc_rht_transform", None, [_P, _SZ, _SZ, _P, _P]),
    ("orc_rms", _F, [_P, _SZ]),
    ("orc_analytic_lambda_c", _F, []),
    ("orc_encode_key", ctypes.c_int, [_P, ctypes.c_int, ctypes.c_int, _P, _P, ctypes.c_uint32,
                                      ctypes.c_uint16, ctypes.c_int, _P]),
    ("orc_query_sign", None, [_P, _P, _P, _P]),
    ("orc_encode_batch", ctypes.c_int, [_P, _SZ, ctypes.c_int, ctypes.c_int, _P, _P,
                                        ctypes.c_uint32, ctypes.c_uint16, _P]),
    ("orc_score_batch", None, [_P, _SZ, _P, _P, _P, _P]),
    ("orc_validate_tile", ctypes.c_int, [_P]),
    ("orc_page_out", None, [_P]),
    ("orc_drop_correction", ctypes.c_int, [_P]),
    ("orc_topk", None, [_P, _SZ, _SZ, _P, _P]),
    ("orc_learned_latent", None, [_P, _SZ, _P, _P]),
    ("orc_learned_query_coarse", None, [_P, _SZ, _P, _P]),
    ("orc_learned_reconstruct", None, [_P, _SZ, _P, _P]),
    ("orc_learned_query", None, [_P, _P, _P, _SZ, _SZ, _P, _P, _P]),
    ("orc_learned_encode", ctypes.c_int, [_P, _P, _P, _SZ, _SZ, _P, ctypes.c_uint32, ctypes.c_int,
                                          ctypes.c_int, _P]),
    ("orc_learned_decode", None, [_P, _P, _SZ, _SZ, ctypes.c_int, _P, ctypes.c_int, _P]),
    ("orc_softmax_into", None, [_P, _SZ, _F, _P]),
    ("orc_aggregate_v", None, [_P, _P, _SZ, _SZ, _P]),
    ("orc_fnv1a", ctypes.c_uint32, [_P, _SZ]),
    ("orc_tile_to_bytes", None, [_P, _P]),
    ("orc_record_checksum", ctypes.c_uint32, [ctypes.c_uint64, ctypes.c_uint32, _P]),
    ("orc_eventlog_record", None, [ctypes.c_uint64, ctypes.c_uint32, _P, ctypes.c_uint32, _P]),
    ("orc_observe_scores", None, [_P, _P, _SZ, _P, _SZ, _F, _P]),
]:
    fn = getattr(lib, name)
    fn.restype = res
    fn.argtypes = args


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


class Rng:
    """The oracle's SplitMix64 (rng.rs)."""

    def __init__(self, seed: int):
        self._state = np.zeros(1, np.uint64)
        lib.orc_rng_init(_p(self._state), ctypes.c_uint64(seed & (2**64 - 1)))

    def next_u64(self) -> int:
        return int(lib.orc_rng_next_u64(_p(self._state)))

    def next_unit(self) -> float:
        return float(lib.orc_rng_next_unit(_p(self._state)))

    def gaussian(self, n: int) -> np.ndarray:
        out = np.empty(n, np.float32)
        lib.orc_rng_fill_gaussian(_p(self._state), _p(out), n)
        return out


QUANTIZERS = {
    1: "orc_quantize_latent_grouped",
    2: "orc_quantize_latent_nf4",
    3: "orc_quantize_latent_mixed",
    4: "orc_quantize_latent_tq3",
    5: "orc_quantize_latent_mix3",
}


def quantize(codec: int, v) -> tuple[np.ndarray, float, np.ndarray]:
    v = f32(v)
    out = np.zeros(64, np.uint8)
    sc = np.zeros(1, np.float32)
    gs = np.full(8, 255, np.uint8)
    if codec == 0:
        lib.orc_quantize_latent(_p(v), _p(out), _p(sc))
    else:
        getattr(lib, QUANTIZERS[codec])(_p(v), _p(out), _p(sc), _p(gs))
    return out, float(sc[0]), gs


def make_tile(latent, scale, gs, flags=0, lam=0.0, sigma=0.0, residual=(0, 0, 0, 0)) -> np.ndarray:
    t = np.zeros(1, TILE_DTYPE)
    t["latent_kv"][0] = np.asarray(latent, np.uint8)
    t["scale"] = scale
    t["group_scales"][0] = np.asarray(gs, np.uint8)
    t["flags"] = flags
    t["dynamic_lambda"] = lam
    t["residual_sigma"] = sigma
    t["residual_bitmap"][0] = np.asarray(residual, np.uint64)
    return t


def dequant(tile) -> np.ndarray:
    t = np.ascontiguousarray(tile, TILE_DTYPE).reshape(-1)
    out = np.zeros(128, np.float32)
    lib.orc_dequant_latent(_p(t), _p(out))
    return out


def score(tiles, q, qs) -> tuple[np.ndarray, np.ndarray]:
    t = np.ascontiguousarray(tiles, TILE_DTYPE).reshape(-1)
    qv = f32(q)
    qsv = np.ascontiguousarray(qs, np.uint64)
    s = np.zeros(len(t), np.float32)
    h = np.zeros(len(t), np.uint32)
    lib.orc_score_batch(_p(t), len(t), _p(qv), _p(qsv), _p(s), _p(h))
    return s, h


def projection(seed: int, d_pad: int = 128) -> np.ndarray:
    z = np.zeros((256, d_pad), np.float32)
    lib.orc_projection_fill(_p(z), d_pad, ctypes.c_uint64(seed & (2**64 - 1)))
    return z


def rht_diag(seed: int, d_pad: int = 128) -> np.ndarray:
    d = np.zeros(d_pad, np.float32)
    lib.orc_rht_diag(_p(d), d_pad, ctypes.c_uint64(seed & (2**64 - 1)))
    return d


def rht(diag, v) -> np.ndarray:
    diag = f32(diag)
    v = f32(v)
    out = np.zeros(len(diag), np.float32)
    lib.orc_rht_transform(_p(diag), len(v), len(diag), _p(v), _p(out))
    return out


def fwht(v) -> np.ndarray:
    v = f32(v).copy()
    lib.orc_fwht_inplace(_p(v), len(v))
    return v


def sign_bits(z, v) -> np.ndarray:
    z = f32(z)
    v = f32(v)
    out = np.zeros(4, np.uint64)
    lib.orc_sign_bits(_p(z), z.shape[1], _p(v), _p(out))
    return out


def query_sign(q, z, diag=None) -> np.ndarray:
    q, z = f32(q), f32(z)
    out = np.zeros(4, np.uint64)
    lib.orc_query_sign(_p(q), _p(z), _p(f32(diag)) if diag is not None else None, _p(out))
    return out


def encode(keys, codec: int, residual_mode: int, z, diag=None, pos0: int = 0, head: int = 0):
    k = f32(keys).reshape(-1, 128)
    z = f32(z)
    out = np.zeros(len(k), TILE_DTYPE)
    d = f32(diag) if diag is not None else None
    rc = lib.orc_encode_batch(_p(k), len(k), codec, residual_mode, _p(z),
                              _p(d) if d is not None else None, pos0, head, _p(out))
    assert rc == 0, rc
    return out


def rms(v) -> float:
    v = f32(v)
    return float(lib.orc_rms(_p(v), len(v)))


def validate(tile) -> int:
    t = np.ascontiguousarray(tile, TILE_DTYPE).reshape(-1)
    return int(lib.orc_validate_tile(_p(t)))


def page_out(tile) -> np.ndarray:
    t = np.array(tile, TILE_DTYPE).reshape(-1).copy()
    lib.orc_page_out(_p(t))
    return t


def drop_correction(tile) -> tuple[np.ndarray, int]:
    t = np.array(tile, TILE_DTYPE).reshape(-1).copy()
    r = lib.orc_drop_correction(_p(t))
    return t, int(r)


def topk(scores, k: int) -> tuple[np.ndarray, np.ndarray]:
    s = f32(scores)
    idx = np.zeros(k, np.uint32)
    val = np.zeros(k, np.float32)
    lib.orc_topk(_p(s), len(s), k, _p(idx), _p(val))
    return idx, val


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round f32 to bf16 (RNE) and widen back to f32, exactly."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


class Learned:
    """The oracle's LearnedModel (learned.rs:257-408) over a loaded projection:
    p [128][d], z [256][d_pad], diag [d_pad] or None."""

    def __init__(self, p, z, diag=None):
        self.p = f32(p)
        self.z = f32(z)
        self.diag = f32(diag) if diag is not None else None
        self.d = self.p.shape[1]
        self.d_pad = self.z.shape[1]
        assert self.p.shape[0] == 128 and self.z.shape[0] == 256

    def _diag(self):
        return _p(self.diag) if self.diag is not None else None

    def latent(self, key) -> np.ndarray:
        k = f32(key)
        h = np.zeros(128, np.float32)
        lib.orc_learned_latent(_p(self.p), self.d, _p(k), _p(h))
        return h

    def reconstruct(self, h) -> np.ndarray:
        h = f32(h)
        out = np.zeros(self.d, np.float32)
        lib.orc_learned_reconstruct(_p(self.p), self.d, _p(h), _p(out))
        return out

    def query(self, q) -> tuple[np.ndarray, np.ndarray]:
        q = f32(q)
        qc = np.zeros(128, np.float32)
        qs = np.zeros(4, np.uint64)
        lib.orc_learned_query(_p(self.p), _p(self.z), self._diag(), self.d, self.d_pad, _p(q),
                              _p(qc), _p(qs))
        return qc, qs

    def encode(self, keys, codec: int, pos0: int = 0, warm: int = 0) -> np.ndarray:
        k = f32(keys).reshape(-1, self.d)
        out = np.zeros(len(k), TILE_DTYPE)
        for i in range(len(k)):
            row = np.ascontiguousarray(k[i])
            rc = lib.orc_learned_encode(_p(self.p), _p(self.z), self._diag(), self.d, self.d_pad,
                                        _p(row), pos0 + i, codec, warm, out[i:i + 1].ctypes.data)
            assert rc == 0, rc
        return out

    def decode(self, tiles, with_residual: bool) -> np.ndarray:
        t = np.ascontiguousarray(tiles, TILE_DTYPE).reshape(-1)
        out = np.zeros((len(t), self.d), np.float32)
        for i in range(len(t)):
            lib.orc_learned_decode(_p(self.p), _p(self.z), self.d, self.d_pad,
                                   int(self.diag is not None), t[i:i + 1].ctypes.data,
                                   int(with_residual), out[i].ctypes.data)
        return out


def softmax(scores, scale: float) -> np.ndarray:
    """metrics.rs:338-409 softmax_into."""
    sc = f32(scores)
    out = np.zeros(len(sc), np.float32)
    lib.orc_softmax_into(_p(sc), len(sc), scale, _p(out))
    return out


def aggregate(weights, values) -> np.ndarray:
    """benchmark_decode.rs:29-38 aggregate_v: weights [n], values [n, d_v]."""
    w = f32(weights)
    v = f32(values)
    out = np.zeros(v.shape[1], np.float32)
    lib.orc_aggregate_v(_p(w), _p(v), len(w), v.shape[1], _p(out))
    return out


def decode_attention(tiles, values, q_coarse, q_sign, scale: float) -> np.ndarray:
    """One query head's decode step over one row: exact eq. 2.3 scores,
    softmax_into, aggregate_v (benchmark_decode.rs:84-90)."""
    sc, _ = score(tiles, q_coarse, q_sign)
    return aggregate(softmax(sc, scale), values)


# --------------------------------------------------------------------------
# EventLog records (eventlog.rs:82-100, 148-170)

def fnv1a(data: bytes) -> int:
    b = np.frombuffer(bytes(data), np.uint8).copy() if len(data) else np.zeros(1, np.uint8)
    return int(lib.orc_fnv1a(_p(b), len(data)))


def tile_to_bytes(tile) -> bytes:
    t = np.ascontiguousarray(tile, TILE_DTYPE).reshape(-1)
    out = np.zeros(128, np.uint8)
    lib.orc_tile_to_bytes(_p(t), _p(out))
    return out.tobytes()


def eventlog_records(tiles, slots, seqs, version: int = 2) -> np.ndarray:
    """144-byte records of tiles[slots[i]] with seq seqs[i] (uint8 [n, 144])."""
    t = np.ascontiguousarray(tiles, TILE_DTYPE).reshape(-1)
    out = np.zeros((len(slots), 144), np.uint8)
    for i, (sl, sq) in enumerate(zip(slots, seqs)):
        one = np.ascontiguousarray(t[int(sl)]).reshape(1)
        row = np.zeros(144, np.uint8)
        lib.orc_eventlog_record(int(sq), int(sl), _p(one), version, _p(row))
        out[i] = row
    return out


def observe_scores(importance, scores, live, temperature: float, slots=None) -> np.ndarray:
    """ccos.rs:257-300 on a copy of `importance` (f32 [n_slots]); scores are
    per slot (slots = arange) unless `slots` is given."""
    imp = np.ascontiguousarray(importance, np.float32).copy()
    sc = np.ascontiguousarray(scores, np.float32)
    sl = np.arange(len(sc), dtype=np.uint32) if slots is None else np.ascontiguousarray(slots, np.uint32)
    lv = np.ascontiguousarray(live, np.uint8)
    lib.orc_observe_scores(_p(sl), _p(sc), len(sc), _p(lv), len(imp), temperature, _p(imp))
    return imp
