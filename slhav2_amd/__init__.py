"""slhav2_amd — MI355X (gfx950) SLHA v2 tile encode + compressed-domain scoring.

Python front of ``libslha.so``, whose C ABI (include/slha.h, include/slha_gpu.h)
is the drop-in boundary. Everything here is a thin ctypes wrapper: the work is
done by the HIP kernels inside the library. Importing this package without a
built ``libslha.so`` raises ImportError; there is no CPU fallback.

Names mirror the reference's C ABI (slha-c/src/lib.rs) and its Rust API
(scirust::attention::slha_v2): ``score_tiles``, ``encode_key``,
``prepare_query`` ... Device wrappers take torch tensors that live on the GPU
(torch is only used for device memory and streams).
"""
from __future__ import annotations

import ctypes
import os
import struct
from pathlib import Path

import numpy as np

__all__ = [
    "SlhaError", "Model", "TILE_DTYPE", "lib", "abi_version", "tile_size", "tile_align",
    "process_tile", "score_tile", "score_tiles", "prepare_query", "encode_key",
    "decode_latent", "decode_key", "audit", "gpu_encode", "gpu_prepare_queries",
    "gpu_score", "gpu_validate_tiles", "gpu_decode", "gpu_ccos_apply",
    "gpu_score_paged_topk",
]

_HERE = Path(__file__).resolve().parent
LIB_PATH = _HERE / "libslha.so"

# slha.h status codes / ids
OK, ERR_NULL, ERR_PANIC, ERR_DIMENSION, ERR_CODEC = 0, -1, -2, -3, -4
ERR_NONFINITE, ERR_INVALID_TILE, ERR_INVALID_HANDLE, ERR_IO, ERR_UTF8 = -5, -6, -7, -8, -9
ERR_DEVICE = -10
CODEC_INT4_SINGLE, CODEC_INT4_GROUPED, CODEC_NF4, CODEC_MIXED, CODEC_TQ3, CODEC_MIX3 = range(6)
CODEC_NAMES = ["int4", "int4_grouped", "nf4", "mixed", "tq3", "mix3"]
FLAG_WARM, FLAG_NF4, FLAG_MIXED, FLAG_TQ3, FLAG_TQ3_NOCORR, FLAG_MIX3 = 1, 2, 4, 8, 16, 32
RESIDUAL_Z, RESIDUAL_R = 0, 1
DTYPE_F32, DTYPE_BF16 = 0, 1
SCORE_FAST, SCORE_EXACT = 0, 1

# tile.rs:52-77 — 128-byte tile.
TILE_DTYPE = np.dtype(
    {
        "names": ["latent_kv", "residual_bitmap", "scale", "dynamic_lambda", "residual_sigma",
                  "token_id", "position", "head_id", "flags", "group_scales"],
        "formats": [("u1", 64), ("<u8", 4), "<f4", "<f4", "<f4", "<u4", "<u4", "<u2", "<u2",
                    ("u1", 8)],
        "offsets": [0, 64, 96, 100, 104, 108, 112, 116, 118, 120],
        "itemsize": 128,
    },
    align=False,
)


class SlhaError(RuntimeError):
    """A non-zero status from the C ABI, with the thread's last error text."""

    def __init__(self, code: int, message: str):
        super().__init__(f"SLHA status {code}: {message}")
        self.code = code
        self.message = message


def _load() -> ctypes.CDLL:
    # torch ships its own HIP/HSA runtimes (SONAME libamdhip64.so.7) and links
    # them by the unversioned name, so loading libslha.so first would put two
    # HIP runtimes in one process. Importing torch first makes libslha.so bind
    # to the runtime torch already loaded. C callers without torch use the
    # system runtime alone.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    # SLHA_LIBRARY names another build of the same library (for example the
    # host-sanitizer build, slhav2_amd/build.py sanitize); default libslha.so.
    path = Path(os.environ.get("SLHA_LIBRARY", "") or LIB_PATH)
    if not path.exists():
        raise ImportError(
            f"{path} is not built; run `python -c 'import __graft_entry__ as g; g.build()'`"
        )
    return ctypes.CDLL(str(path))


lib = _load()

_P = ctypes.c_void_p
_SZ = ctypes.c_size_t
_I32 = ctypes.c_int32
_U32 = ctypes.c_uint32
_U64 = ctypes.c_uint64

_SIGS = {
    "slha_abi_version": (_U32, []),
    "slha_tile_size": (_SZ, []),
    "slha_tile_align": (_SZ, []),
    "slha_last_error_message": (ctypes.c_char_p, []),
    "slha_clear_error": (None, []),
    "slha_init": (_P, []),
    "slha_shutdown": (_I32, [_P]),
    "slha_process_tile": (_I32, [_P, _P, _P, _P]),
    "slha_prepare_query": (_I32, [_P, _P, _SZ, _P, _P]),
    "slha_score_tile": (_I32, [_P, _P, _P, _P, _P]),
    "slha_score_tiles": (_I32, [_P, _P, _SZ, _P, _P, _P]),
    "slha_audit": (_P, []),
    "slha_free_string": (None, [_P]),
    "slha_weights_load": (_P, [ctypes.c_char_p]),
    "slha_model_dim": (_SZ, [_P]),
    "slha_encode_key": (_I32, [_P, _P, _SZ, _U32, _I32, _P]),
    "slha_decode_latent": (_I32, [_P, _P, _P, _SZ]),
    "slha_decode_key": (_I32, [_P, _P, _P, _SZ]),
    "slha_weights_release": (_I32, [_P]),
    "slha_weights_free": (None, [_P]),
    "slha_model_new_raw128": (_P, [_U64, _I32, _I32]),
    "slha_model_projection": (_I32, [_P, _P, _P]),
    "slha_model_pad_dim": (_SZ, [_P]),
    "slha_model_latent_projection": (_I32, [_P, _P]),
    "slha_gpu_encode": (_I32, [_P, _P, _I32, _SZ, _SZ, _SZ, _U32, _I32, _I32, _P, _P]),
    "slha_gpu_prepare_queries": (_I32, [_P, _P, _I32, _SZ, _P, _P, _P]),
    "slha_gpu_score": (_I32, [_P, _SZ, _SZ, _P, _P, _SZ, _I32, _P, _P, _P]),
    "slha_gpu_score_codec": (_I32, [_P, _SZ, _SZ, _P, _P, _SZ, _I32, _I32, _P, _P, _P]),
    "slha_gpu_validate_tiles": (_I32, [_P, _SZ, _P, _P]),
    "slha_gpu_decode": (_I32, [_P, _P, _SZ, _I32, _P, _P]),
    "slha_gpu_score_paged_topk": (_I32, [_P, _SZ, _P, _SZ, _P, _P, _SZ, _SZ, _SZ, _SZ, _P, _P,
                                         _P, _SZ, _P, _P, _P]),
    "slha_gpu_score_paged_topk_noalloc": (_I32, [_P, _SZ, _P, _SZ, _P, _P, _SZ, _SZ, _SZ, _SZ, _P,
                                                 _P, _P, _SZ, _P, _P, _P]),
    "slha_gpu_ccos_apply": (_I32, [_P, _P, _SZ, _I32, _P]),
    "slha_gpu_decode_attention": (_I32, [_P, _P, _I32, _SZ, _SZ, _SZ, _P, _P, _SZ, ctypes.c_float,
                                         _P, _P]),
    "slha_gpu_synchronize": (_I32, [_P]),
    "slha_eventlog_create": (_P, [ctypes.c_char_p, _I32]),
    "slha_eventlog_open": (_P, [ctypes.c_char_p, _I32]),
    "slha_eventlog_append": (_I32, [_P, _P, _SZ, _I32]),
    "slha_eventlog_sync": (_I32, [_P]),
    "slha_eventlog_len": (_U64, [_P]),
    "slha_eventlog_version": (_U32, [_P]),
    "slha_eventlog_read": (_I32, [_P, _U64, _SZ, _P]),
    "slha_eventlog_find_seq": (_I32, [_P, _U64, _P, _P]),
    "slha_eventlog_find_slot": (_I32, [_P, _U32, _P, _P]),
    "slha_eventlog_close": (_I32, [_P]),
    "slha_gpu_eventlog_pack": (_I32, [_P, _P, _P, _SZ, _U32, _P, _P]),
    "slha_gpu_eventlog_unpack": (_I32, [_P, _SZ, _U32, _P, _P, _P, _P]),
    "slha_ccos_new": (_P, [_P, _SZ, _SZ, _I32, _I32, _SZ]),
    "slha_ccos_free": (_I32, [_P]),
    "slha_ccos_attach_event_log": (_I32, [_P, _P, _I32]),
    "slha_ccos_insert": (_I32, [_P, _P, _SZ, _P, _P]),
    "slha_ccos_observe_scores": (_I32, [_P, _P, _SZ, ctypes.c_float, _P]),
    "slha_ccos_enforce_budget": (_I32, [_P, _P, _P]),
    "slha_ccos_page_out": (_I32, [_P, _U32, _P]),
    "slha_ccos_drop_correction": (_I32, [_P, _U32, _P, _P]),
    "slha_ccos_evict": (_I32, [_P, _U32, _P, _P]),
    "slha_ccos_rehydrate": (_I32, [_P, _U64, _P, _P]),
    "slha_ccos_stats": (_I32, [_P, _P]),
    "slha_ccos_slots": (_I32, [_P, _SZ, _P, _P, _P, _P]),
}
for _name, (_res, _args) in _SIGS.items():
    _fn = getattr(lib, _name)
    _fn.restype = _res
    _fn.argtypes = _args


def last_error() -> str:
    msg = lib.slha_last_error_message()
    return msg.decode("utf-8", "replace") if msg else ""


def _check(code: int) -> None:
    if code != OK:
        raise SlhaError(code, last_error())


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def abi_version() -> int:
    return int(lib.slha_abi_version())


def tile_size() -> int:
    return int(lib.slha_tile_size())


def tile_align() -> int:
    return int(lib.slha_tile_align())


def audit() -> str:
    p = lib.slha_audit()
    if not p:
        raise SlhaError(ERR_PANIC, last_error())
    try:
        return ctypes.string_at(p).decode()
    finally:
        lib.slha_free_string(p)


class Model:
    """A projection model: head_dim 128 (slha_model_new_raw128) or, with
    Model.load, a learned d > 128 projection from a .slhw file
    (slha_weights_load)."""

    def __init__(self, seed: int = 0, rht: bool = False, residual_mode: int = RESIDUAL_R):
        h = lib.slha_model_new_raw128(_U64(seed & (2**64 - 1)), int(bool(rht)), residual_mode)
        if not h:
            raise SlhaError(ERR_CODEC, last_error())
        self.handle = h
        self.seed, self.rht, self.residual_mode = seed, bool(rht), residual_mode

    @classmethod
    def load(cls, path) -> "Model":
        """Learned model from a .slhw v1/v2 file (weights.rs:159-311)."""
        h = lib.slha_weights_load(os.fsencode(path))
        if not h:
            raise SlhaError(ERR_IO, last_error())
        m = cls.__new__(cls)
        m.handle = h
        m.seed, m.rht, m.residual_mode = None, None, None
        return m

    @property
    def dim(self) -> int:
        d = lib.slha_model_dim(self.handle)
        if d == 0:
            raise SlhaError(ERR_INVALID_HANDLE, last_error())
        return int(d)

    @property
    def pad_dim(self) -> int:
        d = lib.slha_model_pad_dim(self.handle)
        if d == 0:
            raise SlhaError(ERR_INVALID_HANDLE, last_error())
        return int(d)

    def projection(self) -> tuple[np.ndarray, np.ndarray]:
        """(Z [256, d_pad], RHT diagonal [d_pad]; all +1 without RHT)."""
        dp = self.pad_dim
        z = np.empty((256, dp), np.float32)
        diag = np.empty(dp, np.float32)
        _check(lib.slha_model_projection(self.handle, _ptr(z), _ptr(diag)))
        return z, diag

    def latent_projection(self) -> np.ndarray:
        """P [128, d] (the identity for head_dim 128)."""
        p = np.empty((128, self.dim), np.float32)
        _check(lib.slha_model_latent_projection(self.handle, _ptr(p)))
        return p

    def release(self) -> None:
        if self.handle:
            _check(lib.slha_weights_release(self.handle))
            self.handle = None

    def __enter__(self) -> "Model":
        return self

    def __exit__(self, *exc) -> None:
        self.release()


def _tiles_in(tiles) -> np.ndarray:
    t = np.ascontiguousarray(tiles)
    if t.dtype != TILE_DTYPE:
        t = t.view(TILE_DTYPE) if t.dtype == np.uint8 else t.astype(TILE_DTYPE)
    return t.reshape(-1)


def process_tile(tile, q_coarse, q_sign) -> float:
    t = _tiles_in(tile)
    qc = np.ascontiguousarray(q_coarse, np.float32)
    qs = np.ascontiguousarray(q_sign, np.uint64)
    out = np.zeros(1, np.float32)
    _check(lib.slha_process_tile(_ptr(t), _ptr(qc), _ptr(qs), _ptr(out)))
    return float(out[0])


def score_tile(model: Model, tile, q_coarse, q_sign) -> float:
    t = _tiles_in(tile)
    qc = np.ascontiguousarray(q_coarse, np.float32)
    qs = np.ascontiguousarray(q_sign, np.uint64)
    out = np.zeros(1, np.float32)
    _check(lib.slha_score_tile(model.handle, _ptr(t), _ptr(qc), _ptr(qs), _ptr(out)))
    return float(out[0])


def score_tiles(model: Model, tiles, q_coarse, q_sign) -> np.ndarray:
    t = _tiles_in(tiles)
    qc = np.ascontiguousarray(q_coarse, np.float32)
    qs = np.ascontiguousarray(q_sign, np.uint64)
    out = np.zeros(len(t), np.float32)
    _check(lib.slha_score_tiles(model.handle, _ptr(t), len(t), _ptr(qc), _ptr(qs), _ptr(out)))
    return out


def prepare_query(model: Model, q) -> tuple[np.ndarray, np.ndarray]:
    qv = np.ascontiguousarray(q, np.float32)
    qc = np.zeros(128, np.float32)
    qs = np.zeros(4, np.uint64)
    _check(lib.slha_prepare_query(model.handle, _ptr(qv), qv.size, _ptr(qc), _ptr(qs)))
    return qc, qs


def encode_key(model: Model, key, position: int, codec: int) -> np.ndarray:
    k = np.ascontiguousarray(key, np.float32)
    out = np.zeros(1, TILE_DTYPE)
    _check(lib.slha_encode_key(model.handle, _ptr(k), k.size, position, codec, _ptr(out)))
    return out[0]


def decode_latent(model: Model, tile) -> np.ndarray:
    t = _tiles_in(tile)
    d = model.dim
    out = np.zeros(d, np.float32)
    _check(lib.slha_decode_latent(model.handle, _ptr(t), _ptr(out), d))
    return out


def decode_key(model: Model, tile) -> np.ndarray:
    t = _tiles_in(tile)
    d = model.dim
    out = np.zeros(d, np.float32)
    _check(lib.slha_decode_key(model.handle, _ptr(t), _ptr(out), d))
    return out


SLHW_MAGIC = 0x534C4857


def _fnv1a(data: bytes) -> int:
    h = 0x811C9DC5
    for b in data:
        h = ((h ^ b) * 0x01000193) & 0xFFFFFFFF
    return h


def slhw_bytes(p, seed: int, rht: bool, version: int = 2) -> bytes:
    """A .slhw file image of projection p [128, d] (weights.rs:8-31, 86-141):
    version 2 carries the FNV-1a checksum of header and payload."""
    p = np.ascontiguousarray(p, np.float32)
    if p.ndim != 2 or p.shape[0] != 128 or p.shape[1] <= 128:
        raise ValueError("projection must be [128, d] with d > 128")
    if not np.isfinite(p).all():
        raise ValueError("projection must be finite")
    header = struct.pack("<IIIQB3x", SLHW_MAGIC, version, p.shape[1], seed & (2**64 - 1),
                         int(bool(rht)))
    payload = p.astype("<f4").tobytes()
    if version == 1:
        return header + payload
    return header + struct.pack("<I", _fnv1a(header + payload)) + payload


def save_weights(path, p, seed: int, rht: bool) -> None:
    """Write a version-2 .slhw file (weights::save, weights.rs:275-281)."""
    with open(path, "wb") as f:
        f.write(slhw_bytes(p, seed, rht))


# --------------------------------------------------------------------------
# Device API (torch tensors on the GPU)

def _stream(stream=None) -> int:
    import torch

    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)


def _dev_ptr(t) -> int:
    if t is None:
        return 0
    if not t.is_cuda:
        raise ValueError("device API expects GPU tensors")
    if not t.is_contiguous():
        raise ValueError("device API expects contiguous tensors")
    return int(t.data_ptr())


def gpu_encode(model: Model, keys, codec: int, n_kv_heads: int = 1, pos0: int = 0,
               warm: bool = False, out=None, stream=None):
    """keys: [n_rows, n_tok, 128] (or [n_tok, 128]) f32/bf16 -> tiles uint8 [n_rows, n_tok, 128]."""
    import torch

    k = keys if keys.dim() == 3 else keys.unsqueeze(0)
    n_rows, n_tok, d = k.shape
    if d != model.dim:
        raise ValueError(f"keys must have {model.dim} features")
    dtype = {torch.float32: DTYPE_F32, torch.bfloat16: DTYPE_BF16}[k.dtype]
    if out is None:
        out = torch.empty((n_rows, n_tok, 128), dtype=torch.uint8, device=k.device)
    _check(lib.slha_gpu_encode(model.handle, _dev_ptr(k), dtype, n_rows, n_tok, n_kv_heads, pos0,
                               codec, int(bool(warm)), _dev_ptr(out), _stream(stream)))
    return out if keys.dim() == 3 else out[0]


def gpu_prepare_queries(model: Model, q, stream=None):
    """q: [n, d] f32/bf16 -> (q_coarse f32 [n,128], q_sign int64 [n,4] (u64 bits))."""
    import torch

    qq = q.reshape(-1, model.dim)
    dtype = {torch.float32: DTYPE_F32, torch.bfloat16: DTYPE_BF16}[qq.dtype]
    qc = torch.empty((qq.shape[0], 128), dtype=torch.float32, device=qq.device)
    qs = torch.empty((qq.shape[0], 4), dtype=torch.int64, device=qq.device)
    _check(lib.slha_gpu_prepare_queries(model.handle, _dev_ptr(qq), dtype, qq.shape[0],
                                        _dev_ptr(qc), _dev_ptr(qs), _stream(stream)))
    return qc, qs


def gpu_score(tiles, q_coarse, q_sign, group: int = 1, mode: int = SCORE_FAST,
              hamming: bool = False, out=None, stream=None, codec_hint: int | None = None):
    """tiles uint8 [n_rows, n_tok, 128]; q_* [n_rows*group, ...] -> scores f32 [n_rows*group, n_tok].
    codec_hint: the CODEC_* the tiles were encoded with (slha_gpu_score_codec);
    it selects kernels only."""
    import torch

    t = tiles if tiles.dim() == 3 else tiles.unsqueeze(0)
    n_rows, n_tok, _ = t.shape
    if q_coarse.shape[0] != n_rows * group or q_sign.shape[0] != n_rows * group:
        raise ValueError("expected n_rows*group queries")
    if out is None:
        out = torch.empty((n_rows * group, n_tok), dtype=torch.float32, device=t.device)
    ham = torch.empty((n_rows * group, n_tok), dtype=torch.int32, device=t.device) if hamming else None
    if codec_hint is None:
        _check(lib.slha_gpu_score(_dev_ptr(t), n_rows, n_tok, _dev_ptr(q_coarse), _dev_ptr(q_sign),
                                  group, mode, _dev_ptr(out), _dev_ptr(ham), _stream(stream)))
    else:
        _check(lib.slha_gpu_score_codec(_dev_ptr(t), n_rows, n_tok, _dev_ptr(q_coarse),
                                        _dev_ptr(q_sign), group, mode, int(codec_hint), _dev_ptr(out),
                                        _dev_ptr(ham), _stream(stream)))
    return (out, ham) if hamming else out


def gpu_validate_tiles(tiles, stream=None):
    """Returns (index, status) of the lowest invalid tile, or None."""
    import torch

    t = tiles.reshape(-1, 128)
    st = torch.empty(1, dtype=torch.int64, device=t.device)
    _check(lib.slha_gpu_validate_tiles(_dev_ptr(t), t.shape[0], _dev_ptr(st), _stream(stream)))
    v = int(st.cpu().numpy().view(np.uint64)[0])
    if v == 2**64 - 1:
        return None
    return (v >> 8) - 1, -(v & 0xFF)


def gpu_decode(model: Model, tiles, with_residual: bool = False, stream=None):
    import torch

    t = tiles.reshape(-1, 128)
    out = torch.empty((t.shape[0], model.dim), dtype=torch.float32, device=t.device)
    _check(lib.slha_gpu_decode(model.handle, _dev_ptr(t), t.shape[0], int(bool(with_residual)),
                               _dev_ptr(out), _stream(stream)))
    return out


def gpu_decode_attention(tiles, values, q_coarse, q_sign, group: int = 1, scale: float | None = None,
                         out=None, stream=None):
    """tiles uint8 [n_rows, n_tok, 128], values [n_rows, n_tok, d_v] f32/bf16,
    q_* [n_rows*group, ...] -> out f32 [n_rows*group, d_v] = softmax(s * scale) V
    (scale defaults to 1/sqrt(128), benchmark_decode.rs:51)."""
    import torch

    t = tiles if tiles.dim() == 3 else tiles.unsqueeze(0)
    v = values if values.dim() == 3 else values.unsqueeze(0)
    n_rows, n_tok, _ = t.shape
    d_v = v.shape[2]
    if v.shape[:2] != (n_rows, n_tok):
        raise ValueError("values must be [n_rows, n_tok, d_v]")
    dtype = {torch.float32: DTYPE_F32, torch.bfloat16: DTYPE_BF16}[v.dtype]
    if scale is None:
        scale = 1.0 / np.sqrt(128.0)
    if out is None:
        out = torch.empty((n_rows * group, d_v), dtype=torch.float32, device=t.device)
    _check(lib.slha_gpu_decode_attention(_dev_ptr(t), _dev_ptr(v), dtype, n_rows, n_tok, d_v,
                                         _dev_ptr(q_coarse), _dev_ptr(q_sign), group,
                                         ctypes.c_float(scale), _dev_ptr(out), _stream(stream)))
    return out


def gpu_ccos_apply(tiles, slots, op: int, stream=None) -> None:
    """op 0 = page_out (HOT->WARM), op 1 = drop_correction; slots int32 tensor of tile indices."""
    t = tiles.reshape(-1, 128)
    _check(lib.slha_gpu_ccos_apply(_dev_ptr(t), _dev_ptr(slots), slots.numel(), op,
                                   _stream(stream)))


def gpu_score_paged_topk(arena, page_tiles: int, page_table, max_pages: int, seq_len,
                         n_kv_heads: int, group: int, q_coarse, q_sign, k: int,
                         max_len: int | None = None, scores=None, stream=None,
                         noalloc: bool = False):
    """Paged CCOS scoring + top-k. seq_len: int32 GPU tensor [n_seq].

    Returns (scores f32 flat, topk_idx int32 [n_seq, Hq, k], topk_val f32 [n_seq, Hq, k]);
    scores of sequence s start at score_base[s] = Hq * sum(seq_len[:s]).
    noalloc=True calls slha_gpu_score_paged_topk_noalloc (the library
    allocates nothing; the outputs here are still torch tensors).
    """
    import torch

    n_seq = seq_len.numel()
    hq = n_kv_heads * group
    lens64 = seq_len.to(torch.int64)
    base = torch.zeros(n_seq, dtype=torch.int64, device=seq_len.device)
    if n_seq > 1:
        base[1:] = torch.cumsum(lens64, 0)[:-1] * hq
    if max_len is None:
        max_len = int(lens64.max().item()) if n_seq else 0
    if scores is None:
        total = int(lens64.sum().item()) * hq
        scores = torch.empty(max(total, 1), dtype=torch.float32, device=seq_len.device)
    idx = torch.empty((n_seq, hq, max(k, 1)), dtype=torch.int32, device=seq_len.device)
    val = torch.empty((n_seq, hq, max(k, 1)), dtype=torch.float32, device=seq_len.device)
    fn = lib.slha_gpu_score_paged_topk_noalloc if noalloc else lib.slha_gpu_score_paged_topk
    _check(fn(
        _dev_ptr(arena), page_tiles, _dev_ptr(page_table), max_pages, _dev_ptr(seq_len),
        _dev_ptr(base), n_seq, max_len, n_kv_heads, group, _dev_ptr(q_coarse), _dev_ptr(q_sign),
        _dev_ptr(scores), k, _dev_ptr(idx), _dev_ptr(val), _stream(stream)))
    return scores, idx, val


def synchronize(stream=None) -> None:
    _check(lib.slha_gpu_synchronize(_stream(stream)))


# ---------------------------------------------------------------------------
# EventLog (scirust/src/eventlog.rs) over the C ABI

EVENTLOG_RECORD_BYTES = 144
EVENTLOG_OPEN_STRICT, EVENTLOG_OPEN_RECOVER, EVENTLOG_OPEN_READ_ONLY = 0, 1, 2
RECORD_DTYPE = None  # numpy structured dtype of one record, set on first use


def record_dtype():
    """numpy dtype of one 144-byte record: seq u64, slot u32, checksum u32, tile 128 B."""
    global RECORD_DTYPE
    if RECORD_DTYPE is None:
        import numpy as np

        RECORD_DTYPE = np.dtype([("seq", "<u8"), ("slot", "<u4"), ("checksum", "<u4"), ("tile", "u1", 128)])
    return RECORD_DTYPE


class EventLog:
    """Mirror of `EventLog` (eventlog.rs:179-486): create / create_new / open /
    open_recover / open_read_only, append / append_durable of packed records,
    len, sync, read_all, fetch_by_seq, fetch_last_for_slot. Errors raise
    SlhaError with the reference's messages ("EventLog: bad magic", ...)."""

    def __init__(self, handle):
        self._h = handle

    @classmethod
    def _made(cls, h):
        if not h:
            raise SlhaError(ERR_IO, last_error())
        return cls(h)

    @classmethod
    def create(cls, path) -> "EventLog":
        return cls._made(lib.slha_eventlog_create(os.fsencode(path), 0))

    @classmethod
    def create_new(cls, path) -> "EventLog":
        return cls._made(lib.slha_eventlog_create(os.fsencode(path), 1))

    @classmethod
    def open(cls, path, mode: int = EVENTLOG_OPEN_STRICT) -> "EventLog":
        return cls._made(lib.slha_eventlog_open(os.fsencode(path), mode))

    @classmethod
    def open_recover(cls, path) -> "EventLog":
        return cls.open(path, EVENTLOG_OPEN_RECOVER)

    @classmethod
    def open_read_only(cls, path) -> "EventLog":
        return cls.open(path, EVENTLOG_OPEN_READ_ONLY)

    def append(self, records, durable: bool = False) -> None:
        """records: numpy array of record_dtype() (or raw bytes, 144 per record)."""
        import numpy as np

        buf = np.ascontiguousarray(np.frombuffer(memoryview(records).cast("B"), dtype=np.uint8))
        if buf.size % EVENTLOG_RECORD_BYTES:
            raise ValueError("records must be a whole number of 144-byte records")
        _check(lib.slha_eventlog_append(self._h, buf.ctypes.data, buf.size // EVENTLOG_RECORD_BYTES,
                                        1 if durable else 0))

    def append_durable(self, records) -> None:
        self.append(records, durable=True)

    def __len__(self) -> int:
        n = lib.slha_eventlog_len(self._h)
        if n == 0 and last_error():
            raise SlhaError(ERR_INVALID_HANDLE, last_error())
        return n

    @property
    def version(self) -> int:
        return lib.slha_eventlog_version(self._h)

    def sync(self) -> None:
        _check(lib.slha_eventlog_sync(self._h))

    def read(self, first: int = 0, n: int | None = None):
        import numpy as np

        if n is None:
            n = len(self) - first
        out = np.zeros(n, dtype=record_dtype())
        _check(lib.slha_eventlog_read(self._h, first, n, out.ctypes.data if n else None))
        return out

    def read_all(self):
        return self.read(0)

    def _find(self, fn, key):
        idx, found = ctypes.c_uint64(0), ctypes.c_int32(0)
        _check(fn(self._h, key, ctypes.byref(idx), ctypes.byref(found)))
        return self.read(idx.value, 1)[0] if found.value else None

    def fetch_by_seq(self, seq: int):
        return self._find(lib.slha_eventlog_find_seq, seq)

    def fetch_last_for_slot(self, slot: int):
        return self._find(lib.slha_eventlog_find_slot, slot)

    def close(self) -> None:
        if self._h:
            _check(lib.slha_eventlog_close(self._h))
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def gpu_eventlog_pack(arena, slots, seqs, version: int = 2, stream=None):
    """Records (uint8 GPU tensor [n, 144]) of arena tiles `slots` (int32 [n])
    with insertion sequence numbers `seqs` (int64 [n]) - ElasticKvCache::evict."""
    import torch

    n = slots.numel()
    rec = torch.empty((n, EVENTLOG_RECORD_BYTES), dtype=torch.uint8, device=arena.device)
    _check(lib.slha_gpu_eventlog_pack(_dev_ptr(arena.reshape(-1, 128)), _dev_ptr(slots), _dev_ptr(seqs), n,
                                      version, _dev_ptr(rec), _stream(stream)))
    return rec


def gpu_eventlog_unpack(records, dst_slots, arena, version: int = 2, stream=None):
    """Writes each record's tile into arena slot dst_slots[i] when its checksum
    holds; returns the int32 status [n] (0 restored, 1 checksum mismatch)."""
    import torch

    n = dst_slots.numel()
    status = torch.empty(n, dtype=torch.int32, device=arena.device)
    _check(lib.slha_gpu_eventlog_unpack(_dev_ptr(records), n, version, _dev_ptr(dst_slots),
                                        _dev_ptr(arena.reshape(-1, 128)), _dev_ptr(status), _stream(stream)))
    return status


# ---------------------------------------------------------------------------
# CCOS ElasticKvCache (scirust/src/ccos.rs) over a device arena

PAGE_LOWEST_IMPACT_FIRST, PAGE_OLDEST_FIRST = 0, 1
EVICT_CAUSAL, EVICT_IMPORTANCE = 0, 1
HOT, WARM, COLD = 0, 1, 2


class _CcosStats(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in ("live_bytes", "len", "hot", "warm", "cold", "nocorr",
                                                "reclaimed_correction", "log_errors", "blocked_evictions")]


class ElasticKvCache:
    """Mirror of `ElasticKvCache` (ccos.rs:105-614) with the arena in HBM:
    `arena` is a uint8 GPU tensor [capacity, 128] that the cache fills from
    slot 0. Method names follow the reference; scores come from the GPU."""

    def __init__(self, arena, budget_bytes: int, policy: int = PAGE_LOWEST_IMPACT_FIRST,
                 eviction: int = EVICT_CAUSAL, sink_window: int = 0, stream=None):
        self.arena = arena.reshape(-1, 128)
        self._stream = stream
        self._log = None
        h = lib.slha_ccos_new(_dev_ptr(self.arena), self.arena.shape[0], budget_bytes, policy, eviction,
                              sink_window)
        if not h:
            raise SlhaError(ERR_DIMENSION, last_error())
        self._h = h

    @classmethod
    def with_budget(cls, arena, budget_bytes: int, **kw) -> "ElasticKvCache":
        return cls(arena, budget_bytes, **kw)

    @classmethod
    def with_eviction(cls, arena, budget_bytes: int, sink_window: int | None = None, **kw):
        """EvictionPolicy::Importance { sink_window } when sink_window is given."""
        if sink_window is None:
            return cls(arena, budget_bytes, **kw)
        return cls(arena, budget_bytes, eviction=EVICT_IMPORTANCE, sink_window=sink_window, **kw)

    def close(self) -> None:
        if self._h:
            _check(lib.slha_ccos_free(self._h))
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def attach_event_log(self, log: "EventLog") -> None:
        self._log = log
        _check(lib.slha_ccos_attach_event_log(self._h, log._h, 0))

    def attach_durable_event_log(self, log: "EventLog") -> None:
        self._log = log
        _check(lib.slha_ccos_attach_event_log(self._h, log._h, 1))

    def insert(self, tiles) -> list:
        """Inserts GPU tiles (uint8 [n, 128]) in order; returns their slots."""
        import numpy as np

        t = tiles.reshape(-1, 128)
        out = np.zeros(t.shape[0], np.uint32)
        _check(lib.slha_ccos_insert(self._h, _dev_ptr(t), t.shape[0], out.ctypes.data, _stream(self._stream)))
        return [int(x) for x in out]

    def _stats(self) -> _CcosStats:
        st = _CcosStats()
        _check(lib.slha_ccos_stats(self._h, ctypes.byref(st)))
        return st

    def __len__(self) -> int:
        return self._stats().len

    def live_bytes(self) -> int:
        return self._stats().live_bytes

    def counts(self) -> tuple:
        st = self._stats()
        return st.hot, st.warm, st.cold

    def nocorr_count(self) -> int:
        return self._stats().nocorr

    def reclaimed_correction_bytes(self) -> int:
        return self._stats().reclaimed_correction

    def log_errors(self) -> int:
        return self._stats().log_errors

    def blocked_evictions(self) -> int:
        return self._stats().blocked_evictions

    def _slots(self):
        import numpy as np

        n = len(self)
        state = np.zeros(n, np.int32)
        seq = np.zeros(n, np.uint64)
        imp = np.zeros(n, np.float32)
        _check(lib.slha_ccos_slots(self._h, n, state.ctypes.data, seq.ctypes.data, imp.ctypes.data,
                                   _stream(self._stream)))
        return state, seq, imp

    def state(self, slot: int) -> int:
        return int(self._slots()[0][slot])

    def importance(self, slot: int) -> float:
        return float(self._slots()[2][slot])

    def tile(self, slot: int):
        return self.arena[slot]

    def score_all(self, q_coarse, q_sign):
        """(slots, scores) of every live slot, scored on the GPU in exact mode
        (compute_score, tile.rs:267-281); also returns the dense score row."""
        import numpy as np

        n = len(self)
        dense = gpu_score(self.arena[:n], q_coarse.reshape(1, -1), q_sign.reshape(1, -1), group=1,
                          mode=SCORE_EXACT, stream=self._stream).reshape(-1)
        state = self._slots()[0]
        live = np.nonzero(state != COLD)[0]
        return live, dense.cpu().numpy()[live], dense

    def observe_scores(self, scores, temperature: float) -> None:
        """scores: f32 GPU tensor of the arena prefix (one per slot)."""
        _check(lib.slha_ccos_observe_scores(self._h, _dev_ptr(scores), scores.numel(), temperature,
                                            _stream(self._stream)))

    def enforce_budget(self) -> bool:
        ok = ctypes.c_int32(0)
        _check(lib.slha_ccos_enforce_budget(self._h, ctypes.byref(ok), _stream(self._stream)))
        return bool(ok.value)

    def page_out(self, slot: int) -> None:
        _check(lib.slha_ccos_page_out(self._h, slot, _stream(self._stream)))

    def drop_correction(self, slot: int) -> bool:
        done = ctypes.c_int32(0)
        _check(lib.slha_ccos_drop_correction(self._h, slot, ctypes.byref(done), _stream(self._stream)))
        return bool(done.value)

    def evict(self, slot: int) -> bool:
        done = ctypes.c_int32(0)
        _check(lib.slha_ccos_evict(self._h, slot, ctypes.byref(done), _stream(self._stream)))
        return bool(done.value)

    def rehydrate(self, seq: int):
        slot = ctypes.c_int64(-1)
        _check(lib.slha_ccos_rehydrate(self._h, seq, ctypes.byref(slot), _stream(self._stream)))
        return None if slot.value < 0 else int(slot.value)
