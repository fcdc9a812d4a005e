#!/usr/bin/env python3
"""Writes tests/golden/slha_golden.npz: small known-answer vectors for the
tile path, produced by the CPU oracle (oracle/slha_oracle.c).

Contents (all arrays, no pickles; load with numpy.load(allow_pickle=False)):
  keys        f32 [32, 128]  N(0,1) x per-key scale 10^u, u ~ U[-1, 1)
  queries     f32 [3, 128]   N(0,1)
  z_sum, z_head              checksum and first 8 entries of Z (seed SEED)
  diag        f32 [128]      RHT diagonal of the model with seed SEED
  q_sign_rht{r}       u64 [3, 4]
  tiles_c{c}_r{r}_{v} u8 [32, 128]   codec c, RHT r, variant v in
                                     {hot, warm, nocorr (TQ3/MIX3 only),
                                     modez (INT4 single only)}
  scores_... f32 [3, 32], ham_... u32 [3, 32] for every tiles_... array

The variants: hot = mode R encode (position = 100 + i, head 0); warm =
page_out of hot; nocorr = drop_correction of hot; modez = mode Z encode.
tests/test_golden.py checks the oracle against this file on the CPU and the
GPU library against it on the GPU. Rerun this script only when the tile path's
definition changes on purpose.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))

import oracle_ffi as o  # noqa: E402

SEED = 0x5EED0C0D
RHT_XOR = 0xA2A2A2A2A2A2A2A2  # learned.rs:158-165: the RHT diagonal's seed is seed ^ RHT_XOR
N_KEYS, N_Q, POS0 = 32, 3, 100
OUT = HERE / "slha_golden.npz"


def inputs() -> tuple[np.ndarray, np.ndarray]:
    r = o.Rng(0x601D)
    keys = r.gaussian(N_KEYS * 128).reshape(N_KEYS, 128)
    u = np.array([r.next_unit() for _ in range(N_KEYS)], np.float32) * np.float32(2) - np.float32(1)
    keys = (keys * (np.float32(10.0) ** u)[:, None]).astype(np.float32)
    queries = o.Rng(0x601E).gaussian(N_Q * 128).reshape(N_Q, 128)
    return keys, queries


def build() -> dict[str, np.ndarray]:
    keys, queries = inputs()
    z = o.projection(SEED)
    diag = o.rht_diag(SEED ^ RHT_XOR)
    out: dict[str, np.ndarray] = {
        "keys": keys, "queries": queries, "diag": diag,
        "z_sum": np.array([z.astype(np.float64).sum()]), "z_head": z.reshape(-1)[:8].copy(),
    }
    for r in (0, 1):
        d = diag if r else None
        qs = np.stack([o.query_sign(q, z, d) for q in queries])
        out[f"q_sign_rht{r}"] = qs
        for c in range(6):
            hot = o.encode(keys, c, 1, z, d, pos0=POS0, head=0)
            variants = {"hot": hot, "warm": np.concatenate([o.page_out(t) for t in hot])}
            if c == 0:
                variants["modez"] = o.encode(keys, c, 0, z, d, pos0=POS0, head=0)
            if c in (4, 5):
                variants["nocorr"] = np.concatenate([o.drop_correction(t)[0] for t in hot])
            for v, tiles in variants.items():
                name = f"c{c}_r{r}_{v}"
                out[f"tiles_{name}"] = tiles.view(np.uint8).reshape(N_KEYS, 128).copy()
                sc = np.zeros((N_Q, N_KEYS), np.float32)
                hm = np.zeros((N_Q, N_KEYS), np.uint32)
                for j in range(N_Q):
                    sc[j], hm[j] = o.score(tiles, queries[j], qs[j])
                out[f"scores_{name}"] = sc
                out[f"ham_{name}"] = hm
    return out


if __name__ == "__main__":
    np.savez_compressed(OUT, **build())
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")
