"""C-ABI checks that need no GPU: exports, layout, error contract, models.

Mirrors the reference's C-ABI tests (slha-c/src/lib.rs:915-1886, in particular
the NULL / handle / dimension error cases at :975-1013 and :1222-1256). Nothing
here launches a kernel.
"""
import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

import oracle_ffi as o
import slhav2_amd as s

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    syms = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        syms |= set(re.findall(r"\b(slha_\w+)\s*\(", text))
    return syms


def test_library_exports_every_declared_symbol():
    syms = declared_symbols()
    assert len(syms) >= 20 + 10
    missing = [n for n in sorted(syms) if not hasattr(s.lib, n)]
    assert not missing, missing


def test_reference_abi_symbols_present():
    # The 20 exports of slha-c/include/slha.h:123-278.
    ref = """slha_abi_version slha_tile_size slha_tile_align slha_last_error_message
    slha_clear_error slha_init slha_shutdown slha_process_tile slha_prepare_query
    slha_score_tile slha_score_tiles slha_audit slha_free_string slha_weights_load
    slha_model_dim slha_encode_key slha_decode_latent slha_decode_key
    slha_weights_release slha_weights_free""".split()
    assert len(ref) == 20
    assert set(ref) <= declared_symbols()


def test_product_library_does_not_contain_the_oracle():
    out = subprocess.run(["nm", "-D", str(s.LIB_PATH)], capture_output=True, text=True).stdout
    assert "orc_" not in out and "cpu_score_rows" not in out


def test_layout_and_versions():
    assert s.abi_version() == 1
    assert s.tile_size() == 128 and s.tile_align() == 64
    assert s.TILE_DTYPE.itemsize == 128
    assert s.TILE_DTYPE.fields["flags"][1] == 118
    assert s.TILE_DTYPE.fields["group_scales"][1] == 120


@pytest.mark.parametrize("lang", ["c", "c++"])
@pytest.mark.parametrize("line128", [False, True])
def test_header_alignment_option(tmp_path, lang, line128):
    # slha.h:48-57 and tests.rs:12-20: SLHA_CACHE_LINE_128=1 gives 128-byte
    # alignment, otherwise 64; the tile is 128 bytes with no padding and the
    # same field offsets either way (the header's static asserts hold).
    src = tmp_path / ("t.c" if lang == "c" else "t.cpp")
    src.write_text("""#include <stdio.h>
#include "slha.h"
int main(void) {
    SciRustSlhaTile a[3];
    printf("%u %zu %zu %zu\\n", SLHA_TILE_ALIGN, sizeof(SciRustSlhaTile),
           (size_t)((char*)&a[1] - (char*)&a[0]), (size_t)offsetof(SciRustSlhaTile, group_scales));
    return (int)((unsigned long long)(size_t)a % SLHA_TILE_ALIGN);
}
""")
    exe = tmp_path / "t"
    cc = "gcc" if lang == "c" else "g++"
    std = "-std=c11" if lang == "c" else "-std=c++17"
    cmd = [cc, std, "-Wall", "-Werror", "-I", str(ROOT / "include"), str(src), "-o", str(exe)]
    if line128:
        cmd.insert(1, "-DSLHA_CACHE_LINE_128=1")
    subprocess.run(cmd, check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0
    assert r.stdout.split() == [str(128 if line128 else 64), "128", "128", "120"]


def test_null_pointer_errors_leave_outputs_untouched():
    out = np.full(1, 42.0, np.float32)
    rc = s.lib.slha_process_tile(None, None, None, out.ctypes.data)
    assert rc == s.ERR_NULL and "NULL" in s.last_error() and out[0] == 42.0
    rc = s.lib.slha_score_tiles(None, None, 0, None, None, None)
    assert rc == s.ERR_NULL
    s.lib.slha_clear_error()
    assert s.last_error() == ""


def test_handle_errors():
    m = s.Model(1)
    h = m.handle
    m.release()
    qc = np.zeros(128, np.float32)
    qs = np.zeros(4, np.uint64)
    tile = np.zeros(1, s.TILE_DTYPE)
    out = np.zeros(1, np.float32)
    rc = s.lib.slha_score_tile(h, tile.ctypes.data, qc.ctypes.data, qs.ctypes.data, out.ctypes.data)
    assert rc == s.ERR_INVALID_HANDLE and "not a live" in s.last_error()
    assert s.lib.slha_weights_release(h) == s.ERR_INVALID_HANDLE
    assert s.lib.slha_weights_release(None) == s.OK
    s.lib.slha_weights_free(None)
    assert s.lib.slha_model_dim(h) == 0
    assert s.lib.slha_model_dim(None) == 0 and "NULL" in s.last_error()
    bogus = ctypes.c_uint64(0)
    assert s.lib.slha_model_dim(ctypes.addressof(bogus)) == 0
    assert s.lib.slha_weights_release(ctypes.addressof(bogus) + 1) == s.ERR_INVALID_HANDLE


def test_context_contract():
    ctx = s.lib.slha_init()
    assert ctx and s.lib.slha_init() == ctx
    assert s.lib.slha_shutdown(ctx) == s.OK
    assert s.lib.slha_shutdown(None) == s.OK
    assert s.lib.slha_shutdown(ctx + 8) == s.ERR_INVALID_HANDLE


def test_weights_load_errors():
    assert not s.lib.slha_weights_load(None) and "NULL" in s.last_error()
    assert not s.lib.slha_weights_load(b"\xff\xfe.slhw") and "UTF-8" in s.last_error()
    assert not s.lib.slha_weights_load(b"/nonexistent/model.slhw")
    assert "weights: cannot stat /nonexistent/model.slhw" in s.last_error()


def test_dimension_and_codec_errors_precede_any_device_work():
    with s.Model(3) as m:
        key = np.zeros(64, np.float32)
        out = np.zeros(1, s.TILE_DTYPE)
        rc = s.lib.slha_encode_key(m.handle, key.ctypes.data, 64, 0, 0, out.ctypes.data)
        assert rc == s.ERR_DIMENSION and "received 64, expected 128" in s.last_error()
        key = np.zeros(128, np.float32)
        rc = s.lib.slha_encode_key(m.handle, key.ctypes.data, 128, 0, 9, out.ctypes.data)
        assert rc == s.ERR_CODEC
        key[5] = np.nan
        rc = s.lib.slha_encode_key(m.handle, key.ctypes.data, 128, 0, 1, out.ctypes.data)
        assert rc == s.ERR_NONFINITE and "key[5]" in s.last_error()
        big = 1 << 20
        rc = s.lib.slha_score_tiles(m.handle, out.ctypes.data, big + 1, key.ctypes.data,
                                    key.ctypes.data, key.ctypes.data)
        assert rc == s.ERR_DIMENSION and "safety bound" in s.last_error()
        assert s.lib.slha_score_tiles(m.handle, out.ctypes.data, 0, key.ctypes.data,
                                      key.ctypes.data, key.ctypes.data) == s.OK
        bad = np.zeros(1, s.TILE_DTYPE)
        bad["flags"] = 2 | 4
        qc = np.zeros(128, np.float32)
        qs = np.zeros(4, np.uint64)
        sc = np.full(1, 7.0, np.float32)
        rc = s.lib.slha_score_tiles(m.handle, bad.ctypes.data, 1, qc.ctypes.data, qs.ctypes.data,
                                    sc.ctypes.data)
        assert rc == s.ERR_INVALID_TILE and "more than one" in s.last_error() and sc[0] == 7.0


@pytest.mark.parametrize("seed,rht", [(0, False), (77, True), (2**63 + 5, True)])
def test_model_projection_matches_reference_generator(seed, rht):
    # scenario.rs:59-64 (Z = fill_gaussian, row-major), learned.rs:158-165 +
    # incoherence.rs:89-98 (diag from seed ^ 0xA2..A2). The product's own
    # generator must reproduce the oracle's stream bit for bit.
    with s.Model(seed, rht=rht) as m:
        z, diag = m.projection()
        assert m.dim == 128
    assert np.array_equal(z, o.projection(seed))
    want = o.rht_diag(seed ^ 0xA2A2A2A2A2A2A2A2) if rht else np.ones(128, np.float32)
    assert np.array_equal(diag, want)


def test_bad_residual_mode():
    with pytest.raises(s.SlhaError):
        s.Model(0, residual_mode=7)
