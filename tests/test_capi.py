"""The C ABI library loads and exports every entry point of include/hisparse.h (no GPU needed),
and the product never reaches the CPU oracle."""

import ctypes
import os
import re
import shutil
import subprocess
import sys
from textwrap import dedent

import pytest

from mini_hisparse_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hisparse.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hs_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_expected_entry_points():
    names = declared_functions()
    for required in ("hs_quest_topk", "hs_build_union", "hs_resolve_rows", "hs_resolve_rows_batched",
                     "hs_gather_rows", "hs_gather_rows_batched", "hs_attend_rows", "hs_attend_groups", "hs_attend_window",
                     "hs_host_alias", "hs_last_error"):
        assert required in names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert lib.hs_version() == 1


def test_dynamic_symbol_table_holds_only_the_c_api():
    """Every global symbol the library defines is a declared hs_* entry point: kernel
    handles, device stubs, device variables and per-file ids stay local, so two copies of
    the library in one process cannot meet each other's names."""
    if not shutil.which("readelf"):
        pytest.skip("readelf is not installed")
    out = subprocess.run(["readelf", "--dyn-syms", "-W", str(_lib.LIBRARY_PATH)], capture_output=True, text=True,
                         check=True).stdout
    defined = set()
    for line in out.splitlines():
        parts = line.split()
        if len(parts) >= 8 and parts[4] in ("GLOBAL", "WEAK") and parts[6] != "UND":
            defined.add(parts[7])
    assert defined and defined == set(declared_functions())


def test_descriptor_layout_matches_the_header(tmp_path):
    """Field offsets of hs_resolve_desc as a C compiler lays it out == the ctypes mirror."""
    fields = [name for name, _ in _lib.ResolveDesc._fields_]
    source = tmp_path / "layout.c"
    source.write_text(
        "#include <stdio.h>\n#include <stddef.h>\n#include \"hisparse.h\"\nint main(void){\n"
        + 'printf("%zu\\n", sizeof(hs_resolve_desc));\n'
        + "".join(f'printf("%zu\\n", offsetof(hs_resolve_desc, {f}));\n' for f in fields)
        + "return 0;}\n"
    )
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(source), "-o", str(exe)], check=True)
    values = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    assert values[0] == ctypes.sizeof(_lib.ResolveDesc)
    assert values[1:] == [getattr(_lib.ResolveDesc, f).offset for f in fields]


def test_host_queries_and_argument_errors_without_a_gpu():
    lib = _lib.load()
    assert lib.hs_resolve_workspace_bytes(1000, 4096, 256, 512) > 0
    assert lib.hs_quest_workspace_bytes(2, 8, 100) >= 2 * 8 * 100 * 4
    assert lib.hs_attend_workspace_bytes(2, 1, 8, 2, 64, 100) > 0
    assert lib.hs_resolve_noalloc_max_bytes() == 32 << 20
    desc = _lib.ResolveDesc()  # all null: rejected on the host, before any launch
    assert lib.hs_resolve_rows(desc, None, 0, None) == -1
    assert b"nonempty" in lib.hs_last_error()
    status = lib.hs_attend_rows(None, 0, 0, None, 7, 16, 8, 128, 0, None, 0, 0, 0, 1, 1, 64, None, 0, 0, None, 0, None)
    assert status == -1 and b"dtype" in lib.hs_last_error()


def _fake_resolve_desc(hot_rows=64, lru_i16=0):
    """A descriptor that passes the null and shape checks (pointers are never dereferenced
    on the host: every case below is rejected before any launch)."""
    d = _lib.ResolveDesc()
    for i, name in enumerate(("positions", "source", "resident", "hot", "tags", "lru", "physical",
                              "miss_host_rows", "miss_device_rows", "counts")):
        setattr(d, name, 0x10000 * (i + 1))
    d.n, d.length, d.page_size, d.n_pages = 8, 64, 16, 4
    d.hot_rows, d.hot_blocks, d.lru_i16 = hot_rows, (hot_rows + 15) // 16, lru_i16
    return d


def test_resolver_lru_dtype_rules_without_a_gpu():
    """int16 LRU tables: the flag is 0 or 1, hot_rows even (pairs per 32-bit load), one
    dtype per batch; all rejected on the host."""
    lib = _lib.load()
    assert lib.hs_resolve_rows(_fake_resolve_desc(lru_i16=2), None, 0, None) == -1
    assert b"lru_i16 must be 0 or 1" in lib.hs_last_error()
    assert lib.hs_resolve_rows(_fake_resolve_desc(hot_rows=63, lru_i16=1), None, 0, None) == -1
    assert b"even hot_rows" in lib.hs_last_error()
    pair = (_lib.ResolveDesc * 2)(_fake_resolve_desc(lru_i16=1), _fake_resolve_desc(lru_i16=0))
    assert lib.hs_resolve_rows_batched(pair, 2, None, 0, None) == -1
    assert b"share lru_i16" in lib.hs_last_error()
    # a valid batch gets as far as the workspace check
    same = (_lib.ResolveDesc * 2)(_fake_resolve_desc(lru_i16=1), _fake_resolve_desc(lru_i16=1))
    assert lib.hs_resolve_rows_batched(same, 2, None, 0, None) == -1
    assert b"workspace too small" in lib.hs_last_error()


def test_rotary_split_append_argument_errors_without_a_gpu():
    """Rejected on the host before any launch: a bad shape, a device row outside the
    pool, a host row without its host alias."""
    from ctypes import c_int64, c_void_p

    lib = _lib.load()
    rows = (c_int64 * 2)(0, 5)
    host = (c_int64 * 2)(3, 4)
    alias = (c_void_p * 2)(0x1000, 0x2000)
    bounds = (c_void_p * 2)(0x3000, 0x4000)
    p = [0x10000 * i for i in range(1, 7)]

    def call(head_dim=64, dev=rows, alias_=alias, pool_rows=16):
        return lib.hs_rotary_split_append(p[0], (8 + 4) * head_dim, p[1], p[2], p[3], p[4], 2, 8, 2, head_dim, 1e6,
                                          2, p[5], pool_rows, 16, dev, alias_, host, 64, bounds, bounds, None)

    assert call(head_dim=63) == -1 and b"invalid rotary shape" in lib.hs_last_error()
    assert call(pool_rows=4) == -1 and b"outside the pool" in lib.hs_last_error()
    assert call(alias_=None) == -1 and b"host alias" in lib.hs_last_error()


def test_resolver_split_front_rules_without_a_gpu():
    """The split front needs a union page bitmap and a power-of-two page of at most 32
    tokens, and one setting per batch; all rejected on the host."""
    lib = _lib.load()

    def split(page_bits=0x90000, page_size=16, flag=1):
        d = _fake_resolve_desc(lru_i16=1)
        d.page_bits, d.page_size, d.split_front = page_bits, page_size, flag
        d.length = min(d.length, page_size * d.n_pages)
        return d

    assert lib.hs_resolve_rows(split(flag=2), None, 0, None) == -1
    assert b"split_front must be 0 or 1" in lib.hs_last_error()
    for bad in (split(page_bits=None), split(page_size=12), split(page_size=64)):
        assert lib.hs_resolve_rows(bad, None, 0, None) == -1
        assert b"split_front needs a union page bitmap" in lib.hs_last_error()
    mixed = (_lib.ResolveDesc * 2)(split(), split(flag=0))
    assert lib.hs_resolve_rows_batched(mixed, 2, None, 0, None) == -1
    assert b"share split_front" in lib.hs_last_error()
    same = (_lib.ResolveDesc * 2)(split(), split())
    assert lib.hs_resolve_rows_batched(same, 2, None, 0, None) == -1
    assert b"workspace too small" in lib.hs_last_error()


def test_union_page_bitmap_stride_checked_without_a_gpu():
    lib = _lib.load()
    lengths = (ctypes.c_int64 * 1)(4096)  # 256 pages: 8 bitmap words
    args = [0x1000, 64, 8, lengths, 16, 1, 8, 2, 0x2000, 4096, 0x3000, 128, 0x4000, 0x5000, 0x6000, 4096,
            0x7000, 0x8000]
    assert lib.hs_build_union(*args, 0x9000, 7, None, None) == -1
    assert b"page bitmap stride" in lib.hs_last_error()


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(_lib.HipLibraryError, match="missing"):
        _lib.load(tmp_path / "libhisparse_hip.so")


def test_a_second_copy_of_the_library_is_refused(tmp_path):
    import shutil

    _lib.load()
    copy = tmp_path / "libhisparse_hip.so"
    shutil.copy(_lib.LIBRARY_PATH, copy)
    with pytest.raises(_lib.HipLibraryError, match="second copy"):
        _lib.load(copy)
    assert _lib.load(_lib.LIBRARY_PATH) is _lib.load()


def test_loaded_library_is_returned_without_a_filesystem_lookup(monkeypatch):
    """Every kernel wrapper calls ``load()`` once per launch: once the package's build is
    loaded, the call must not resolve paths (a path lookup per launch made a decode step
    of ~400 launches host-bound)."""
    lib = _lib.load()

    def no_lookup(self, *args, **kwargs):
        raise AssertionError("load() looked the library path up again")

    monkeypatch.setattr(_lib.Path, "resolve", no_lookup)
    assert _lib.load() is lib


def test_product_runs_without_the_oracle_or_tests_packages():
    program = dedent("""
        import importlib.abc, sys
        class Blocked(importlib.abc.MetaPathFinder):
            def find_spec(self, fullname, path=None, target=None):
                if fullname.split('.')[0] in {'oracle', 'tests'}:
                    raise ImportError('product imported test infrastructure: ' + fullname)
        sys.meta_path.insert(0, Blocked())
        import mini_hisparse_amd, mini_hisparse_amd.engine, mini_hisparse_amd.cli, mini_hisparse_amd.batched
        import mini_hisparse_amd.ops, mini_hisparse_amd.model
        print('ok')
    """)
    result = subprocess.run([sys.executable, "-c", program], cwd=ROOT, capture_output=True, text=True, timeout=120)
    assert result.returncode == 0, result.stderr
    assert result.stdout.strip() == "ok"
