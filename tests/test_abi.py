"""CPU: the C-ABI library loads, exports every function the header declares, and
its host-only entry points (version, status strings, size queries, argument
checks) behave as documented.  No call here launches GPU work: every call
either queries sizes or fails its argument check before touching the device."""
import ctypes
import os
import re

import pytest

from g2ptq_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "g2ptq_hip.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(g2ptq_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_header_declares_the_entry_points():
    names = header_functions()
    assert len(names) >= 29
    assert "g2ptq_compensate" in names and "g2ptq_inv_chol_upper" in names


def test_library_exports_every_header_symbol(lib):
    raw = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in header_functions() if not hasattr(raw, n)]
    assert not missing, missing


def test_bindings_cover_exactly_the_header(lib):
    assert sorted(set(_lib.SIGNATURES) | set(_lib.STRING_FUNCS)) == header_functions()


def test_abi_version_and_status_strings(lib):
    assert lib.g2ptq_abi_version() == 1
    for code in (0, -1, -2, -3, -4):
        s = lib.g2ptq_status_string(code)
        assert s and isinstance(s, bytes)
    assert lib.g2ptq_status_string(0) != lib.g2ptq_status_string(-1)


def test_size_queries(lib):
    assert _lib.query_size("g2ptq_factor_workspace", 2, 4096) >= 2 * 4096 * 4096 * 4
    assert _lib.query_size("g2ptq_compensate_workspace", 0, 2, 4096, 4096, 128) >= 2 * 4096 * 128 * 4
    assert _lib.query_size("g2ptq_trust_region_workspace", 4, 256, 4096) > 0
    assert _lib.query_size("g2ptq_hessian_workspace", 8192, 4096, 0, 0) > 0
    assert _lib.query_size("g2ptq_hessian_gram_workspace", 32768, 4096) >= 0
    # GPTAQ stages 3 planes and the weighted update Xᵀ plus G weight rows; both
    # need split partials (the weighted ones for all G groups)
    h = _lib.query_size("g2ptq_hessian_workspace", 8192, 4096, 0, 0)
    assert _lib.query_size("g2ptq_hessian_workspace", 8192, 4096, 1, 0) > h
    assert (_lib.query_size("g2ptq_hessian_workspace", 8192, 4096, 2, 4)
            > _lib.query_size("g2ptq_hessian_workspace", 8192, 4096, 2, 1))
    assert _lib.query_size("g2ptq_gptaq_gram_workspace", 32768, 4096) > 0
    assert (_lib.query_size("g2ptq_weighted_gram_workspace", 32768, 4096, 4)
            > _lib.query_size("g2ptq_weighted_gram_workspace", 32768, 4096, 1) > 0)
    rows = _lib.query_size_i64("g2ptq_hessian_stage_rows", 4096)
    assert rows >= 4096 and rows % 256 == 0
    # any-dtype staging: Xᵀ takes 1 / 2 / 3 bf16 planes for bf16 / fp16 / fp32
    planes = lambda kind, dt, G=0: _lib.query_size_i64("g2ptq_hessian_stage_planes", kind, dt, G)
    assert [planes(0, dt) for dt in (0, 1, 2)] == [1, 2, 3]
    assert [planes(1, dt) for dt in (0, 1, 2)] == [3, 4, 5]
    assert [planes(2, dt, 4) for dt in (0, 1, 2)] == [1, 10, 11]
    # buffer heights in rows of bf16: planes × rows, and the bf16 weighted
    # kind's G fp32 weight rows (2G bf16 rows)
    height = lambda kind, dt, G=0: _lib.query_size_i64("g2ptq_hessian_stage_height", kind, dt,
                                                       4096, G)
    assert [height(0, dt) for dt in (0, 1, 2)] == [rows, 2 * rows, 3 * rows]
    assert height(1, 0) == 3 * rows
    assert [height(2, dt, 4) for dt in (0, 1, 2)] == [rows + 8, 10 * rows, 11 * rows]
    ex = lambda kind, dt: _lib.query_size("g2ptq_hessian_gram_ex_workspace", kind, dt, 32768, 4096,
                                          4 if kind == 2 else 0)
    assert ex(0, 0) == _lib.query_size("g2ptq_hessian_gram_workspace", 32768, 4096)
    assert ex(1, 0) == _lib.query_size("g2ptq_gptaq_gram_workspace", 32768, 4096)
    assert ex(2, 0) == _lib.query_size("g2ptq_weighted_gram_workspace", 32768, 4096, 4)
    assert ex(0, 1) > 0 and ex(0, 2) > 0


@pytest.mark.parametrize("call", [
    ("g2ptq_find_params", (None, None, 4, 4, 4, 4, 1, None, None, 1, None)),
    ("g2ptq_find_params", (None, None, 4, 4, 4, 17, 1, None, None, 1, None)),
    ("g2ptq_weighted_gram", (None, None, 64, 0, 128, 0, 1.0, 0.0, None, 128, 0, None, 0)),
    ("g2ptq_gptaq_stage", (None, None, None, 8, 128, 128, 128, None, 64, 0)),
    ("g2ptq_hessian_stage_planes", (0, 3, 0, None)),
    ("g2ptq_hessian_stage_height", (2, 0, 4096, 0, None)),
    ("g2ptq_weighted_gram_workspace", (4096, 4096, 0, None)),
    ("g2ptq_hessian_stage_ex", (None, 0, 5, None, None, 8, 128, 128, 128, None, 0, 0, 1.0, None,
                                64, 0, None, 0.0, 1.0)),
    ("g2ptq_hessian_stage_ex", (None, 1, 1, None, None, 8, 128, 128, 128, None, 0, 0, 1.0, None,
                                64, 0, None, 0.0, 1.0)),
])
def test_argument_errors_return_arg_status(lib, call):
    name, args = call
    fn = getattr(lib, name)
    assert fn(*args) == -1
    assert lib.g2ptq_last_error()


def test_call_raises_value_error_on_bad_arguments(lib):
    with pytest.raises(ValueError):
        _lib.call("g2ptq_find_params", None, None, 4, 4, 4, 4, 1, None, None, 1, None)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    """The product path has no fallback: a missing library is an error."""
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "absent.so"))
    monkeypatch.setattr(_lib, "_LIB", None)
    with pytest.raises(_lib.HipLibraryError):
        _lib.load()


def test_fastcall_module_binds_the_same_entry_point(lib):
    """The CPython fast-call module is built with the library, shares its one
    loaded copy (one status and error state), and reports argument errors as
    the ctypes binding does."""
    fast = _lib.fastcall()
    assert fast is not None, "g2ptq_amd/_fastcall is not built"
    maps = [l for l in open("/proc/self/maps") if "libg2ptq_hip.so" in l and "r-xp" in l]
    assert len(maps) == 1
    with pytest.raises(TypeError):
        fast.hessian_stage(0, 0, 1)
    status = fast.hessian_stage(None, None, 4, 8, 8, None, 8, 0)  # no XT: argument error
    assert status == -1
    assert b"hessian_stage" in lib.g2ptq_last_error()
    with pytest.raises(ValueError, match="hessian_stage: bad arguments"):
        _lib.raise_status("g2ptq_hessian_stage", status)
