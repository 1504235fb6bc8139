"""The C-ABI library: it loads without a GPU, exports every function include/mxq_hip.h declares, and the host
side's argument table covers exactly those functions.  No compute calls (they need a GPU)."""
import ctypes
import os
import re

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "mxq_hip.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return sorted(set(re.findall(r"\b(mxq_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = _declared()
    assert "mxq_systolic" in names and "mxq_block_quantize" in names and "mxq_lut_tables" in names
    assert len(names) >= 19


def test_library_exports_every_declared_symbol():
    from mxq import _lib
    lib = _lib.load()
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, f"declared in include/mxq_hip.h but not exported: {missing}"


def test_signature_table_matches_header():
    from mxq import _lib
    assert sorted(_lib.SIGNATURES) == _declared()


def test_version_and_error_without_gpu():
    """mxq_version and mxq_last_error touch no device."""
    from mxq import _lib
    lib = _lib.load()
    text = open(HEADER).read()
    assert f"#define MXQ_ABI_VERSION {_lib.ABI_VERSION}\n" in text
    assert lib.mxq_version() == _lib.ABI_VERSION
    lib.mxq_last_error.restype = ctypes.c_char_p
    assert isinstance(lib.mxq_last_error(), bytes)


def test_structs_match_header():
    """ctypes layouts of mxq_block_spec / mxq_arith_spec against the header's field lists."""
    from mxq import _lib
    text = open(HEADER).read()
    for struct, py in (("mxq_block_spec", _lib.BlockSpec), ("mxq_arith_spec", _lib.ArithSpec),
                       ("mxq_systolic_layout", _lib.SystolicLayout)):
        body = re.search(r"typedef struct " + struct + r"\s*\{(.*?)\}\s*" + struct + ";", text, flags=re.S).group(1)
        body = re.sub(r"/\*.*?\*/|//[^\n]*", "", body, flags=re.S)
        fields = [(t, n.strip()) for t, names in re.findall(r"\b(int32_t|float|double|int64_t)\s+([a-z_0-9, ]+);", body)
                  for n in names.split(",")]
        ctypes_of = {"int32_t": ctypes.c_int32, "float": ctypes.c_float, "double": ctypes.c_double,
                     "int64_t": ctypes.c_int64}
        assert [(n, ctypes_of[t]) for t, n in fields] == [(n, t) for n, t in py._fields_], struct


def test_struct_offsets_match_header(tmp_path):
    """Field offsets and sizes of every struct the host side passes, ctypes against the header compiled by gcc
    (pointer fields included)."""
    import subprocess

    from mxq import _lib
    structs = {"mxq_block_spec": _lib.BlockSpec, "mxq_arith_spec": _lib.ArithSpec,
               "mxq_systolic_layout": _lib.SystolicLayout, "mxq_systolic_hints": _lib.SystolicHints,
               "mxq_systolic_epilogue": _lib.SystolicEpilogue}
    lines = ['#include <stddef.h>', '#include <stdio.h>', '#include "mxq_hip.h"', "int main(void) {"]
    for name, py in structs.items():
        lines.append(f'  printf("{name} size %zu\\n", sizeof({name}));')
        for f, _ in py._fields_:
            lines.append(f'  printf("{name} {f} %zu\\n", offsetof({name}, {f}));')
    lines.append("  return 0;\n}")
    src, exe = tmp_path / "offsets.c", tmp_path / "offsets"
    src.write_text("\n".join(lines))
    subprocess.run(["gcc", "-I", os.path.join(REPO, "include"), str(src), "-o", str(exe)], check=True)
    got = dict(line.rsplit(" ", 1) for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                                 check=True).stdout.splitlines())
    for name, py in structs.items():
        assert int(got[f"{name} size"]) == ctypes.sizeof(py), name
        for f, _ in py._fields_:
            assert int(got[f"{name} {f}"]) == getattr(py, f).offset, f"{name}.{f}"


def test_mfma_refuses_empty_contraction():
    """mxq_mx_mfma with K64 == 0 (or not a multiple of 64) returns MXQ_EINVAL before any HIP call: its kernel's
    prologue would read a K step that does not exist."""
    from mxq import _lib
    lib = _lib.load()
    lib.mxq_last_error.restype = ctypes.c_char_p
    buf = (ctypes.c_uint8 * 64)()
    out = (ctypes.c_float * 4)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    for K64 in (0, 32, -64):
        rc = lib.mxq_mx_mfma(p, p, 0, p, p, 0, ctypes.cast(out, ctypes.c_void_p), ctypes.c_int64(K64),
                             ctypes.c_int64(2), ctypes.c_int64(2), ctypes.c_void_p(0))
        assert rc == 1, K64
        assert b"K64" in lib.mxq_last_error()
