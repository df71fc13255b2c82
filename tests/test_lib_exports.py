"""The HIP library loads and exports every function include/*.h declares
(no GPU needed: nothing is called)."""
import ctypes
import glob
import os
import re

from desireeia_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        for m in re.finditer(r"\b([A-Za-z_][A-Za-z0-9_]*)\s*\(", text):
            name = m.group(1)
            before = text[:m.start()].rstrip()
            if before.endswith(("#define", "sizeof")) or name in ("if", "while", "for", "return", "sizeof"):
                continue
            # a declaration: preceded by a type token at statement level
            line = text[text.rfind("\n", 0, m.start()) + 1:m.start()]
            if line.lstrip().startswith("#"):
                continue
            if re.search(r"(int|void|float|size_t|uint32_t|int32_t|int64_t|uint64_t|bool|char)\s*\**\s*$", line):
                names.add(name)
    return names


def test_header_declares_functions():
    names = declared_functions()
    assert "dq_gemv" in names and "dq_dequantize_row" in names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    missing = [n for n in sorted(declared_functions()) if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_covers_header():
    assert declared_functions() <= set(_lib.SIGNATURES), declared_functions() - set(_lib.SIGNATURES)


def test_no_oracle_in_product_library():
    # the product library must not depend on the CPU checker
    import subprocess
    out = subprocess.run(["nm", "-D", _lib.LIB_PATH], capture_output=True, text=True).stdout
    assert "dqo_" not in out and "dqr_" not in out


def test_lds_probe_patterns():
    """bench.lds_probe_patterns: 64 in-range, 16-byte aligned offsets each;
    in a quad-pair pattern only quads i and j touch the first 16 banks, at
    different addresses, and every other lane reads one address per slot."""
    import bench
    pats = dict(bench.lds_probe_patterns())
    assert len(pats) == 39
    for name, offs in pats.items():
        assert len(offs) == 64 and all(0 <= o <= 65536 - 16 and o % 16 == 0 for o in offs), name
    for i, j in ((0, 3), (1, 2), (0, 15)):
        offs = pats[f"quads({i},{j})"]
        low = sorted({l // 4 for l in range(64) if offs[l] % 256 < 64})
        assert low == [i, j]
        assert {offs[4 * i + l] for l in range(4)}.isdisjoint({offs[4 * j + l] for l in range(4)})
        assert {offs[l] for l in range(64) if l // 4 not in (i, j)} == {64, 80, 96, 112}
