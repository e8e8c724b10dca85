"""The C-ABI library: it loads without a GPU and exports every function include/*.h declares
(no compute calls are made here)."""
import ctypes as C
import os
import re

import glm53h

INC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include")


def declared_functions():
    names = set()
    for f in os.listdir(INC):
        if not f.endswith(".h"):
            continue
        src = open(os.path.join(INC, f)).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        for m in re.finditer(r"^(?!\s*static)(?!\s*#)[^;{}()]*?\b((?:glm53f|g53h)_\w+)\s*\(", src, re.M):
            if "typedef" in m.group(0) or "(*" in m.group(0):
                continue
            names.add(m.group(1))
    return sorted(names)


def test_library_loads_and_exports_all_declared_symbols():
    L = C.CDLL(glm53h.LIB_PATH)
    names = declared_functions()
    assert len(names) > 30
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_declared_globals_exported():
    L = C.CDLL(glm53h.LIB_PATH)
    assert C.c_long.in_dll(L, "glm53f_expert_drops").value >= 0
    assert C.c_int.in_dll(L, "glm53f_quiet").value in (0, 1)
    assert C.c_char_p.in_dll(L, "glm53f_i4_dir").value is None


def test_python_mirror_covers_the_abi():
    """Every declared function has a ctypes signature in the host binding."""
    missing = [n for n in declared_functions() if n not in glm53h.exported_names()]
    assert not missing, missing


def test_struct_layouts_match_c():
    # sizes computed from the C declarations (x86-64 LP64)
    assert C.sizeof(glm53h.G53hMat) == 40
    assert C.sizeof(glm53h.G53hExpert) == 120
    assert C.sizeof(glm53h.Glm53fMat) == 40
    assert C.sizeof(glm53h.Glm53fExpertSrc) == 40
