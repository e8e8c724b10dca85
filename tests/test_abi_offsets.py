"""The shared structs field for field: tests/golden/offsets.json holds sizeof/offsetof of every
field of Glm53fCfg, Glm53fMat, Glm53fExpertQ, Glm53fExpertSrc, Glm53fMoeW, Glm53fCache,
Glm53fSt and Glm53fTensor compiled against the reference's headers
(tests/golden/make_offsets.py). The same probe compiled against include/ must print the same
numbers, so the reference's callers (e.g. src/model/glm53f_model.c:177-233 reading
cache.nslot / slot_bytes / i4_layers, src/cli/glm53f_run.c:485-489 reading the statistics)
work unchanged against this library; the Python mirror must agree too."""
import ctypes as C
import json
import os
import shutil
import sys

import pytest

import glm53h

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_offsets as MO  # noqa: E402

INC = os.path.join(os.path.dirname(HERE), "include")
GOLD = json.load(open(os.path.join(HERE, "golden", "offsets.json")))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="no C compiler")
def test_headers_match_reference_offsets():
    got = MO.offsets([INC])
    assert set(got) == set(GOLD)
    for s in GOLD:
        for f, v in GOLD[s].items():
            assert got[s][f] == v, (s, f, got[s][f], v)


@pytest.mark.parametrize("name", ["Glm53fCfg", "Glm53fMat", "Glm53fExpertQ", "Glm53fExpertSrc", "Glm53fMoeW",
                                  "Glm53fCache", "Glm53fSt", "Glm53fTensor"])
def test_python_mirror_matches_reference_offsets(name):
    cls = getattr(glm53h, name)
    assert C.sizeof(cls) == GOLD[name]["sizeof"]
    for f, v in GOLD[name].items():
        if f == "sizeof":
            continue
        assert getattr(cls, f).offset == v, (name, f)
