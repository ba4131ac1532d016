"""The boundary from C: tests/c_abi/abi_harness is compiled against include/rad_abi.h and
include/r3d_gfx950.h and linked against the built library, so a header prototype or an
export that drifted from the binary fails its build.  Here its view of the ABI is held
against the ctypes mirror (libr3d_amd) the other tests call through -- field offsets and
sizes of every structure, the row table, the schemas -- and, on a GPU, it launches one
decode and one prefill row by hand-built RadArgs and checks them against the oracle."""
import json
import os
import subprocess

import pytest

import libr3d_amd as R

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HARNESS = os.path.join(ROOT, "tests", "c_abi", "abi_harness")

MIRRORS = ["RadTensor", "RadParam", "RadTunableValue", "RadTunable", "RadArgs", "RadConstraint",
           "RadKernelInfo", "RadParamSpec", "RadOperandSpec", "RadOpSchema", "RadPluginInfo",
           "RadEncPlane", "RadEncoding", "RadLayout", "RadPlanesHeader", "RadPlanesEntry"]


def _harness(mode, timeout=60):
    if not os.path.exists(HARNESS):
        pytest.fail("tests/c_abi/abi_harness is not built (run __graft_entry__.build())")
    return subprocess.run([HARNESS, mode], capture_output=True, text=True, timeout=timeout)


def test_c_layout_matches_ctypes_mirror():
    out = _harness("layout")
    assert out.returncode == 0, out.stderr
    lay = json.loads(out.stdout)
    import ctypes
    seen = set()
    for key, val in lay.items():
        if key == "RAD_MAX_RANK":
            assert val == R.RAD_MAX_RANK
            continue
        if key.startswith("sizeof."):
            name = key.split(".", 1)[1]
            assert ctypes.sizeof(getattr(R, name)) == val, key
            seen.add(name)
            continue
        name, field = key.split(".")
        f = getattr(getattr(R, name), field)
        assert [f.offset, f.size] == val, (key, f.offset, f.size, val)
    assert seen == set(MIRRORS)
    # every field of every mirror was compared (the C side lists all of them)
    for name in MIRRORS:
        fields = [f[0] for f in getattr(R, name)._fields_]
        assert all("%s.%s" % (name, f) in lay for f in fields), name


def test_c_table_matches_python_view():
    out = _harness("table")
    assert out.returncode == 0, out.stderr
    t = json.loads(out.stdout)
    assert t["abi"] == 26 and t["plugin"] == [1, "libr3d_gfx950", "gfx950"]
    assert t["build_id"] == R.build_id()
    assert [s[0] for s in t["schemas"]] == [s["op"] for s in R.schemas()]
    assert [[s["op"], len(s["params"]), len(s["operands"])] for s in R.schemas()] == t["schemas"]
    rows = R.rows()
    assert [r[0] for r in t["rows"]] == [r["name"] for r in rows]
    for c, p in zip(t["rows"], rows):
        assert c[1:] == [p["op"], p["priority"], len(p["constraints"]), 1]


def test_c_harness_calls_the_layout_hooks():
    """The logits row's hooks through RadKernelInfo from C, with a hand-built RadEncoding:
    layout / relayout / unrelayout on an accepted head, and the declines."""
    out = _harness("hooks")
    assert out.returncode == 0 and out.stdout.strip() == "PASS", out.stdout + out.stderr


def test_library_built_from_this_tree():
    """The loaded binary reports the SHA-256 of the sources it was compiled from; it must
    be the tree's (a stale library would test other code than the tree holds)."""
    R.check_build_id()


@pytest.mark.gpu
def test_c_harness_launches_rows(gpu):
    out = _harness("run", timeout=120)
    print(out.stdout)
    assert out.returncode == 0 and out.stdout.strip().endswith("PASS"), out.stdout + out.stderr
