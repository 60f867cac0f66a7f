"""The C-ABI libraries load and export every function their headers declare
(no compute calls: this suite runs without a GPU)."""
import ctypes as C
import os
import re

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header):
    text = open(os.path.join(REPO, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b(n[a-z0-9_]+)\s*\(", text)
    return sorted({n for n in names if n.startswith(("nda_", "nd_gpu_", "ndp_"))})


def test_nda_exports_every_declared_symbol():
    import ndattn
    names = declared("nda.h")
    assert len(names) >= 30
    assert sorted(ndattn.ABI_SYMBOLS) == names
    lib = C.CDLL(ndattn.LIB_PATH)
    for n in names:
        assert hasattr(lib, n), n


def test_host_shim_exports_every_declared_symbol():
    import ndattn
    names = declared("nd_attn_gpu.h")
    assert sorted(ndattn.HOST_SYMBOLS) == names
    lib = C.CDLL(ndattn.HOST_LIB_PATH)
    for n in names:
        assert hasattr(lib, n), n


def test_probe_exports_every_declared_symbol():
    import ndattn
    names = declared("ndp.h")
    assert sorted(ndattn.PROBE_SYMBOLS) == names
    lib = C.CDLL(ndattn.PROBE_LIB_PATH)
    for n in names:
        assert hasattr(lib, n), n


def test_libraries_carry_gfx950_code():
    import ndattn
    blob = open(ndattn.LIB_PATH, "rb").read()
    assert b"gfx950" in blob


def test_config_struct_matches_header():
    """Field order and size of nda_config as the header lays it out."""
    import ndattn
    assert C.sizeof(ndattn.Config) == 4 * 10 + 8 + 4 * 2
    text = open(os.path.join(REPO, "include", "nda.h")).read()
    body = text[text.index("typedef struct {", text.index("Geometry and capacities")):]
    body = body[:body.index("} nda_config;")]
    fields = re.findall(r"uint(?:32|64)_t\s+(\w+);", body)
    assert fields == [f[0] for f in ndattn.Config._fields_]


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU is present")
def test_create_without_gpu_reports_nodev():
    import ndattn
    with pytest.raises(ndattn.NdaError) as e:
        ndattn.Context(1, 8, 8, 64, 64, 64)
    assert e.value.code == -7
