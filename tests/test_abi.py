"""CPU-side checks of the drop-in boundary: the C-ABI library loads and exports every symbol that
include/yalm_hip.h declares (no device calls are made)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols(name):
    text = open(os.path.join(ROOT, "include", name)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(yhip_[a-z_0-9]+)\s*\(", text)))


def test_hip_library_exports_every_declared_symbol():
    from yalm_amd import hip as H
    assert os.path.exists(H.LIB_PATH), "build first: python -c 'import __graft_entry__ as g; g.build()'"
    lib = ctypes.CDLL(H.LIB_PATH)
    declared = header_symbols("yalm_hip.h")
    assert len(declared) >= 15
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, missing
    assert sorted(H.EXPORTS) == declared


def test_hip_binding_signatures_load():
    from yalm_amd import hip as H
    H.lib()  # sets restype/argtypes for every entry point; no device call


def test_create_without_device_fails_cleanly():
    import torch  # noqa: F401  (device count only)
    if torch.cuda.device_count() > 0:
        pytest.skip("a GPU is visible")
    from yalm_amd import hip as H
    from tests.util import MICRO
    with pytest.raises(H.HipError):
        H.HipModel(dict(MICRO))


def header_arities(name):
    text = open(os.path.join(ROOT, "include", name)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"\b(yhip_[a-z_0-9]+)\s*\(([^)]*)\)\s*;", text):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_binding_argument_counts_match_header():
    from yalm_amd import hip as H
    L = H.lib()
    for name, n in header_arities("yalm_hip.h").items():
        assert len(getattr(L, name).argtypes) == n, name


def test_host_library_exports_and_binding_arities():
    from yalm_amd import host as HO
    lib = ctypes.CDLL(HO.LIB_PATH)
    text = open(os.path.join(ROOT, "include", "yalm_host.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decl = {m.group(1): (0 if m.group(2).strip() in ("", "void") else m.group(2).count(",") + 1)
            for m in re.finditer(r"\b(yalm_[a-z_0-9]+)\s*\(([^)]*)\)\s*;", text)}
    assert sorted(decl) == sorted(HO.EXPORTS)
    L = HO.lib()
    for name, n in decl.items():
        assert hasattr(lib, name), name
        assert len(getattr(L, name).argtypes) == n, name
