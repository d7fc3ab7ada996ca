"""CPU checks of the C-ABI library: it loads without a GPU and exports every
symbol its public headers declare."""
import os
import re

from bnneon import hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b((?:bnh|bnn)_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    L = hip.lib()
    for header in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if not header.endswith(".h"):
            continue
        missing = [n for n in declared(header) if not hasattr(L, n)]
        assert not missing, (header, missing)


def test_binding_covers_the_kernel_abi():
    assert set(declared("bnneon_hip.h")) <= set(hip._SIGS)


def test_no_device_is_an_error_not_a_crash():
    L = hip.lib()
    if L.bnh_device_count() == 0:
        assert L.bnh_malloc(16) is None
        assert b"hipMalloc" in L.bnh_last_error()
