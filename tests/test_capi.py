"""CPU-side checks of the C ABI: the library loads without a GPU, exports
every function include/krunch_hip.h declares, and the ctypes table binds
exactly those; size queries work without a device."""
import os
import re

from krunch_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                      "include", "krunch_hip.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kr_[a-z0-9_]+)\s*\(", text)))


def test_header_symbols_exported_and_bound():
    names = declared()
    assert len(names) >= 25
    L = _lib.lib()
    for n in names:
        assert hasattr(L, n), f"{n} not exported"
    assert sorted(_lib.exported_symbols()) == names


def test_size_queries_without_device():
    L = _lib.lib()
    assert L.kr_state_bytes(12, 1, 768) == 147456          # 12 layers x 12288 B/stream
    assert L.kr_forward_workspace_bytes(1024, 768, 3072) >= 1024 * 768 * (8 * 2 + 2 * 4) + 1024 * 3072 * 2
    assert L.kr_abi_version() == 2


def test_argument_errors_are_reported():
    rc = _lib.lib().kr_probs_to_cdf(None, 1, 10, 10, None, 24, None)
    assert rc != 0
    assert b"null" in _lib.lib().kr_last_error()
