"""The C-ABI library loads on the CPU host and exports every entry point of the header."""
import os
import re

from omnimem_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header_functions():
    text = open(os.path.join(ROOT, "include", "omnimem_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(omm_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert _header_functions() == sorted(_lib.PROTOTYPES)


def test_library_exports_every_header_symbol():
    assert _lib.lib().omm_abi_version() == 4
    assert _lib.missing_symbols() == []


def test_library_binds_torch_hip_runtime():
    # the library's HIP dependency resolves to the runtime torch already loaded
    maps = open("/proc/self/maps").read()
    hip = {l.split()[-1] for l in maps.splitlines() if "libamdhip64" in l}
    assert len(hip) == 1, hip
