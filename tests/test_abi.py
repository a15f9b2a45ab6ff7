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


def _view(ptr, size, stride):
    v = _lib.View4()
    v.data = ptr
    for i in range(4):
        v.size[i], v.stride[i] = size[i], stride[i]
    return v


def test_selection_rejects_views_past_32_bit_offsets():
    """The dense accessors form block-id offsets in 32 bits and token offsets of a (batch, head)
    k / v slice in 32 bits: larger views are rejected on the host (OMM_EUNSUPPORTED) before
    anything is launched, so fake device addresses never reach a kernel."""
    import ctypes
    L = _lib.lib()
    M, N, H, D, G, T = 64, 256, 1, 128, 64, 4
    q = _view(0x10000, (1, M, H, D), (M * H * D, H * D, D, 1))
    k = _view(0x20000, (1, N, H, D), (N * H * D, H * D, D, 1))
    out = _view(0x30000, (1, M, H, D), (M * H * D, H * D, D, 1))
    ids_ok = _view(0x40000, (1, 1, H, T), (T, T, T, 1))
    ids_big = _view(0x40000, (1, 1, H, T), (T, T, T, 2 ** 30))  # last element at 3 * 2^30
    k_big = _view(0x20000, (1, 3, H, D), (3 * 2 ** 31, 2 ** 31, D, 1))  # 2 * 2^31 >= 2^32
    args = lambda kk, ids: (ctypes.byref(q), ctypes.byref(kk), ctypes.byref(kk), ctypes.byref(ids),
                            _lib.OMM_BF16, 64, 1, 0, G, 0.088, ctypes.byref(out), None, None)
    assert L.omm_sel_fwd(*args(k, ids_big)) == 2  # OMM_EUNSUPPORTED
    assert "2^31" in _lib.last_error()
    assert L.omm_sel_fwd(*args(k_big, ids_ok)) == 2
    assert "2^32" in _lib.last_error()
