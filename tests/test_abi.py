"""CPU checks of the C-ABI library: it loads, exports every symbol that
include/g4hip.h declares, its Params structs have the WGSL layouts, and its
host-side error paths behave without a GPU (no kernel is launched here)."""
import ctypes
import os
import re
import subprocess

import pytest

import g4hip
from g4hip import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "g4hip.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*|void\*|uint64_t)\s+(g4_\w+)\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    assert os.path.exists(_lib.LIB_PATH), "build libg4hip.so first (__graft_entry__.build())"
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if ln.strip()}
    decl = declared_symbols()
    assert len(decl) >= 55
    missing = [s for s in decl if s not in exported]
    assert not missing, missing
    # and the Python host binds exactly those
    assert sorted(_lib.SIGNATURES) == decl


def test_library_loads_and_reports_version():
    L = g4hip.lib()
    assert L.g4_version() == 1


def test_params_layouts_match_wgsl():
    # 4-byte fields, in WGSL declaration order
    assert ctypes.sizeof(g4hip.MatmulParams) == 8
    assert ctypes.sizeof(g4hip.KvStoreParams) == 16
    assert ctypes.sizeof(g4hip.AttnScoreParams) == 24
    assert g4hip.AttnScoreParams.scale.offset == 16 and g4hip.AttnScoreParams.sliding_window.offset == 20
    assert ctypes.sizeof(g4hip.SoftmaxParams) == 8
    assert ctypes.sizeof(g4hip.AttnOutputParams) == 16
    assert ctypes.sizeof(g4hip.PerHeadNormParams) == 16
    assert ctypes.sizeof(g4hip.NormRopeParams) == 24
    # position is patched at byte 12 of the fused norm+rope uniform (src/engine.ts:1494-1495)
    assert g4hip.NormRopeParams.position.offset == 12
    # position at byte 8 of kvCacheStore, seq_len at byte 12 of attnScore (src/engine.ts:1496-1497)
    assert g4hip.KvStoreParams.position.offset == 8 and g4hip.AttnScoreParams.seq_len.offset == 12
    assert g4hip.SoftmaxParams.seq_len.offset == 4
    assert ctypes.sizeof(g4hip.RmsNormParams) == 8 and ctypes.sizeof(g4hip.SoftcapParams) == 8


def test_error_paths_without_device():
    L = g4hip.lib()
    # null context -> G4_ERR_INVALID with a message, before any device call
    rc = L.g4_rmsNorm(None, None, None, None, g4hip.RmsNormParams(1536, 1e-6))
    assert rc == -1 and b"null context" in L.g4_last_error()
    rc = L.g4_init(0, None)
    assert rc == -1
    size = ctypes.c_size_t()
    # shape validation is host-only
    bad = g4hip.AttnScoreParams(8, 3, 256, 10, 1.0, 0)
    assert L.g4_attnDecode_workspace_size(bad, ctypes.byref(size)) == -1
    good = g4hip.AttnScoreParams(8, 1, 256, 32768, 1.0, 0)
    assert L.g4_attnDecode_workspace_size(good, ctypes.byref(size)) == 0
    # 32768 positions in 64-position splits: 512 splits x 8 heads x (256 + 2) floats
    assert size.value == 512 * 8 * 258 * 4


def test_init_without_gpu_fails_cleanly():
    """In a container with no GPU, g4_init reports G4_ERR_NO_DEVICE (not a crash)."""
    if os.path.exists("/dev/kfd") and os.access("/dev/kfd", os.R_OK | os.W_OK):
        pytest.skip("a GPU is present; covered by the gpu tests")
    L = g4hip.lib()
    h = ctypes.c_void_p()
    rc = L.g4_init(0, ctypes.byref(h))
    assert rc == -6 and h.value is None
    with pytest.raises(g4hip.G4Error):
        g4hip.Context(0)


def test_splitmix64_matches_oracle():
    import oracle as O

    for seed, idx in [(0, 0), (1234567, 3), (2 ** 63 + 5, 10 ** 12)]:
        assert g4hip.device.splitmix64(seed, idx) == O.splitmix64(seed, idx)


def test_header_constants_match_the_python_host():
    """Status codes and the o projection's share count, as the header defines them."""
    text = open(HEADER).read()
    defs = dict(re.findall(r"^#define\s+(G4_\w+)\s+\(?(-?\d+)\)?", text, re.M))
    assert int(defs["G4_O_SHARES"]) == _lib.O_SHARES
    for code, name in _lib.ERRORS.items():
        assert int(defs[name]) == code, name
