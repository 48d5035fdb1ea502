"""The C-ABI library loads and exports every symbol include/qraf_hip.h
declares, and argument validation fails with the documented codes.  No
compute calls: these tests run without a GPU."""
import ctypes as C
import os
import re

import numpy as np

from tests.conftest import ROOT


def declared_symbols():
    syms = set()
    for name in os.listdir(os.path.join(ROOT, "include")):
        if name.endswith(".h"):
            text = open(os.path.join(ROOT, "include", name)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            syms |= set(re.findall(r"\b(qraf_\w+)\s*\(", text))
    return syms


def test_library_exports_every_declared_symbol():
    import qraf_amd
    lib = C.CDLL(qraf_amd.LIB_PATH)
    syms = declared_symbols()
    assert len(syms) > 30
    missing = [s for s in sorted(syms) if not hasattr(lib, s)]
    assert not missing, missing
    # and the Python binding covers them all
    from qraf_amd._lib import SIGNATURES
    assert not (syms - set(SIGNATURES)), sorted(syms - set(SIGNATURES))


def test_argument_validation_without_device():
    from qraf_amd._lib import ERR_DTYPE, ERR_INVALID, lib
    x = np.ones(64, np.float32)
    y = np.zeros(4, np.float32)
    fp = C.POINTER(C.c_float)
    w = np.zeros(4 * 72, np.uint8)
    rc = lib.qraf_hip_matvec_q(w.ctypes.data, 0, 99, 32, 4, 64, x.ctypes.data_as(fp), y.ctypes.data_as(fp))
    assert rc == ERR_DTYPE and b"dtype" in lib.qraf_hip_last_error()
    rc = lib.qraf_hip_matvec_q(None, 0, 10, 32, 4, 64, x.ctypes.data_as(fp), y.ctypes.data_as(fp))
    assert rc == ERR_INVALID
    rc = lib.qraf_hip_matvec_q(w.ctypes.data, 16, 10, 32, 4, 64, x.ctypes.data_as(fp), y.ctypes.data_as(fp))
    assert rc == ERR_INVALID and b"bytes" in lib.qraf_hip_last_error()  # w_size too small


def test_version_names_gfx950():
    from qraf_amd._lib import lib
    assert lib.qraf_hip_version().startswith(b"gfx950")


def test_noalloc_attention_refuses_shapes_beyond_its_scratch():
    """The no-allocation attention checks the workspace a shape needs against
    its fixed scratch on the host, before it touches the device: a shape
    beyond it is refused (no GPU needed)."""
    from qraf_amd._lib import ERR_INVALID, lib
    n, H, Hkv, hd, max_ctx = 1024, 64, 8, 128, 8192
    assert lib.qraf_hip_attention_workspace_bytes(n, H, Hkv, hd, max_ctx) > lib.qraf_hip_attention_noalloc_max_bytes()
    rc = lib.qraf_hip_paged_attention_noalloc_dev(None, None, None, 1, None, max_ctx // 16, None, n, H, Hkv, hd, 16,
                                                  0.1, max_ctx, None, None)
    assert rc == ERR_INVALID
    assert b"scratch holds" in lib.qraf_hip_last_error()


def test_integration_guide_names_every_declared_symbol():
    """INTEGRATION.md, the guide a reference maintainer binds from, names every
    entry point the header declares."""
    guide = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    missing = [s for s in sorted(declared_symbols()) if not re.search(r"\b" + s + r"\b", guide)]
    assert not missing, missing


def test_launch_floor_refuses_workgroup_counts_outside_its_range():
    """qraf_hip_launch_floor_dev takes 1..65536 workgroups; other counts are
    refused before anything is launched (no GPU needed)."""
    from qraf_amd._lib import ERR_INVALID, lib
    for w in (0, -1, 65537):
        assert lib.qraf_hip_launch_floor_dev(w, None) == ERR_INVALID
        assert b"workgroups" in lib.qraf_hip_last_error()
