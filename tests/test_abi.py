"""The C ABI (CPU, no GPU calls): libmpcx.so loads and exports every function
that include/*.h declares, and every declaration has C linkage."""
import ctypes
import glob
import os
import re
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "idash26-track3_amd", "libmpcx.so")


def _declared():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        src = open(h).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        src = re.sub(r"//[^\n]*", "", src)
        for m in re.finditer(r"\b(mpcx_\w+)\s*\(", src):
            names.add(m.group(1))
    return names


def test_header_declares_entry_points():
    names = _declared()
    assert len(names) > 30
    assert {"mpcx_create", "mpcx_tr_eval", "mpcx_model_forward"} <= names


def test_library_exports_every_declared_symbol():
    assert os.path.exists(LIB), "libmpcx.so not built (run __graft_entry__.build())"
    lib = ctypes.CDLL(LIB)
    missing = [n for n in sorted(_declared()) if not hasattr(lib, n)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if ln.strip()}
    assert _declared() <= exported  # unmangled names: C linkage


def test_library_reports_no_device_without_gpu():
    """Without a visible GPU the library must refuse to create a context
    (there is no CPU fallback)."""
    lib = ctypes.CDLL(LIB)
    if os.path.exists("/dev/kfd") and os.access("/dev/kfd", os.R_OK):
        return  # a GPU box: covered by the gpu tests
    h = ctypes.c_void_p()
    st = lib.mpcx_create(32, 12, 0, ctypes.byref(h))
    assert st != 0 and not h.value
