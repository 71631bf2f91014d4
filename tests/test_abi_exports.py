"""The C-ABI library loads and exports what include/*.h declare (no GPU
needed: nothing here launches work)."""
import ctypes as C
import os
import re
import subprocess

import ctbind as cb

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header):
    text = open(os.path.join(REPO, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b((?:backend|hipb)_[A-Za-z0-9_]+)\s*\(", text))


def exported(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", lib], check=True,
                         capture_output=True, text=True).stdout
    return {ln.split()[-1] for ln in out.splitlines() if " T " in ln}


def test_backend_abi_exports():
    names = declared("backend.h")
    assert len(names) == 40
    assert names == set(cb.ABI_SIGS)
    syms = exported(cb.HIP_LIB)
    assert names <= syms
    lib = C.CDLL(cb.HIP_LIB)
    for n in names:
        assert getattr(lib, n)


def test_engine_exports():
    path = os.path.join(REPO, "include", "hipb.h")
    if not os.path.exists(path):
        return
    names = declared("hipb.h")
    assert names and names <= exported(cb.HIP_LIB)


def test_product_does_not_link_the_oracle():
    syms = subprocess.run(["nm", "-D", cb.HIP_LIB], check=True, capture_output=True, text=True).stdout
    assert "orc_" not in syms
    deps = subprocess.run(["ldd", cb.HIP_LIB], capture_output=True, text=True).stdout
    assert "oracle" not in deps and "ref_cpu" not in deps


def test_kernel_struct_mirrors_match():
    """The tests' ctypes mirrors of CtGemv and CtWarmSet have the C structs' sizes."""
    from structs import CtGemv, CtWarmSet
    lib = C.CDLL(cb.HIP_LIB)
    lib.ctk_gemv_sizeof.restype = C.c_int
    lib.ctk_warmset_sizeof.restype = C.c_int
    assert C.sizeof(CtGemv) == lib.ctk_gemv_sizeof()
    assert C.sizeof(CtWarmSet) == lib.ctk_warmset_sizeof()
