"""The C-ABI library loads and exports every function include/q38hip.h declares
(CPU only: no compute calls)."""
import ctypes
import os
import re

import q38hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = []
    for header in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if not header.endswith(".h"):
            continue
        text = open(os.path.join(ROOT, "include", header)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"^[A-Za-z_][\w \*]*?\b(q38\w*)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_header_declares_entry_points():
    names = declared_functions()
    for required in ("q38_quantize_q8_k", "q38_tensor_gemv_q8_k", "q38_tensor_gemm_q8_k",
                     "q38hip_gemm_q8_k", "q38hip_argmax", "q38hip_accept"):
        assert required in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(q38hip.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    assert set(q38hip.EXPORTS) <= set(declared_functions())
