"""The C ABI: the library loads, exports every function include/*.h
declares (qw6_hip.h, qw6_gguf.h), and the host layer rejects bad arguments
before any device work."""
import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

import qw6_amd as Q

HEADERS = sorted((Path(__file__).resolve().parents[1] / "include").glob("*.h"))


def declared_functions():
    text = "".join(re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S) for h in HEADERS)
    return sorted(set(re.findall(r"\b(qw6_hip_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    names = declared_functions()
    assert len(names) >= 20
    lib = C.CDLL(str(Q.LIB_PATH))
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_no_symbol_without_declaration():
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", str(Q.LIB_PATH)], capture_output=True,
                         text=True).stdout
    exported = set(re.findall(r"\b(qw6_hip_\w+)$", out, flags=re.M))
    assert exported <= set(declared_functions()), exported - set(declared_functions())


def test_host_ops_reject_bad_shapes_without_device_work():
    # cols % 256 != 0 and quant checks happen before any HIP call
    w = np.zeros(144, np.uint8)
    x = np.zeros(100, np.float32)
    with pytest.raises(Q.Qw6HipError, match="cols"):
        Q.matmul_host(Q.Q_Q4_K_M, w, x, 1, 100)
    with pytest.raises(Q.Qw6HipError, match="bounds"):
        Q.moe_route_host(np.zeros(300, np.float32), 8)
    with pytest.raises(Q.Qw6HipError, match="bounds"):
        Q.moe_route_host(np.zeros(16, np.float32), 9)
    with pytest.raises(Q.Qw6HipError, match="bounds"):
        Q.moe_gather_host(np.zeros((9, 4), np.float32), np.zeros(9, np.float32), None, 0.0)
    assert Q.lib().qw6_hip_matmul_q4k_host(None, x, np.zeros(1, np.float32), 1, 256) == -1


def test_gpu_processes_never_load_the_reference_build():
    """qw6's compiled CPU path (oracle/_ref) checks the oracle in the
    container the repository is built in; no process on the GPU host loads
    it. Every GPU test, the smoke entry and the bench compare against (and
    time) the oracle port only: none of them reaches oracle.ref(), a ref_*
    wrapper, or the oracle test module that does."""
    root = Path(__file__).resolve().parents[1]
    files = sorted((root / "tests").glob("test_gpu*.py")) + sorted((root / "tests").glob("test_zz*.py"))
    files += [root / "bench.py", root / "__graft_entry__.py", root / "tests" / "cases.py",
              root / "tests" / "conftest.py"]
    pat = re.compile(r"\bO\.ref\(|\bO\.ref_\w+|\bref_moe_\w+\(|\btest_oracle\b")
    bad = [(f.name, m.group(0)) for f in files if f.exists() for m in pat.finditer(f.read_text())]
    assert not bad, bad
