"""The device API driven from C on the GPU: tests/c/qw6_layer_caller.c, a
C11 program built with qw6's warning flags (reference Makefile:5) by
build(), runs the self-test and the F32 host probe by qw6's Vulkan names
(qw6.c:3540, 1877), generates the seeded Q4_K / Q6_K decode layer on the
device, runs one token through qw6_hip_moe_forward eagerly and as a
captured HIP graph replayed three times, and checks each result against
qw6's own qw6_apply_layer_moe output for that layer and token (the
committed golden, passed as raw binary files)."""
from __future__ import annotations

import subprocess
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
EXE = ROOT / "tests" / "c" / "qw6_layer_caller"


def test_c_caller_graph_capture_vs_golden(tmp_path):
    assert EXE.exists(), "tests/c/qw6_layer_caller is not built: run __graft_entry__.build()"
    G = np.load(ROOT / "tests" / "golden" / "golden.npz")
    np.ascontiguousarray(G["layer_q4k_s11_idx"], np.int32).tofile(tmp_path / "idx.bin")
    np.ascontiguousarray(G["layer_q4k_s11_w"], np.float32).tofile(tmp_path / "w.bin")
    np.ascontiguousarray(G["layer_q4k_s11_out"], np.float32).tofile(tmp_path / "out.bin")
    print("running", EXE, flush=True)
    r = subprocess.run([str(EXE), str(tmp_path)], capture_output=True, text=True, timeout=240)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, (r.stdout, r.stderr)
    lines = r.stdout.strip().splitlines()
    assert lines[-1] == "ok"
    assert sum("graph replay" in ln and ln.endswith("-> ok") for ln in lines) == 3
