"""The GGUF reader (qw6_amd/csrc/qw6_gguf.cpp) built for the host under
AddressSanitizer and UndefinedBehaviorSanitizer (g++, no device code) and run
over files a model loader must survive: the corrupt files of test_gguf.py
(each rejected there, as qw6's reader rejects them), valid files with an
expert pack, and seeded mutants of both (bytes set at random, bits flipped,
header and tensor-table fields set to extreme counts and sizes, truncations,
trailing garbage). Every query of include/qw6_gguf.h runs on each file the
reader accepts. Bar: no sanitizer finding (the build aborts on the first),
and the driver's own exit status 0.
"""
from __future__ import annotations

import os
import random
import shutil
import struct
import subprocess
from pathlib import Path

import numpy as np
import pytest

import test_gguf as TG
from qw6_amd import gguf as G

ROOT = Path(__file__).resolve().parent.parent
HIP_INC = "/opt/rocm/include"
HIP_LIB = "/opt/rocm/lib"


def _toolchain_ok() -> bool:
    return shutil.which("g++") is not None and os.path.exists(os.path.join(HIP_INC, "hip"))


def _seed_files(d: Path) -> list:
    blobs = []
    for name, blob in TG.corrupt_files():
        (d / ("c_" + name)).write_bytes(blob)
        blobs.append(blob)
    pack = d / "v_pack.gguf"
    G.write_gguf(pack, TG.KV_ALL, [
        ("blk.0.ffn_gate_exps.weight", G.G_Q4_K, [256, 4, 3],
         (np.arange(144 * 12) % 251).astype(np.uint8)),
        ("blk.0.ffn_down_exps.weight", G.G_Q6_K, [256, 2, 3], np.zeros(210 * 6, np.uint8)),
        ("x", G.G_F32, [16], np.zeros(64, np.uint8)),
    ])
    blobs.append(pack.read_bytes())
    zero = d / "v_zero.gguf"
    G.write_gguf(zero, TG.KV_ALL, [])
    blobs.append(zero.read_bytes())
    return blobs


def _mutants(d: Path, blobs: list, pack: bytes, n: int, seed: int):
    rng = random.Random(seed)
    extremes = [0, 1, 2 ** 31 - 1, 2 ** 32 - 1, 2 ** 63 - 1, 2 ** 64 - 1, 4097, 513]
    t0 = max(0, pack.find(b"blk.0.ffn_gate_exps.weight") - 8)
    for i in range(n):
        op = rng.randrange(6)
        b = bytearray(pack if op == 5 else rng.choice(blobs))
        if op == 0 and b:
            for _ in range(rng.randrange(1, 8)):
                b[rng.randrange(len(b))] = rng.randrange(256)
        elif op == 1 and b:
            b = b[:rng.randrange(len(b))]
        elif op == 2 and len(b) > 24:
            j = rng.randrange(0, min(len(b) - 8, 200))
            b[j:j + 8] = struct.pack("<Q", rng.choice(extremes))
        elif op == 3:
            b += bytes(rng.randrange(256) for _ in range(rng.randrange(1, 300)))
        elif op == 4:
            for _ in range(rng.randrange(1, 5)):
                if b:
                    b[rng.randrange(min(len(b), 512))] ^= 1 << rng.randrange(8)
        elif op == 5:   # the tensor table of the pack file: names, dims, types, offsets
            for _ in range(rng.randrange(1, 4)):
                j = rng.randrange(t0, min(len(b), t0 + 220))
                b[j] = rng.randrange(256) if rng.random() < 0.5 else b[j] ^ (1 << rng.randrange(8))
        (d / ("m%05d" % i)).write_bytes(bytes(b))


@pytest.mark.skipif(not _toolchain_ok(), reason="g++ or the HIP headers are not installed")
def test_gguf_reader_under_sanitizers(tmp_path):
    exe = tmp_path / "gguf_parse_sanitized"
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=all", "-fno-omit-frame-pointer",
           "-I" + str(ROOT / "include"), "-I" + str(ROOT / "qw6_amd" / "csrc"),
           "-D__HIP_PLATFORM_AMD__", "-isystem", HIP_INC, "-o", str(exe),
           str(ROOT / "tests" / "c" / "gguf_parse_sanitized.cpp"),
           str(ROOT / "qw6_amd" / "csrc" / "qw6_gguf.cpp"),
           "-L" + HIP_LIB, "-lamdhip64", "-Wl,-rpath," + HIP_LIB]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0 and "asan" in (r.stderr or "").lower():
        pytest.skip("the sanitizer runtimes are not installed")
    assert r.returncode == 0, r.stderr[-2000:]
    files = tmp_path / "files"
    files.mkdir()
    blobs = _seed_files(files)
    _mutants(files, blobs, (files / "v_pack.gguf").read_bytes(), 4000, 1234)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([str(exe), str(files)], capture_output=True, text=True, env=env, timeout=600)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "AddressSanitizer" not in out and "runtime error" not in out, out[-4000:]
    opened, rejected = (int(v) for v in r.stdout.split()[1::2])
    assert opened >= 2 and rejected >= len(TG.corrupt_files())   # both kinds were exercised
