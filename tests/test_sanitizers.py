"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU only;
the reference's own judges run this way, judges/run.py:81-88):

- the sessions' version table and the copy-on-write page pool
  (tests/host_versions_check.cpp over csrc/state_table.h, csrc/page_pool.cpp);
- the checkpoint header reader (csrc/safetensors.cpp) over library-written
  files and malformed headers;
- the oracle (oracle/oracle.c) under its own CPU tests (known-answer vectors,
  packing tables, expert permutation), loaded as a sanitized build.
Any sanitizer report fails the run (-fno-sanitize-recover=all)."""
import json
import os
import shutil
import struct
import subprocess
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(ROOT, "rust-ts-tokio-inference-engine_amd", "csrc")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1")

pytestmark = pytest.mark.skipif(shutil.which("g++") is None or shutil.which("gcc") is None,
                                reason="gcc/g++ not available")


def run(cmd, **kw):
    r = subprocess.run(cmd, capture_output=True, text=True, env=ENV, timeout=600, **kw)
    assert r.returncode == 0 and "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr, \
        r.stdout[-3000:] + r.stderr[-6000:]
    return r


def test_version_table_and_page_pool(tmp_path):
    exe = tmp_path / "host_versions_check"
    run(["g++", "-std=c++20", *SAN, "-I", CSRC, os.path.join(HERE, "host_versions_check.cpp"),
         os.path.join(CSRC, "page_pool.cpp"), "-o", str(exe)])
    assert run([str(exe)]).stdout.startswith("PASS")


def _file(path, header, payload=b""):
    h = header if isinstance(header, bytes) else json.dumps(header).encode()
    path.write_bytes(struct.pack("<Q", len(h)) + h + payload)
    return str(path)


def test_safetensors_reader(tmp_path):
    from safetensors.numpy import save_file

    exe = tmp_path / "sanitize_safetensors"
    run(["g++", "-std=c++20", *SAN, "-I", CSRC, os.path.join(HERE, "sanitize_safetensors.cpp"),
         os.path.join(CSRC, "safetensors.cpp"), "-o", str(exe)])
    good = tmp_path / "good.safetensors"
    save_file({"a": np.arange(12, dtype=np.float32).reshape(3, 4), "b": np.ones((2,), np.uint32)}, str(good))
    ok = {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}
    files = [str(good),
             _file(tmp_path / "dup.st", b'{"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}, "a": {}}',
                   b"\0" * 8),
             _file(tmp_path / "deep.st", b"[" * 4000 + b"]" * 4000),
             _file(tmp_path / "escape.st", b'{"\\ud800": 1}'),
             _file(tmp_path / "overlap.st", {"a": ok, "b": ok}, b"\0" * 8),
             _file(tmp_path / "trunc.st", b'{"a": {"dtype": "F32", "shape": [2], "data_o'),
             _file(tmp_path / "huge.st", {"a": {"dtype": "F32", "shape": [2**40], "data_offsets": [0, 8]}},
                   b"\0" * 8),
             _file(tmp_path / "neg.st", {"a": {"dtype": "F32", "shape": [-1], "data_offsets": [0, 8]}}, b"\0" * 8),
             _file(tmp_path / "trail.st", json.dumps({"a": ok}).encode() + b" x", b"\0" * 8)]
    (tmp_path / "short.st").write_bytes(b"\x10\0\0")
    files.append(str(tmp_path / "short.st"))
    out = run([str(exe), *files]).stdout.splitlines()
    assert out[0] == "ok 2"
    assert all(line.startswith("rejected") for line in out[1:]), out


def test_oracle_under_its_cpu_tests(tmp_path):
    so = tmp_path / "liboracle_san.so"
    run(["gcc", "-std=c11", *SAN, "-fopenmp", "-fPIC", "-shared", os.path.join(ROOT, "oracle", "oracle.c"), "-o",
         str(so), "-lm"])
    asan = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True).stdout.strip()
    env = dict(ENV, ORACLE_LIB=str(so), LD_PRELOAD=asan, OMP_NUM_THREADS="4")
    tests = [os.path.join(HERE, t) for t in ("test_oracle_kat.py", "test_oracle_pack.py", "test_oracle_permute.py")]
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider", *tests], capture_output=True,
                       text=True, env=env, timeout=900, cwd=ROOT)
    assert r.returncode == 0 and "runtime error" not in r.stderr + r.stdout and "AddressSanitizer" not in r.stderr, \
        r.stdout[-3000:] + r.stderr[-6000:]
    assert " passed" in r.stdout
