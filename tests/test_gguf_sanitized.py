"""The GGUF reader (arf_amd/csrc/arfq_gguf.cpp) under AddressSanitizer and
UBSan, host code only: tests/gguf_fuzz_driver.cpp is built with the reader and
walks every query of its C ABI over seeded random GGUF files and mutations of
them (every truncation point of the header, byte flips, huge length fields).
A read outside a buffer, a use after free, a leak or undefined behaviour
aborts the driver, and so does a tensor range past the end of the file or an
upload slice outside its tensor (the mapping is not watched by the
sanitizers, so the driver checks those ranges itself); the other GGUF tests
check what the reader returns.  The reference's own malformed-input tests (gguf.rs:2396-2480) cover
the magic, version and truncation cases singly."""
import os
import shutil
import struct
import subprocess

import numpy as np
import pytest

from test_gguf import _random_file

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def _build(tmp_path):
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("no g++")
    exe = str(tmp_path / "gguf_drv")
    cmd = [cxx, "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-I", os.path.join(ROOT, "include"), os.path.join(ROOT, "arf_amd", "csrc", "arfq_gguf.cpp"),
           os.path.join(HERE, "gguf_fuzz_driver.cpp"), "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        if "asan" in r.stderr.lower() or "sanitize" in r.stderr.lower():
            pytest.skip("no sanitizer runtime: " + r.stderr[-300:])
        raise AssertionError(r.stderr)
    return exe


def _mutants(data, rng, header_end):
    out = [data]
    hdr = max(1, min(len(data), header_end))
    for cut in np.unique(np.linspace(0, len(data), 48).astype(int)):
        out.append(data[:cut])
    for _ in range(96):  # byte flips, mostly in the header and tensor table
        b = bytearray(data)
        pos = int(rng.integers(0, hdr)) if rng.random() < 0.85 or len(data) == hdr else int(rng.integers(hdr, len(data)))
        b[pos] = int(rng.integers(0, 256))
        out.append(bytes(b))
    for _ in range(32):  # 8-byte fields overwritten with huge or negative counts and lengths
        b = bytearray(data)
        if len(b) < 16:
            break
        pos = int(rng.integers(8, min(len(b), hdr + 8) - 7))
        big = (2**63 - 1, 2**64 - 1, 2**32, 2**31 - 1, 2**40, 0)
        v = big[int(rng.integers(0, len(big)))]
        b[pos:pos + 8] = struct.pack("<Q", v)
        out.append(bytes(b))
    return out


def test_reader_under_sanitizers(tmp_path):
    exe = _build(tmp_path)
    rng = np.random.default_rng(0xA7F0A5A5)
    files = []
    for seed in range(10):
        (data, offs), _ = _random_file(100 + seed)
        header_end = min(offs) if offs else len(data)
        for i, m in enumerate(_mutants(data, rng, header_end)):
            p = tmp_path / f"f{seed}_{i}.gguf"
            p.write_bytes(m)
            files.append(str(p))
    files.append(str(tmp_path / "missing.gguf"))
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:halt_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([exe, *files], capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0, r.stderr[-4000:]
    lines = r.stdout.splitlines()
    assert len(lines) == len(files) + 1
    opened = sum(" open=0 " in ln for ln in lines)
    # the unmutated files and some mutants open; most mutants are refused
    assert 10 <= opened < len(files)
