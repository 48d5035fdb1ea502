"""The library's .qraf parser (qraf_amd/csrc/qraf_file.cpp: the host code
behind qraf_file_read_config and qraf_engine_create_from_file) built with
AddressSanitizer and UndefinedBehaviorSanitizer (tests/cpp/qraf_file_check)
and run over a file the reference's QrafWriter wrote, the corruptions
test_loader.py checks, and a few hundred seeded random corruptions of the
header, the directories and the string table.  Every run must end without a
sanitizer report, and its status must be the one the library returns for the
same file.  No GPU use: this runs in the CPU suite.
"""
import os
import subprocess

import numpy as np
import pytest

from oracle import pyoracle as po
from tests.test_loader import (H_FILE_SIZE, H_MAGIC, H_NUM_TENSORS, H_STRINGS_SIZE, H_TENSOR_DIR, H_VERSION, KW,
                               first_tensor, read_config, u32, u64)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CHECK = os.path.join(ROOT, "tests", "cpp", "qraf_file_check")
need_ref = pytest.mark.skipif(po.ref() is None, reason="oracle/_ref (the compiled reference) is not built")


@pytest.fixture(scope="module")
def checker():
    r = subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "tests", "cpp"), "qraf_file_check"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return CHECK


def run_checker(checker, paths):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1", UBSAN_OPTIONS="halt_on_error=1")
    r = subprocess.run([checker, *paths], capture_output=True, text=True, env=env, timeout=300)
    assert r.returncode == 0 and "Sanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr[-4000:]
    lines = r.stdout.strip().split("\n")
    assert len(lines) == len(paths)
    return [tuple(int(v) for v in ln.split()) for ln in lines]


@pytest.fixture(scope="module")
def written(tmp_path_factory):
    m = po.Model(po.make_config(**KW), 21)
    path = str(tmp_path_factory.mktemp("qraf_san") / "m.qraf")
    m.write_qraf(path)
    yield m, path
    m.close()


def corruptions(b, rng, n):
    """n seeded corruptions of the file bytes b: random bytes written into
    the header, the tensor / quant / config records and the string table,
    header fields set to boundary values, and random truncations."""
    hdr = np.frombuffer(bytes(b[:128]), np.uint8)
    tdir = int.from_bytes(b[48:56], "little")
    out = []
    fields64 = [8, 16, 24, 48, 56, 64, 72, 80, 88, 96]
    fields32 = [0, 4, 104, 108]
    for i in range(n):
        c = bytearray(b)
        kind = i % 5
        if kind == 0:  # random bytes in the header
            for _ in range(int(rng.integers(1, 6))):
                c[int(rng.integers(0, 128))] = int(rng.integers(0, 256))
        elif kind == 1:  # a header field at a boundary value
            if rng.integers(0, 2):
                off = int(rng.choice(fields64))
                v = int(rng.choice([0, 1, len(b) - 1, len(b), len(b) + 1, 2 ** 63, 2 ** 64 - 1, 2 ** 32]))
                c[off:off + 8] = (v % 2 ** 64).to_bytes(8, "little")
            else:
                off = int(rng.choice(fields32))
                v = int(rng.choice([0, 1, 2, 2 ** 31, 2 ** 32 - 1, 1 << 24]))
                c[off:off + 4] = v.to_bytes(4, "little")
        elif kind == 2:  # random bytes in the tensor directory (names, shapes, offsets, sizes)
            for _ in range(int(rng.integers(1, 8))):
                p = tdir + int(rng.integers(0, 80 * 4))
                if p < len(c):
                    c[p] = int(rng.integers(0, 256))
        elif kind == 3:  # random bytes anywhere before the tensor data
            lim = min(len(c), int(hdr[120:128].view(np.uint64)[0]) or len(c))
            for _ in range(int(rng.integers(1, 10))):
                c[int(rng.integers(0, max(lim, 129)))] = int(rng.integers(0, 256))
        else:  # truncation (with the size field kept or fixed up)
            cut = int(rng.integers(0, len(c)))
            c = c[:cut]
            if rng.integers(0, 2) and len(c) >= 16:
                c[8:16] = len(c).to_bytes(8, "little")
        out.append(bytes(c))
    return out


@need_ref
def test_sanitized_parser_on_written_and_corrupted_files(checker, written, tmp_path):
    m, path = written
    b = bytearray(open(path, "rb").read())
    named = {
        "magic": u32(bytearray(b), H_MAGIC, 0x12345678),
        "version": u32(bytearray(b), H_VERSION, 2),
        "size_field": u64(bytearray(b), H_FILE_SIZE, len(b) + 64),
        "appended": bytearray(b) + b"\0",
        "truncated": bytearray(b)[: len(b) // 2],
        "tiny": bytearray(b)[:100],
        "name_offset": u32(bytearray(b), first_tensor(b) + 8, 0x7FFFFFF0),
        "data_past_end": u64(bytearray(b), first_tensor(b) + 56, len(b)),
        "string_table_cut": u64(bytearray(b), H_STRINGS_SIZE, 3),
        "tensor_count": u32(bytearray(b), H_NUM_TENSORS, 1 << 30),
        "tensor_dir_past_end": u64(bytearray(b), H_TENSOR_DIR, len(b) - 8),
        "empty": bytearray(),
    }
    files = [path]
    for name, data in named.items():
        p = str(tmp_path / f"{name}.qraf")
        open(p, "wb").write(bytes(data))
        files.append(p)
    rng = np.random.default_rng(2024)
    for i, data in enumerate(corruptions(b, rng, 400)):
        p = str(tmp_path / f"rand{i}.qraf")
        open(p, "wb").write(data)
        files.append(p)
    got = run_checker(checker, files)
    # the valid file parses, with every tensor of the model
    assert got[0][0] == 0 and got[0][1] == len(m.tensors())
    # the named corruptions are refused
    for (rc, _, _), name in zip(got[1:1 + len(named)], named):
        assert rc != 0, name
    # every status equals the library's for the same file
    for f, (rc, nt, _) in zip(files, got):
        rc_lib, _, n_lib = read_config(f)
        assert rc == rc_lib, (f, rc, rc_lib)
        if rc == 0:
            assert nt == n_lib
    refused = sum(1 for g in got[1 + len(named):] if g[0] != 0)
    assert 0 < refused < 400  # the random set holds both refused and accepted files
