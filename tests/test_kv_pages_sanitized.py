"""The engine's host-side KV page bookkeeping (qraf_amd/csrc/kv_pages.cpp:
sequences, their pages and the free list behind qraf_engine_seq_create /
_seq_release / _step) built with AddressSanitizer and UndefinedBehaviorSanitizer
(tests/cpp/kv_pages_check) and driven by seeded random operations over 200
pools per seed: valid and invalid steps (unknown or released sequences,
positions outside the cache or past a sequence's length), pools that run out,
releases and re-admission.  Every status must follow the step rules, a refused
step must change nothing, and no sanitizer may report.  No GPU use: this runs
in the CPU suite.
"""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def checker():
    r = subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "tests", "cpp"), "kv_pages_check"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return os.path.join(ROOT, "tests", "cpp", "kv_pages_check")


@pytest.mark.parametrize("seed", [1, 1000])
def test_sanitized_page_bookkeeping(checker, seed):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1", UBSAN_OPTIONS="halt_on_error=1")
    r = subprocess.run([checker, str(seed), "300"], capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0 and "Sanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr[-4000:]
    m = re.search(r"(\d+) steps accepted, (\d+) invalid refused, (\d+) refused for lack of pages", r.stdout)
    assert m, r.stdout
    accepted, invalid, nomem = (int(g) for g in m.groups())
    assert accepted > 1000 and invalid > 1000 and nomem > 100  # every outcome exercised
