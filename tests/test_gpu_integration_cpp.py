"""The reference-side bindings of the C ABI, compiled as C++ against the
reference's own headers (tests/cpp/integration_test.cpp, built by
tests/cpp/Makefile from `__graft_entry__.build()`), run against the
reference's own code: the Backend::HIP branch of dispatch_matvec_q against
the reference's dispatch_matvec_q (backend.cpp:131-199), and HipTransformer's
forward against the reference Transformer::forward (transformer.h:55-61) on
a .qraf file the reference's QrafWriter wrote, logits within 1e-3 relative +
1e-4 absolute and the same greedy token at every position, before and after
reset().  The binary and the compiled reference travel with the working
tree; a missing one fails the test."""
import os
import subprocess

import pytest

from oracle import pyoracle as po

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("reference")]

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "integration_test")
BATCH_BIN = os.path.join(ROOT, "tests", "cpp", "batch_integration_test")


@pytest.mark.parametrize("name,tokens", [("q8_llama", 24), ("q4_qwen2_tied_bias", 24), ("q8_hd64_gqa3", 12)])
def test_reference_bindings_compiled_against_reference_headers(hip, tmp_path, name, tokens):
    from tests.test_gpu_engine import SMALL
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is missing; build it with `make -C tests/cpp` (needs the reference checkout)")
    kw, seed = SMALL[name]
    m = po.Model(po.make_config(**kw), seed)
    path = str(tmp_path / "m.qraf")
    m.write_qraf(path)
    m.close()
    print(f"integration_test {name} tokens={tokens}", flush=True)
    r = subprocess.run([BIN, path, str(tokens)], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, f"exit {r.returncode}\n{r.stdout}\n{r.stderr[-2000:]}"
    assert r.stdout.strip().endswith("PASS")


@pytest.mark.parametrize("name,requests,seed", [("q4_qwen2_tied_bias", 24, 5), ("q8_hd64_gqa3", 24, 6),
                                                ("q4_gqa8_hd128", 16, 7)])
def test_batch_scheduler_binding_against_reference(hip, tmp_path, name, requests, seed):
    """tests/cpp/batch_integration_test: HipBatchScheduler (the reference
    BatchScheduler's interface over qraf_engine_step_async / _step_collect,
    compiled against runtime/batch_scheduler.h) runs ragged requests with
    admission into 6 slots and a 32-row budget; every stream equals the
    reference Transformer's decode of that request alone, pipelined and with
    every logit row read back, the logits of the first 32 tokens within
    1e-3/1e-4.  The same binary checks the elementwise Backend::HIP branches
    against the reference's dispatch_* functions."""
    from tests.test_gpu_engine import SMALL
    if not os.path.exists(BATCH_BIN):
        pytest.fail(f"{BATCH_BIN} is missing; build it with `make -C tests/cpp` (needs the reference checkout)")
    kw, mseed = SMALL[name]
    m = po.Model(po.make_config(**kw), mseed)
    path = str(tmp_path / "m.qraf")
    m.write_qraf(path)
    m.close()
    print(f"batch_integration_test {name} requests={requests} seed={seed}", flush=True)
    r = subprocess.run([BATCH_BIN, path, str(requests), str(seed)], capture_output=True, text=True, timeout=150)
    print(r.stdout)
    assert r.returncode == 0, f"exit {r.returncode}\n{r.stdout}\n{r.stderr[-2000:]}"
    assert r.stdout.strip().endswith("PASS")
