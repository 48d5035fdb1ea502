"""The continuous-batch workload of the decode benchmark at its real shape,
against greedy streams the compiled reference wrote (tests/golden/
gen_c5_golden.py): the Qwen2.5-3B architecture (36 layers, hidden 2048,
16 / 2 heads, FFN 11008, vocab 151936, tied Q4 embedding, QKV bias), Q4
weights from the device generator (seed 3), f32 KV pages (the reference's
KVCache values).

160 requests with seeded prompts U[16,512] and outputs U[64,256] run through
the BatchScheduler as the benchmark runs them: 128 slots, a 512-row budget
per step, prompts fed in chunks of up to 512 tokens after the decode rows,
requests admitted as others retire (whose KV pages they then reuse).  For
four requests (the first two admitted, and the last two, which wait for
slots) every logit vector that picks one of their first 32 greedy tokens is
compared with the reference's single-sequence decode (InferenceEngine::
generate_tokens, src/runtime/inference.cpp:68-159): 80 logits per position
(the reference's top 16 and 64 fixed indices) within 1e-3 relative + 1e-4
absolute, and the 32 tokens identical.
"""
import numpy as np
import pytest

from tests.conftest import golden
from tests.golden import gen_c5_golden as G
from tests.test_gpu_engine import check_logits

pytestmark = pytest.mark.gpu


def test_qwen25_3b_continuous_batch_matches_reference(hip):
    from qraf_amd._lib import F32, Q4_0
    from qraf_amd.engine import BatchScheduler, Engine, model_config
    g = golden("c5_qwen25_3b_q4.npz")
    work = G.c5_workload(int(g["workload_seed"]), int(g["n_requests"]))
    checked = [int(i) for i in g["checked"]]
    for i in checked:
        assert np.array_equal(np.array(work[i][0], np.int32), g[f"prompt_{i}"]), "workload generator changed"
    q = G.QWEN
    cfg = model_config(*(q[k] for k in ("vocab", "hidden", "layers", "heads", "kv_heads", "inter", "max_seq",
                                        "rope_theta", "eps")))
    # 128 sequences of at most 512 + 256 positions: 48 pages of 16 each
    e = Engine(cfg, kv_dtype=F32, max_batch=512, num_pages=128 * 48 + 64)
    try:
        e.generate_weights(Q4_0, Q4_0, Q4_0, True, True, int(g["weight_seed"]))
        e.finalize()
        sched = BatchScheduler(e, max_batch=128, max_rows=512, prefill_chunk=512)
        ids = [sched.submit(p, o) for p, o in work]
        which = {ids[i]: i for i in checked}
        got = {i: [] for i in checked}  # per checked request: (probed logits, token) per position

        def observe(sc, lrows, nx):
            for k, r in enumerate(lrows):
                i = which.get(r.id)
                if i is None or len(got[i]) >= G.GEN:
                    continue
                lg = sc.engine.read_logits(k)[0]
                got[i].append((lg[g[f"idx_{i}"][len(got[i])]], int(nx[k])))

        sched.observer = observe
        done = {r.id: r for r in sched.run()}
        print(f"{sched.steps} steps, {sched.rows} rows", flush=True)
        assert len(done) == len(work)
        for rid, i in which.items():
            r = done[rid]
            assert len(r.generated) == work[i][1]  # no EOS: every request runs to its max_tokens
            if i >= 128:
                assert r.admit_step > 0, f"request {i} was admitted at step 0"
            want_tok = g[f"tokens_{i}"]
            assert len(got[i]) == G.GEN
            for j, (vals, tok) in enumerate(got[i]):
                ref = g[f"val_{i}"][j]
                print(f"request {i} token {j}: max |diff| {np.abs(vals - ref).max():.2e} "
                      f"(reference top-2 gap {g[f'gap_{i}'][j]:.2e})", flush=True)
                check_logits(vals, ref.astype(np.float64), f"request {i}, token {j}")
                assert tok == int(want_tok[j]), f"request {i}, token {j}: {tok} vs reference {int(want_tok[j])}"
            assert r.generated[:G.GEN] == want_tok.tolist()
    finally:
        e.close()
