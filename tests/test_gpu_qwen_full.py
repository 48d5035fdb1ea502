"""The continuous-batch workload at its real shape against the compiled
reference: the Qwen2.5-3B architecture (36 layers, hidden 2048, 16 / 2
heads, FFN 11008, vocab 151936, tied Q4 embedding, QKV bias), Q4 weights,
at 1 sequence per step (the batch-1 matvec path) and at 128 sequences per
step, where every step runs the 128-row kernels of the decode benchmark
(pipelined GEMMs, batched attention, fused norms).

KV pages are f32, the reference's KVCache (fp16 pages round every cached k
and v by 2^-11, which 36 layers carry past the logit bar at this depth).
The weights are the engine's device-generated ones, written to a .qraf file
in the reference's format; the reference's own QrafModel + Transformer load
it (oracle/_ref) and decode sequence 0 on the host (one sequence: a
4-token prompt, then 32 greedy tokens).  The
engine's logits for sequence 0 at every position must be within the engine
bar of the reference's (1e-3 relative + 1e-4 absolute), and its greedy
tokens equal.
"""
import numpy as np
import pytest

from oracle import pyoracle as po
from tests.test_gpu_engine import check_logits

GEN = 32  # greedy tokens of sequence 0 compared with the reference's

pytestmark = [pytest.mark.gpu,
              pytest.mark.usefixtures("reference")]


@pytest.mark.parametrize("n", [1, 128])
def test_qwen25_3b_q4_sequence_matches_reference(hip, tmp_path, n):
    import bench
    from qraf_amd._lib import call
    from qraf_amd.backend import DeviceBuffer, Stream
    from qraf_amd.engine import Engine, model_config
    q = bench.QWEN
    V = q["vocab"]
    cfg = model_config(*(q[k] for k in ("vocab", "hidden", "layers", "heads", "kv_heads", "inter", "max_seq",
                                        "rope_theta", "eps")))
    e = Engine(cfg, kv_dtype=po.F32, max_batch=max(n, 2), num_pages=n * 4 + 8)
    e.generate_weights(po.Q4_0, po.Q4_0, po.Q4_0, True, True, 3)
    e.finalize()
    path = str(tmp_path / "qwen25_3b_q4.qraf")
    bench.write_qraf_synthetic(path, q, po.Q4_0, 3, dict(call=call, DeviceBuffer=DeviceBuffer, stream=Stream()))
    print("file written; reference loading", flush=True)
    ref = po.RefModel(path, V)
    rng = np.random.default_rng(2025)
    seqs = [e.seq_create() for _ in range(n)]
    tok0 = [int(t) for t in rng.integers(0, V, 4)]  # sequence 0's prompt
    want_logits = np.zeros(n, np.uint8)
    want_logits[0] = 1
    try:
        for pos in range(len(tok0) - 1 + GEN):
            t0 = tok0[pos]
            toks = [t0] + rng.integers(0, V, n - 1).tolist()
            lg, nx = e.step(seqs, toks, [pos] * n, want_logits=want_logits, logits=True, argmax=True)
            want = ref.forward(t0, pos)
            print(f"position {pos}: max |diff| {np.abs(lg[0] - want).max():.2e}", flush=True)
            check_logits(lg[0], want, f"sequence 0 position {pos}")
            greedy = int(np.argmax(want))  # Sampler::argmax: first index of the maximum
            assert int(nx[0]) == greedy, f"position {pos}: greedy {nx[0]} vs reference {greedy}"
            if pos >= 3:
                tok0.append(greedy)
    finally:
        ref.close()
        e.close()
