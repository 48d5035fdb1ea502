"""Golden streams of the continuous-batch workload, written by the compiled
reference: the Qwen2.5-3B architecture (36 layers, hidden 2048, 16 / 2
heads, FFN 11008, vocab 151936, tied Q4 embedding, QKV bias), Q4 weights of
the repo's synthetic generator (seed 3), decoded by the reference's own
QrafModel + Transformer (oracle/_ref, src/nn/transformer.cpp:573-643) one
sequence at a time, as InferenceEngine::generate_tokens does
(src/runtime/inference.cpp:68-159: prompt token by token, then greedy).

The workload (c5_workload) is 160 requests with seeded prompt lengths
U[16, 512], output lengths U[64, 256] and uniform token ids; 128 run at once
and the rest are admitted as others finish.  For the requests in CHECKED
(the first two admitted, and the last two, which enter only after earlier
requests retire and free their KV pages) this script stores, for each of
the first GEN greedy tokens, the logits that chose it: the top-16 indices
and values, the values at 64 fixed random indices, and the gap between the
two largest logits.  The GPU test runs the whole workload through the
engine's scheduler and compares those sequences with these records.

Run from the repository root (about 15 minutes on 4 cores):

    make -C oracle all && python tests/golden/gen_c5_golden.py
"""
from __future__ import annotations

import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c5_qwen25_3b_q4.npz")

QWEN = dict(vocab=151936, hidden=2048, layers=36, heads=16, kv_heads=2, inter=11008, max_seq=1024, rope_theta=1e6,
            eps=1e-6)
WEIGHT_SEED = 3
WORKLOAD_SEED = 11
N_REQUESTS = 160
CHECKED = (0, 1, 158, 159)
GEN = 32      # greedy tokens compared per checked request
TOPK = 16     # largest logits stored per position
NPROBE = 64   # fixed random logit indices stored per position


def c5_workload(seed=WORKLOAD_SEED, n=N_REQUESTS, vocab=QWEN["vocab"]):
    """[(prompt token ids, max generated tokens)] in submission order."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        plen, olen = int(rng.integers(16, 513)), int(rng.integers(64, 257))
        out.append((rng.integers(0, vocab, plen).tolist(), olen))
    return out


def probe_indices(vocab=QWEN["vocab"]):
    return np.sort(np.random.default_rng(WORKLOAD_SEED + 1).choice(vocab, NPROBE, replace=False)).astype(np.int64)


def _decode(args):
    """The reference's greedy decode of one request: every logit vector that
    picks one of the first GEN tokens, summarised."""
    path, prompt = args
    sys.path.insert(0, ROOT)
    from oracle import pyoracle as po
    V = QWEN["vocab"]
    probe = probe_indices(V)
    ref = po.RefModel(path, V)
    t0 = time.perf_counter()
    try:
        for pos, t in enumerate(prompt):
            lg = ref.forward(t, pos)
        toks, idx, val, gaps = [], [], [], []
        pos = len(prompt)
        while True:
            top = np.argsort(-lg, kind="stable")[:TOPK]  # stable: equal values keep the lower index first
            nxt = int(np.argmax(lg))  # Sampler::argmax: first index of the maximum
            assert nxt == int(top[0])
            toks.append(nxt)
            idx.append(np.concatenate([top, probe]))
            val.append(lg[idx[-1]])
            s = np.sort(lg)
            gaps.append(float(s[-1] - s[-2]))
            if len(toks) == GEN:
                break
            lg = ref.forward(nxt, pos)
            pos += 1
    finally:
        ref.close()
    secs = time.perf_counter() - t0
    return (np.array(toks, np.int32), np.array(idx, np.int32), np.array(val, np.float32), np.array(gaps, np.float32),
            secs, len(prompt) + GEN - 1)


def main():
    import multiprocessing as mp
    sys.path.insert(0, ROOT)
    from oracle import pyoracle as po
    work = c5_workload()
    tmp = tempfile.mkdtemp()
    path = os.path.join(tmp, "qwen25_3b_q4.qraf")
    m = po.Model(po.make_config(wdtype=po.Q4_0, tied=True, qkv_bias=True, **QWEN), WEIGHT_SEED)
    m.write_qraf(path)
    m.close()
    print("model written", flush=True)
    try:
        with mp.get_context("fork").Pool(len(CHECKED)) as pool:
            res = pool.map(_decode, [(path, work[i][0]) for i in CHECKED])
    finally:
        os.remove(path)
        os.rmdir(tmp)
    d = dict(weight_seed=WEIGHT_SEED, workload_seed=WORKLOAD_SEED, n_requests=N_REQUESTS,
             checked=np.array(CHECKED, np.int32), probe=probe_indices())
    for i, (toks, idx, val, gaps, secs, fwd) in zip(CHECKED, res):
        d[f"prompt_{i}"] = np.array(work[i][0], np.int32)
        d[f"tokens_{i}"] = toks
        d[f"idx_{i}"] = idx
        d[f"val_{i}"] = val
        d[f"gap_{i}"] = gaps
        d[f"cpu_s_per_forward_{i}"] = np.float64(secs / fwd)
        print(f"request {i}: prompt {len(work[i][0])}, {fwd} forwards in {secs:.0f} s, "
              f"min top-2 gap {gaps.min():.2e}, tokens {toks[:8].tolist()}...", flush=True)
    np.savez_compressed(OUT, **d)
    print("wrote", OUT)


if __name__ == "__main__":
    main()
