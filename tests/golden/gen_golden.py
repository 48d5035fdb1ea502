"""Write the golden fixtures under tests/golden/ from the compiled reference.

Runs the reference implementation itself (oracle/_ref/libqraf_ref.so, built
by oracle/Makefile from the reference's own sources) on seeded inputs and
stores inputs + outputs as .npz data files.  Run from the repository root:

    make -C oracle all && python tests/golden/gen_golden.py

Fixtures:
  quant.npz     quantize_q8_0 / quantize_q4_0 bytes (block sizes 32, 8, 4;
                special values), dequantize_tensor, dot_q8_0_f32 / dot_q4_0_f32
  fp16.npz      fp32_to_fp16 on special and random values; fp16_to_fp32 of all codes
  matvec.npz    dispatch_matvec_q at small shapes incl. K = 576 and ragged K;
                dispatch_matvec_opt
  ops.npz       rms_norm / softmax / silu / rope / argmax / repetition penalty
  model_*.npz   Transformer::forward logits for a few positions and the greedy
                stream of InferenceEngine::generate_tokens, for tiny models
                built from the repo's synthetic weights (Q8 llama, Q4 qwen2
                tied+bias, F32 llama)
"""
from __future__ import annotations

import ctypes as C
import os
import sys
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import pyoracle as po  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))
fp = po._fp


def special_vector(rng, n):
    x = (rng.standard_normal(n) * rng.choice([1e-3, 0.02, 1.0, 50.0], n)).astype(np.float32)
    x[:8] = [0, -0.0, 1e-8, -1e-8, 3.4e38, 1e-40, 0.5, -0.5]
    x[40:72] = 0.0  # an all-zero block
    x[100] = np.nan
    x[130] = np.inf
    x[131] = -np.inf
    return x


def gen_quant(R):
    rng = np.random.default_rng(1234)
    d = {}
    for dt in (po.Q8_0, po.Q4_0):
        for bs in (32, 8, 4):
            for tag, x in (("rand", rng.standard_normal(997).astype(np.float32) * 0.05),
                           ("special", special_vector(rng, 300))):
                nbytes = po.lib().or_q_tensor_bytes(dt, x.size, bs)
                q = np.zeros(nbytes, np.uint8)
                R.ref_quantize(dt, x.ctypes.data_as(fp), x.size, bs, q.ctypes.data_as(po._u8p))
                deq = np.zeros(x.size, np.float32)
                R.ref_dequantize(q.ctypes.data, dt, x.size, bs, deq.ctypes.data_as(fp))
                xs = rng.standard_normal(x.size).astype(np.float32)
                dot = R.ref_dot(dt, q.ctypes.data, xs.ctypes.data_as(fp), x.size, bs)
                k = f"{dt}_{bs}_{tag}"
                d["x_" + k], d["q_" + k], d["deq_" + k] = x, q, deq
                d["xs_" + k], d["dot_" + k] = xs, np.float32(dot)
    # the reference's own test vector (tests/test_quantize.cpp:40-50)
    a = np.array([1, 2, 3, 4], np.float32)
    b = np.array([0.5] * 4, np.float32)
    q = np.zeros(8, np.uint8)
    R.ref_quantize(po.Q8_0, a.ctypes.data_as(fp), 4, 4, q.ctypes.data_as(po._u8p))
    d["kat_q8_dot"] = np.float32(R.ref_dot(po.Q8_0, q.ctypes.data, b.ctypes.data_as(fp), 4, 4))
    np.savez_compressed(os.path.join(OUT, "quant.npz"), **d)


def gen_fp16(R):
    rng = np.random.default_rng(7)
    vals = np.concatenate([
        np.array([0, -0.0, 1.0, -1.0, 65504, 65520, 1e5, -1e5, 6.1e-5, 6.0e-5, 2 ** -14, 2 ** -15, 2 ** -24,
                  np.inf, -np.inf, np.nan, 0.1, 1 / 3], np.float32),
        (rng.standard_normal(2000) * np.exp(rng.uniform(-20, 12, 2000))).astype(np.float32)]).astype(np.float32)
    enc = np.array([R.ref_fp32_to_fp16(float(v)) for v in vals], np.uint16)
    dec = np.array([R.ref_fp16_to_fp32(h) for h in range(65536)], np.float32)
    np.savez_compressed(os.path.join(OUT, "fp16.npz"), vals=vals, enc=enc, dec=dec)


def gen_matvec(R):
    rng = np.random.default_rng(99)
    d = {}
    for dt in (po.Q8_0, po.Q4_0):
        for (n, k, bs) in ((64, 576, 32), (33, 100, 32), (16, 2048, 32), (7, 45, 8), (5, 19, 4), (3, 31, 32)):
            w = (rng.standard_normal(n * k) * 0.02).astype(np.float32)
            # quantised per row, as every tensor the path reads
            rows = [po.quantize(dt, w[i * k:(i + 1) * k], bs) for i in range(n)]
            wq = np.concatenate(rows)
            x = rng.standard_normal(k).astype(np.float32)
            y = np.zeros(n, np.float32)
            R.ref_matvec_q(wq.ctypes.data, dt, bs, n, k, x.ctypes.data_as(fp), y.ctypes.data_as(fp))
            key = f"{dt}_{n}_{k}_{bs}"
            d["w_" + key], d["x_" + key], d["y_" + key] = wq, x, y
    W = rng.standard_normal((40, 96)).astype(np.float32)
    x = rng.standard_normal(96).astype(np.float32)
    y = np.zeros(40, np.float32)
    R.ref_matvec_f32(W.ctypes.data_as(fp), x.ctypes.data_as(fp), y.ctypes.data_as(fp), 40, 96)
    d["f32_W"], d["f32_x"], d["f32_y"] = W, x, y
    np.savez_compressed(os.path.join(OUT, "matvec.npz"), **d)


def gen_ops(R):
    rng = np.random.default_rng(5)
    d = {}
    x = rng.standard_normal(576).astype(np.float32) * 3
    w = rng.uniform(0.5, 1.5, 576).astype(np.float32)
    y = x.copy()
    R.ref_rms_norm(y.ctypes.data_as(fp), w.ctypes.data_as(fp), 576, 1e-5)
    d["rms_x"], d["rms_w"], d["rms_y"] = x, w, y
    s = (rng.standard_normal(1000) * 4).astype(np.float32)
    t = s.copy()
    R.ref_softmax(t.ctypes.data_as(fp), 1000)
    d["sm_x"], d["sm_y"] = s, t
    g = (rng.standard_normal(1536) * 4).astype(np.float32)
    h = g.copy()
    R.ref_silu(h.ctypes.data_as(fp), 1536)
    d["silu_x"], d["silu_y"] = g, h
    for hd, pos, theta in ((64, 0, 1e5), (64, 17, 1e5), (128, 1000, 1e6), (128, 4095, 1e6), (16, 3, 1e4)):
        q = rng.standard_normal(hd).astype(np.float32)
        k = rng.standard_normal(hd).astype(np.float32)
        q2, k2 = q.copy(), k.copy()
        R.ref_rope(q2.ctypes.data_as(fp), k2.ctypes.data_as(fp), hd, pos, theta)
        key = f"{hd}_{pos}"
        d["rope_q_" + key], d["rope_k_" + key], d["rope_qo_" + key], d["rope_ko_" + key] = q, k, q2, k2
        d["rope_theta_" + key] = np.float32(theta)
    lg = rng.standard_normal(5000).astype(np.float32)
    lg[17] = lg[4000] = lg.max() + 1  # tie: lowest index wins
    d["am_x"], d["am_i"] = lg, np.uint32(R.ref_argmax(lg.ctypes.data_as(fp), 5000))
    toks = np.array([3, 3, 17, 4999, 5000, 12], np.uint32)
    pl = lg.copy()
    R.ref_penalty(pl.ctypes.data_as(fp), 5000, toks.ctypes.data_as(po._u32p), toks.size, 1.1)
    d["pen_x"], d["pen_t"], d["pen_y"] = lg, toks, pl
    np.savez_compressed(os.path.join(OUT, "ops.npz"), **d)


MODELS = {
    # name: (make_config kwargs, seed, prompt length, n positions of logits, greedy tokens)
    "model_q8_llama": (dict(vocab=512, hidden=64, layers=2, heads=4, kv_heads=2, inter=128, max_seq=128,
                            rope_theta=1e5, eps=1e-5, wdtype=po.Q8_0), 11, 8, 8, 32),
    "model_q4_qwen2": (dict(vocab=640, hidden=128, layers=2, heads=4, kv_heads=1, inter=160, max_seq=128,
                            rope_theta=1e6, eps=1e-6, wdtype=po.Q4_0, tied=True, qkv_bias=True), 12, 6, 6, 32),
    "model_f32_llama": (dict(vocab=300, hidden=64, layers=2, heads=2, kv_heads=2, inter=96, max_seq=128,
                             rope_theta=1e4, eps=1e-5, wdtype=po.F32), 13, 5, 5, 24),
}


def gen_models():
    tmp = tempfile.mkdtemp()
    for name, (kw, seed, np_, nlog, ngen) in MODELS.items():
        cfg = po.make_config(**kw)
        m = po.Model(cfg, seed)
        path = os.path.join(tmp, name + ".qraf")
        m.write_qraf(path)
        prompt = np.array([po.lib().or_gen_token(seed, i, cfg.vocab) for i in range(np_)], np.uint32)
        rm = po.RefModel(path, cfg.vocab)
        logits = np.stack([rm.forward(int(prompt[i]), i) for i in range(nlog)])
        rm.close()
        eng = po.RefEngine(path)
        stream, _ = eng.generate(prompt, ngen, 1.0)
        stream_pen, _ = eng.generate(prompt, ngen, 1.1)
        eng.close()
        cfg_arr = np.array([kw.get(k, 0) for k in ("vocab", "hidden", "layers", "heads", "kv_heads", "inter",
                                                   "max_seq")], np.uint32)
        np.savez_compressed(os.path.join(OUT, name + ".npz"), config=cfg_arr, seed=np.uint64(seed), prompt=prompt,
                            logits=logits, stream=np.array(stream, np.uint32),
                            stream_pen=np.array(stream_pen, np.uint32))


def main():
    R = po.ref()
    if R is None:
        sys.exit("oracle/_ref/libqraf_ref.so is not built: run `make -C oracle all` first")
    gen_quant(R)
    gen_fp16(R)
    gen_matvec(R)
    gen_ops(R)
    gen_models()
    print("golden fixtures written to", OUT)


if __name__ == "__main__":
    main()
