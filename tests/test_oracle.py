"""Pins the CPU oracle (oracle/oracle.c) before anything is compared with it.

Each oracle function is checked against (a) golden vectors written by the
compiled reference (tests/golden/gen_golden.py), (b) the compiled reference
itself when oracle/_ref is built, and (c) closed forms / brute force that a
plausible mistake (dropped term, wrong sign, swapped nibble, wrong GQA
mapping) would fail.
"""
import os
import tempfile

import numpy as np
import pytest

from tests.conftest import golden
from oracle import pyoracle as po

L = po.lib()


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def same_bits(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return bool(np.all((bits(a) == bits(b)) | (np.isnan(a) & np.isnan(b))))


# ------------------------------------------------------------------ fp16

def test_fp16_decode_exhaustive_ieee_and_golden():
    g = golden("fp16.npz")
    codes = np.arange(65536, dtype=np.uint32)
    ours = np.array([L.or_fp16_to_fp32(int(h)) for h in codes], np.float32)
    ieee = codes.astype(np.uint16).view(np.float16).astype(np.float32)
    fin = np.isfinite(ieee)
    assert same_bits(ours[fin], ieee[fin])          # every finite code incl. subnormals, exact
    assert np.all(np.isinf(ours[np.isinf(ieee)]))
    assert np.all(np.isnan(ours[np.isnan(ieee)]))
    assert np.array_equal(bits(ours), bits(g["dec"]))  # bit-exact vs reference incl. NaN payloads


def test_fp16_encode_golden_and_closed_form():
    g = golden("fp16.npz")
    enc = np.array([L.or_fp32_to_fp16(float(v)) for v in g["vals"]], np.uint16)
    assert np.array_equal(enc, g["enc"])
    # closed form of the truncating, flush-to-zero encoder (dtype.cpp:39-59)
    v = g["vals"]
    b = bits(v)
    e = ((b >> 23) & 0xFF).astype(np.int64) - 127
    exp_form = np.where(e > 15, ((b >> 16) & 0x8000) | 0x7C00,
                        np.where(e > -15, ((b >> 16) & 0x8000) | ((e + 15) << 10) | ((b & 0x7FFFFF) >> 13),
                                 (b >> 16) & 0x8000)).astype(np.uint16)
    assert np.array_equal(enc, exp_form)


# ------------------------------------------------------------------ quantizers

@pytest.mark.parametrize("dt", [po.Q8_0, po.Q4_0])
@pytest.mark.parametrize("bs", [32, 8, 4])
@pytest.mark.parametrize("tag", ["rand", "special"])
def test_quantize_dequantize_dot_golden(dt, bs, tag):
    g = golden("quant.npz")
    k = f"{dt}_{bs}_{tag}"
    x = g["x_" + k]
    q = po.quantize(dt, x, bs)
    assert np.array_equal(q, g["q_" + k]), "quantizer bytes differ from the reference"
    assert same_bits(po.dequantize(dt, q, x.size, bs), g["deq_" + k])
    d = po.dot(dt, q, g["xs_" + k], bs)
    assert same_bits(d, g["dot_" + k])


def test_reference_known_answer():
    # tests/test_quantize.cpp:40-50: [1,2,3,4] . [0.5]*4 ~= 5.0 (+-0.1)
    q = po.quantize(po.Q8_0, np.array([1, 2, 3, 4], np.float32), 4)
    d = po.dot(po.Q8_0, q, np.full(4, 0.5, np.float32), 4)
    assert abs(d - 5.0) < 0.1
    assert same_bits(d, golden("quant.npz")["kat_q8_dot"])


def test_quantizer_closed_form():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(32 * 200) * 0.02).astype(np.float32)
    x[:32] = 0
    q8 = po.quantize(po.Q8_0, x).reshape(-1, 36)
    sc = q8[:, :4].copy().view(np.float32)[:, 0]
    qs = q8[:, 4:].view(np.int8).astype(np.int32)
    xb = x.reshape(-1, 32)
    amax = np.abs(xb).max(1)
    assert np.array_equal(bits(sc), bits(amax / np.float32(127)))
    assert np.all(np.abs(qs) <= 127) and sc[0] == 0 and not qs[0].any()
    inv = np.where(sc > 0, np.float32(1) / sc, np.float32(0)).astype(np.float32)
    v = np.clip(xb * inv[:, None], -127, 127)
    expect = np.sign(v) * np.floor(np.abs(v) + 0.5)  # round half away from zero
    assert np.array_equal(qs, expect.astype(np.int32))
    q4 = po.quantize(po.Q4_0, x).reshape(-1, 18)
    nib = np.stack([q4[:, 2:] & 15, q4[:, 2:] >> 4], -1).reshape(-1, 32).astype(np.int32)
    assert nib[1:].min() >= 1 and nib.max() <= 15  # -8 never produced for finite input
    s4 = q4[:, :2].copy().view(np.uint16)[:, 0]
    inv4 = np.where(amax / np.float32(7) > 0, np.float32(1) / (amax / np.float32(7)), 0).astype(np.float32)
    v4 = np.clip(np.sign(xb * inv4[:, None]) * np.floor(np.abs(xb * inv4[:, None]) + 0.5), -8, 7)
    assert np.array_equal(nib[1:] - 8, v4[1:].astype(np.int32))  # even elem = low nibble
    assert s4[0] == 0


def test_dot_closed_forms():
    rng = np.random.default_rng(4)
    w = (rng.standard_normal(256) * 0.02).astype(np.float32)
    for dt in (po.Q8_0, po.Q4_0):
        q = po.quantize(dt, w)
        deq = po.dequantize(dt, q, 256)
        for i in (0, 31, 32, 200, 255):  # one-hot x picks (f32)q_i * scale exactly
            e = np.zeros(256, np.float32)
            e[i] = 1
            assert same_bits(po.dot(dt, q, e), deq[i])
        x = rng.standard_normal(256).astype(np.float32)
        exact = float(np.dot(deq.astype(np.float64), x.astype(np.float64)))
        bound = 260 * 2.0 ** -24 * float(np.abs(deq.astype(np.float64) * x).sum())
        assert abs(po.dot(dt, q, x) - exact) <= bound
        # a swapped nibble order would break the one-hot identity above
        if dt == po.Q4_0:
            swapped = q.copy().reshape(-1, 18)
            swapped[:, 2:] = (swapped[:, 2:] >> 4) | ((swapped[:, 2:] & 15) << 4)
            e = np.zeros(256, np.float32)
            e[0] = 1
            assert not same_bits(po.dot(dt, swapped.ravel(), e), deq[0]) or deq[0] == deq[1]


# ------------------------------------------------------------------ matvec

def test_matvec_golden():
    g = golden("matvec.npz")
    for key in [k[2:] for k in g.files if k.startswith("w_")]:
        dt, n, k, bs = (int(v) for v in key.split("_"))
        y = po.matvec_q(g["w_" + key], dt, n, k, g["x_" + key], bs)
        assert same_bits(y, g["y_" + key]), key
    assert same_bits(po.matvec_f32(g["f32_W"], g["f32_x"]), g["f32_y"])


def test_matvec_unknown_dtype_zero_fills():
    y = np.full(4, 7, np.float32)
    rc = L.or_matvec_q(np.zeros(64, np.uint8).ctypes.data, 99, 32, 4, 32,
                       np.ones(32, np.float32).ctypes.data_as(po._fp), y.ctypes.data_as(po._fp))
    assert rc == -1 and not y.any()  # backend.cpp:195-198


# ------------------------------------------------------------------ elementwise

def test_ops_golden():
    g = golden("ops.npz")
    x = g["rms_x"].copy()
    L.or_rms_norm(x.ctypes.data_as(po._fp), g["rms_w"].ctypes.data_as(po._fp), x.size, 1e-5)
    assert same_bits(x, g["rms_y"])  # sqrtf is correctly rounded: exact anywhere
    s = g["sm_x"].copy()
    L.or_softmax(s.ctypes.data_as(po._fp), s.size)
    np.testing.assert_allclose(s, g["sm_y"], rtol=2e-6, atol=0)  # libm expf
    h = g["silu_x"].copy()
    L.or_silu(h.ctypes.data_as(po._fp), h.size)
    np.testing.assert_allclose(h, g["silu_y"], rtol=2e-6, atol=1e-30)
    for key in [k[7:] for k in g.files if k.startswith("rope_q_")]:
        hd, pos = (int(v) for v in key.split("_"))
        for src, dst in (("rope_q_", "rope_qo_"), ("rope_k_", "rope_ko_")):
            v = g[src + key].copy()
            L.or_rope(v.ctypes.data_as(po._fp), hd, pos, float(g["rope_theta_" + key]))
            np.testing.assert_allclose(v, g[dst + key], rtol=1e-5, atol=1e-6)
    assert L.or_argmax(g["am_x"].ctypes.data_as(po._fp), g["am_x"].size) == int(g["am_i"]) == 17
    p = g["pen_x"].copy()
    t = g["pen_t"]
    L.or_repetition_penalty(p.ctypes.data_as(po._fp), p.size, t.ctypes.data_as(po._u32p), t.size, 1.1)
    assert same_bits(p, g["pen_y"])


def test_elementwise_closed_forms():
    x = np.array([1, 2, 3, 4], np.float32)
    L.or_softmax(x.ctypes.data_as(po._fp), 4)
    e = np.exp(np.arange(4) - 3.0)
    np.testing.assert_allclose(x, e / e.sum(), rtol=1e-6)
    v = np.random.default_rng(0).standard_normal(64).astype(np.float32)
    r = v.copy()
    L.or_rope(r.ctypes.data_as(po._fp), 64, 0, 1e4)
    assert same_bits(r, v)  # pos 0 is the identity (tests/test_nn_ops.cpp:85-95)
    L.or_rope(r.ctypes.data_as(po._fp), 64, 123, 1e4)
    n0 = np.hypot(v[0::2], v[1::2])
    n1 = np.hypot(r[0::2], r[1::2])
    np.testing.assert_allclose(n0, n1, rtol=1e-5)  # rotation keeps each pair's norm
    ang = np.arctan2(r[1::2], r[0::2]) - np.arctan2(v[1::2], v[0::2])
    want = 123 * (1e4 ** (-np.arange(0, 64, 2) / 64.0))
    np.testing.assert_allclose(np.cos(ang), np.cos(want), atol=2e-4)  # interleaved pairs, angle pos*freq


def _attention_f64(q, K, V, H, Hkv, hd, kv_map=None):
    rep = H // Hkv
    out = np.zeros(H * hd)
    for h in range(H):
        kh = (h // rep) if kv_map is None else kv_map(h)
        k = K[:, kh * hd:(kh + 1) * hd].astype(np.float64)
        v = V[:, kh * hd:(kh + 1) * hd].astype(np.float64)
        s = k @ q[h * hd:(h + 1) * hd].astype(np.float64) / np.sqrt(hd)
        p = np.exp(s - s.max())
        out[h * hd:(h + 1) * hd] = (p / p.sum()) @ v
    return out


def test_attention_vs_textbook_f64():
    rng = np.random.default_rng(8)
    H, Hkv, hd, ctx = 16, 2, 128, 300
    q = rng.standard_normal(H * hd).astype(np.float32)
    K = rng.standard_normal((ctx, Hkv * hd)).astype(np.float32)
    V = rng.standard_normal((ctx, Hkv * hd)).astype(np.float32)
    ours = po.attention_decode(q, K, V, H, Hkv, hd)
    ref = _attention_f64(q, K, V, H, Hkv, hd)
    np.testing.assert_allclose(ours, ref, rtol=1e-4, atol=2e-5)
    wrong = _attention_f64(q, K, V, H, Hkv, hd, kv_map=lambda h: h % Hkv)  # planted GQA mistake
    assert np.abs(wrong - ours).max() > 1e-2


# ------------------------------------------------------------------ synthetic weights

def test_generator_moments_and_determinism():
    a = po.gen_normal(5, 77, 1 << 20, 0.02)
    b = po.gen_normal(5, 77, 1 << 20, 0.02)
    assert np.array_equal(bits(a), bits(b))
    assert abs(a.mean()) < 1e-4 and abs(a.std() - 0.02) < 2e-4
    kurt = ((a / a.std()) ** 4).mean()
    assert 2.7 < kurt < 3.0  # 8-term Irwin-Hall: 3 - 1.2/8 = 2.85
    c = po.gen_normal(5, 78, 1 << 10, 0.02)
    assert not np.array_equal(a[:1024], c)
    toks = [L.or_gen_token(3, i, 1000) for i in range(5000)]
    assert min(toks) >= 0 and max(toks) < 1000 and len(set(toks)) > 900


# ------------------------------------------------------------------ model

@pytest.mark.parametrize("name", ["model_q8_llama", "model_q4_qwen2", "model_f32_llama"])
def test_model_forward_and_greedy_golden(name):
    from tests.golden.gen_golden import MODELS
    g = golden(name + ".npz")
    kw, seed, np_, nlog, ngen = MODELS[name]
    m = po.Model(po.make_config(**kw), seed)
    prompt = g["prompt"]
    assert np.array_equal(prompt, [L.or_gen_token(seed, i, kw["vocab"]) for i in range(np_)])
    m.reset()
    for i in range(nlog):
        assert same_bits(m.forward(int(prompt[i]), i), g["logits"][i]), f"logits differ at position {i}"
    assert m.generate(prompt, ngen, 1.0, eos=2) == g["stream"].tolist()
    assert m.generate(prompt, ngen, 1.1, eos=2) == g["stream_pen"].tolist()
    m.close()


# ------------------------------------------------------------------ against the compiled reference

needs_ref = pytest.mark.skipif(po.ref() is None, reason="oracle/_ref not built (no reference checkout)")


@needs_ref
def test_oracle_vs_reference_random():
    R = po.ref()
    rng = np.random.default_rng(21)
    for trial in range(20):
        dt = (po.Q8_0, po.Q4_0)[trial % 2]
        n, k = int(rng.integers(1, 40)), int(rng.integers(1, 700))
        bs = int(rng.choice([32, 32, 16, 8, 4]))
        w = (rng.standard_normal(n * k) * rng.choice([0.02, 1, 300])).astype(np.float32)
        wq = np.concatenate([po.quantize(dt, w[i * k:(i + 1) * k], bs) for i in range(n)])
        x = rng.standard_normal(k).astype(np.float32)
        y = np.zeros(n, np.float32)
        R.ref_matvec_q(wq.ctypes.data, dt, bs, n, k, x.ctypes.data_as(po._fp), y.ctypes.data_as(po._fp))
        assert same_bits(po.matvec_q(wq, dt, n, k, x, bs), y)


@needs_ref
def test_oracle_vs_reference_model_gqa8():
    cfg = po.make_config(vocab=700, hidden=256, layers=3, heads=16, kv_heads=2, inter=320, max_seq=64,
                         rope_theta=1e6, eps=1e-6, wdtype=po.Q4_0, tied=True, qkv_bias=True)
    m = po.Model(cfg, 31)
    path = os.path.join(tempfile.mkdtemp(), "m.qraf")
    m.write_qraf(path)
    rm = po.RefModel(path, 700)
    for pos, tok in enumerate([5, 699, 0, 42, 42, 7, 100]):
        assert same_bits(m.forward(tok, pos), rm.forward(tok, pos))
    rm.close()
    m.close()


@needs_ref
@pytest.mark.parametrize("bs,dt", [(8, po.Q8_0), (16, po.Q4_0), (4, po.Q4_0)])
def test_oracle_vs_reference_model_block_sizes(bs, dt):
    """The oracle's model at quant block sizes other than 32 (its weights
    written to a .qraf file whose quant scheme carries the block size, read
    back by the compiled reference's own loader): forward logits bit-identical
    at every position."""
    cfg = po.make_config(vocab=300, hidden=128, layers=2, heads=4, kv_heads=2, inter=192, max_seq=64,
                         rope_theta=1e5, eps=1e-5, wdtype=dt, tied=(dt == po.Q4_0), block_size=bs)
    m = po.Model(cfg, 40 + bs)
    path = os.path.join(tempfile.mkdtemp(), "m.qraf")
    m.write_qraf(path)
    rm = po.RefModel(path, 300)
    for pos, tok in enumerate([5, 299, 0, 42, 42, 7]):
        assert same_bits(m.forward(tok, pos), rm.forward(tok, pos)), f"position {pos}"
    rm.close()
    m.close()
