"""The oracle's restatement of the int8 KV scheme (kv_cache_quant.h, which
the reference defines but does not use) against the compiled header:
QuantizedKVCache::store bytes and scales, dot_with_key and dequant_value bit
for bit; and the int8 attention restatement at one position (softmax of one
score is 1, so the output is the dequantized V row exactly) and against the
fp32 attention on the dequantized cache (tolerance of the K rounding).
"""
import ctypes as C

import numpy as np
import pytest

from oracle import pyoracle as po

need_ref = pytest.mark.skipif(po.ref() is None, reason="oracle/_ref (the compiled reference) is not built")
fp = C.POINTER(C.c_float)


def heads(rng, Hkv, hd, kind):
    x = rng.standard_normal((Hkv, hd)).astype(np.float32)
    if kind == "zero_head":
        x[0] = 0.0
    elif kind == "wide":
        x *= np.float32(1e4)
        x[:, 3] = np.float32(-2.5e4)
    elif kind == "halves":  # x * inv lands on .5 steps: round half away from zero
        x = (np.arange(Hkv * hd, dtype=np.float32).reshape(Hkv, hd) % 9 - 4) * np.float32(0.5)
        x[:, 0] = np.float32(127 * 0.5)
    return x


@need_ref
@pytest.mark.parametrize("kind", ["normal", "zero_head", "wide", "halves"])
@pytest.mark.parametrize("Hkv,hd", [(2, 128), (3, 64), (1, 32)])
def test_store_dot_dequant_equal_reference(kind, Hkv, hd):
    rng = np.random.default_rng(hd + Hkv)
    k, v = heads(rng, Hkv, hd, kind), heads(rng, Hkv, hd, kind)[::-1].copy()
    query = rng.standard_normal((Hkv, hd)).astype(np.float32)
    kq, vq = np.zeros((Hkv, hd), np.int8), np.zeros((Hkv, hd), np.int8)
    ks, vs = np.zeros(Hkv, np.float32), np.zeros(Hkv, np.float32)
    dots, vdeq = np.zeros(Hkv, np.float32), np.zeros((Hkv, hd), np.float32)
    po.ref().ref_kv_quant(k.ctypes.data_as(fp), v.ctypes.data_as(fp), Hkv, hd, query.ctypes.data_as(fp), kq.ctypes.data,
                          ks.ctypes.data_as(fp), vq.ctypes.data, vs.ctypes.data_as(fp), dots.ctypes.data_as(fp),
                          vdeq.ctypes.data_as(fp))
    okq, oks = po.kv_quant_heads(k, Hkv, hd)
    ovq, ovs = po.kv_quant_heads(v, Hkv, hd)
    assert np.array_equal(okq, kq) and np.array_equal(oks, ks)
    assert np.array_equal(ovq, vq) and np.array_equal(ovs, vs)
    L = po.lib()
    for h in range(Hkv):
        assert L.or_kv_dot_key(okq[h].ctypes.data, float(oks[h]), query[h].ctypes.data_as(fp), hd) == dots[h]
        # attention at one position: out = 1 * dequant_value(V)
        out = po.attention_decode_i8(query[h], okq[h:h + 1].reshape(1, 1, hd), oks[h:h + 1].reshape(1, 1),
                                     ovq[h:h + 1].reshape(1, 1, hd), ovs[h:h + 1].reshape(1, 1), 1, 1, hd)
        assert np.array_equal(out, vdeq[h])


def test_attention_i8_close_to_fp32_on_dequantized_cache():
    rng = np.random.default_rng(3)
    H, Hkv, hd, ctx = 8, 2, 64, 300
    K = rng.standard_normal((ctx, Hkv, hd)).astype(np.float32)
    V = rng.standard_normal((ctx, Hkv, hd)).astype(np.float32)
    q = rng.standard_normal(H * hd).astype(np.float32)
    K8, Ks, V8, Vs = [], [], [], []
    for t in range(ctx):
        a, b = po.kv_quant_heads(K[t], Hkv, hd)
        c, d = po.kv_quant_heads(V[t], Hkv, hd)
        K8.append(a), Ks.append(b), V8.append(c), Vs.append(d)
    K8, Ks, V8, Vs = map(np.array, (K8, Ks, V8, Vs))
    got = po.attention_decode_i8(q, K8, Ks, V8, Vs, H, Hkv, hd)
    Kd = (K8.astype(np.float32) * Ks[:, :, None]).astype(np.float32)
    Vd = (V8.astype(np.float32) * Vs[:, :, None]).astype(np.float32)
    want = po.attention_decode(q, Kd.reshape(ctx, -1), Vd.reshape(ctx, -1), H, Hkv, hd)
    assert np.allclose(got, want, rtol=1e-4, atol=1e-5)
    # and within int8 rounding of the unquantized attention
    full = po.attention_decode(q, K.reshape(ctx, -1), V.reshape(ctx, -1), H, Hkv, hd)
    assert np.abs(got - full).max() < 0.05


def test_model_with_int8_cache_stays_near_f32_cache():
    """The oracle model with QuantizedKVCache in place of KVCache: position 0
    attends to itself only, so its attention output is the dequantized V row
    and its logits move by the V rounding alone; over a prompt the logits stay
    within the int8 rounding of the f32 cache's (a dropped scale or a
    transposed cache index would move them by O(1))."""
    kw = dict(vocab=500, hidden=256, layers=2, heads=4, kv_heads=2, inter=512, max_seq=64, rope_theta=1e4,
              eps=1e-5, wdtype=po.Q8_0)
    a, b = po.Model(po.make_config(**kw), 5), po.Model(po.make_config(**kw), 5)
    b.set_kv_int8()
    toks = [po.lib().or_gen_token(5, i, kw["vocab"]) for i in range(12)]
    worst = 0.0
    for pos, t in enumerate(toks):
        la, lb = a.forward(t, pos), b.forward(t, pos)
        assert not np.array_equal(la, lb)
        worst = max(worst, float(np.abs(la - lb).max() / np.abs(la).max()))
    assert worst < 0.03, worst
    b.reset()
    lb0 = b.forward(toks[0], 0)
    a.reset()
    assert np.abs(a.forward(toks[0], 0) - lb0).max() / np.abs(lb0).max() < 0.03
    a.close()
    b.close()
