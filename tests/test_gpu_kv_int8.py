"""int8 KV pages on the device against the oracle's restatement of
QuantizedKVCache (kv_cache_quant.h), itself pinned bit for bit against the
compiled header in test_oracle_kv8.py.

- The quantizing append (bias + RoPE + store) writes the reference's bytes
  and scales exactly: the same rotated values, the same absmax, divisions and
  round-half-away-from-zero.
- Attention over int8 pages: scores (sum q_k * query) * k_scale / sqrt(hd),
  values q_v * v_scale, within |gpu - oracle| <= 1e-5 + 1e-4 |oracle| (the
  fp16/fp32 attention bar: the int8 values widen to fp16 exactly and the
  scales are applied in fp32).
- The engine with int8 pages against the oracle model with the same cache:
  greedy streams token for token (continuous batching with chunked prefill
  included), and logits within 2e-3 of the logit range.  The engine's k and v
  agree with the oracle's to a few fp32 ulps, not bit for bit (another
  summation order in the projections), so an element within an ulp of a .5
  rounding boundary can quantize one int8 step (1/127 of its head's absmax)
  apart; one such step moves the logits by ~3e-4 of their range, above the
  fp32 cache's 1e-3-relative bar for logits near zero.

Device page block per (page, KV head), page_size ps: K = int8 [ps][hd] then
f32 scales [ps]; V = int8 [hd][ps] (dimension-major) then f32 scales [ps].
"""
import numpy as np
import pytest

from oracle import pyoracle as po
from tests.test_gpu_engine import SMALL, engine_config, oracle_model

pytestmark = pytest.mark.gpu


@pytest.fixture(params=[1, 2], ids=["chunk", "split"])
def form(request, hip):
    """Both work decompositions (1: chunk grid, 2: balanced split); the
    automatic choice is restored afterwards."""
    hip._lib.call("qraf_hip_set_attention_tuning", request.param)
    yield request.param
    hip._lib.call("qraf_hip_set_attention_tuning", 0)


def blocks(K8, Ks, V8, Vs):
    """Logical int8 [pages][Hkv][ps][hd] + f32 [pages][Hkv][ps] -> device pools (uint8)."""
    P, Hkv, ps, hd = K8.shape
    kb = np.concatenate([K8.reshape(P, Hkv, ps * hd).view(np.uint8), Ks.astype(np.float32).view(np.uint8)], axis=2)
    vt = np.ascontiguousarray(V8.transpose(0, 1, 3, 2)).reshape(P, Hkv, hd * ps)
    vb = np.concatenate([vt.view(np.uint8), Vs.astype(np.float32).view(np.uint8)], axis=2)
    return np.ascontiguousarray(kb), np.ascontiguousarray(vb)


def quantize(x):
    """absmax int8 per last-axis vector (test data; the store's own rounding is pinned elsewhere)."""
    x = x.astype(np.float32)
    scale = (np.abs(x).max(axis=-1) / np.float32(127)).astype(np.float32)
    q = np.clip(np.rint(x / np.where(scale > 0, scale, 1)[..., None]), -127, 127).astype(np.int8)
    return q, scale


def build_i8_cache(rng, ctxs, Hkv, hd, ps, k_scale=2.5 / 127, v_scale=2.5 / 127, extra_pages=5, poison=True):
    n = len(ctxs)
    max_pages = (max(ctxs) + ps - 1) // ps
    need = sum((c + ps - 1) // ps for c in ctxs)
    P = need + extra_pages
    perm = rng.permutation(P)
    table = np.zeros((n, max_pages), np.int32)
    k = 0
    for s, c in enumerate(ctxs):
        for j in range((c + ps - 1) // ps):
            table[s, j] = perm[k]
            k += 1
    # N(0,1) heads quantized per (position, head) as the store does, so the
    # bytes and scales have a real cache's distribution; then rescaled
    K8, Ks = quantize(rng.standard_normal((P, Hkv, ps, hd)))
    V8, Vs = quantize(rng.standard_normal((P, Hkv, ps, hd)))
    Ks = (Ks * np.float32(k_scale * 127 / 2.5)).astype(np.float32)
    Vs = (Vs * np.float32(v_scale * 127 / 2.5)).astype(np.float32)
    if poison:  # past each context in its last page: any byte, non-finite scales
        for s, c in enumerate(ctxs):
            if c % ps:
                last = table[s, (c - 1) // ps]
                K8[last, :, c % ps:, :] = -128
                Ks[last, :, c % ps:] = np.nan
                Vs[last, :, c % ps:] = np.inf
    return table, K8, Ks, V8, Vs, max_pages


def oracle_i8(q, table, K8, Ks, V8, Vs, ctxs, H, Hkv, hd, ps):
    out = []
    for s, c in enumerate(ctxs):
        t = np.arange(c)
        pg, off = table[s, t // ps], t % ps
        out.append(po.attention_decode_i8(q[s], K8[pg, :, off, :], Ks[pg, :, off], V8[pg, :, off, :], Vs[pg, :, off],
                                          H, Hkv, hd))
    return np.stack(out)


def run_i8(hip, q, table, K8, Ks, V8, Vs, ctxs, H, Hkv, hd, ps, repeats=1):
    from qraf_amd.backend import DeviceBuffer
    call = hip._lib.call
    n = len(ctxs)
    max_ctx = max(ctxs)
    kb, vb = blocks(K8, Ks, V8, Vs)
    ws_bytes = hip.lib.qraf_hip_attention_workspace_bytes(n, H, Hkv, hd, max_ctx)
    ws = DeviceBuffer(ws_bytes)
    dq, dK, dV = DeviceBuffer.from_array(q), DeviceBuffer.from_array(kb), DeviceBuffer.from_array(vb)
    dt, dc = DeviceBuffer.from_array(table), DeviceBuffer.from_array(np.array(ctxs, np.int32))
    out = DeviceBuffer(n * H * hd * 4)
    res = []
    for _ in range(repeats):
        call("qraf_hip_paged_attention_dev", dq.ptr, dK.ptr, dV.ptr, po.I8, dt.ptr, table.shape[1], dc.ptr, n, H, Hkv,
             hd, ps, np.float32(1.0 / np.sqrt(np.float32(hd))), max_ctx, out.ptr, ws.ptr, ws_bytes, None)
        call("qraf_hip_stream_synchronize", None)
        res.append(out.download(np.float32, n * H * hd).reshape(n, H * hd))
    return res


def check(got, want):
    err = np.abs(got.astype(np.float64) - want)
    tol = 1e-5 + 1e-4 * np.abs(want)
    assert np.all(err <= tol), f"max err {err.max():.3e}, worst ratio {(err / tol).max():.2f}"


def test_attention_i8_ragged_batch(hip, form):
    # 128 sequences, context lengths U[128, 4096], 16 q / 2 kv heads, head_dim 128
    rng = np.random.default_rng(2024)
    ctxs = rng.integers(128, 4097, 128).tolist()
    H, Hkv, hd, ps = 16, 2, 128, 16
    print(f"int8 attention n=128 sum_ctx={sum(ctxs)}", flush=True)
    table, K8, Ks, V8, Vs, _ = build_i8_cache(rng, ctxs, Hkv, hd, ps)
    q = rng.standard_normal((128, H * hd)).astype(np.float32)
    got = run_i8(hip, q, table, K8, Ks, V8, Vs, ctxs, H, Hkv, hd, ps, repeats=2)
    assert np.array_equal(got[0], got[1])
    check(got[0], oracle_i8(q, table, K8, Ks, V8, Vs, ctxs, H, Hkv, hd, ps))


@pytest.mark.parametrize("H,Hkv,hd", [(9, 3, 64), (16, 16, 64), (4, 1, 128), (32, 4, 128), (12, 2, 64), (16, 1, 128)])
def test_attention_i8_edge_lengths(hip, form, H, Hkv, hd):
    rng = np.random.default_rng(H * 7 + hd)
    ctxs = [1, 2, 15, 16, 17, 255, 256, 257, 511, 512, 513, 1000, 3]
    print(f"int8 attention H={H} Hkv={Hkv} hd={hd}", flush=True)
    table, K8, Ks, V8, Vs, _ = build_i8_cache(rng, ctxs, Hkv, hd, 16)
    q = (rng.standard_normal((len(ctxs), H * hd)) * 2).astype(np.float32)
    got = run_i8(hip, q, table, K8, Ks, V8, Vs, ctxs, H, Hkv, hd, 16)
    check(got[0], oracle_i8(q, table, K8, Ks, V8, Vs, ctxs, H, Hkv, hd, 16))


@pytest.mark.parametrize("ps", [4, 8, 32, 64, 256])
def test_attention_i8_page_sizes(hip, form, ps):
    rng = np.random.default_rng(ps)
    ctxs = [1, 5, 33, 64, 100, 257, 700]
    H, Hkv, hd = 16, 2, 128
    print(f"int8 attention page_size={ps}", flush=True)
    table, K8, Ks, V8, Vs, _ = build_i8_cache(rng, ctxs, Hkv, hd, ps)
    q = rng.standard_normal((len(ctxs), H * hd)).astype(np.float32)
    got = run_i8(hip, q, table, K8, Ks, V8, Vs, ctxs, H, Hkv, hd, ps)
    check(got[0], oracle_i8(q, table, K8, Ks, V8, Vs, ctxs, H, Hkv, hd, ps))


@pytest.mark.parametrize("ks,vs", [(1e-20, 1e7), (2.5 / 127, 1e-25), (2.5 / 127, 3e30)],
                         ids=["tinyK_hugeV", "tinyV", "V3e30"])
def test_attention_i8_scale_range(hip, form, ks, vs):
    """Value scales far outside fp16's range: the per-wave power of two keeps
    the probability x scale operand finite and normal."""
    rng = np.random.default_rng(5)
    ctxs = [7, 300, 64, 1]
    H, Hkv, hd = 8, 2, 64
    table, K8, Ks, V8, Vs, _ = build_i8_cache(rng, ctxs, Hkv, hd, 16, k_scale=ks, v_scale=vs)
    q = rng.standard_normal((len(ctxs), H * hd)).astype(np.float32)
    got = run_i8(hip, q, table, K8, Ks, V8, Vs, ctxs, H, Hkv, hd, 16)
    want = oracle_i8(q, table, K8, Ks, V8, Vs, ctxs, H, Hkv, hd, 16)
    assert np.all(np.isfinite(got))
    check(got[0] / vs, want / vs)  # relative bar at the values' own scale


def test_attention_i8_refuses_unsupported_shapes(hip):
    from qraf_amd._lib import ERR_INVALID, HipError
    rng = np.random.default_rng(1)
    table, K8, Ks, V8, Vs, _ = build_i8_cache(rng, [5], 1, 32, 16)
    q = rng.standard_normal((1, 2 * 32)).astype(np.float32)
    with pytest.raises(HipError) as e:
        run_i8(hip, q, table, K8, Ks, V8, Vs, [5], 2, 1, 32, 16)
    assert e.value.code == ERR_INVALID
    table, K8, Ks, V8, Vs, _ = build_i8_cache(rng, [5], 1, 64, 12)  # page size not a power of two
    q = rng.standard_normal((1, 2 * 64)).astype(np.float32)
    with pytest.raises(HipError) as e:
        run_i8(hip, q, table, K8, Ks, V8, Vs, [5], 2, 1, 64, 12)
    assert e.value.code == ERR_INVALID


def test_attention_i8_both_forms_many_sequences(hip, form):
    rng = np.random.default_rng(77)
    ctxs = rng.integers(1, 900, 200).tolist()
    H, Hkv, hd = 16, 2, 128
    table, K8, Ks, V8, Vs, _ = build_i8_cache(rng, ctxs, Hkv, hd, 16)
    q = rng.standard_normal((len(ctxs), H * hd)).astype(np.float32)
    got = run_i8(hip, q, table, K8, Ks, V8, Vs, ctxs, H, Hkv, hd, 16)
    check(got[0], oracle_i8(q, table, K8, Ks, V8, Vs, ctxs, H, Hkv, hd, 16))


@pytest.mark.parametrize("Hkv,hd,bias,kind", [(2, 128, True, "normal"), (3, 64, False, "normal"), (2, 128, False, "special"),
                                              (5, 64, True, "normal")])
def test_rope_append_i8_equals_reference_store(hip, Hkv, hd, bias, kind):
    """Bytes and scales equal QuantizedKVCache::store of the rotated k and of
    v (the oracle's kv_quant_heads, pinned against the header); every byte of
    the pools outside the written rows and scales stays as it was."""
    from qraf_amd.backend import DeviceBuffer
    call = hip._lib.call
    L = po.lib()
    rng = np.random.default_rng(Hkv * hd)
    H, ps, theta = 4 * Hkv, 16, 1e6
    pos = np.array([0, 1, 17, 1000, 4095, 33], np.int32)
    n = len(pos)
    max_pages = 4096 // ps
    P = n * max_pages
    table = rng.permutation(P).reshape(n, max_pages).astype(np.int32)
    row = (H + 2 * Hkv) * hd
    qkv = (rng.standard_normal((n, row)) * 3).astype(np.float32)
    if kind == "special":
        qkv[0, H * hd:(H + 1) * hd] = 0.0  # a zero K head: scale 0, bytes 0
        qkv[1, (H + Hkv) * hd:(H + Hkv + 1) * hd] = 0.0  # a zero V head
        v = (np.arange(hd) % 255 - 127).astype(np.float32) * np.float32(0.25)
        v[0] = np.float32(127 * 0.5)  # amax 63.5: scale 0.5, x * inv = k / 2 lands on halves
        qkv[2, (H + Hkv) * hd:(H + Hkv + 1) * hd] = v
        qkv[3, (H + Hkv) * hd + 5] = np.float32(1e30)  # one huge element
    b = (rng.standard_normal(row) * 0.02).astype(np.float32) if bias else None
    blk = ps * (hd + 4)
    init = rng.integers(0, 256, P * Hkv * blk).astype(np.uint8)  # prior contents must survive
    dK, dV = DeviceBuffer.from_array(init), DeviceBuffer.from_array(init[::-1].copy())
    dq = DeviceBuffer(n * H * hd * 4)
    rope = np.zeros(4096 * hd, np.float32)
    call("qraf_hip_rope_table_host", 4096, hd, np.float32(theta), rope.ctypes.data_as(po._fp))
    d_qkv, d_pos, d_t, d_r = (DeviceBuffer.from_array(a) for a in (qkv, pos, table, rope))
    d_b = DeviceBuffer.from_array(b) if bias else None
    print(f"int8 rope_append Hkv={Hkv} hd={hd} bias={bias} {kind}", flush=True)
    call("qraf_hip_rope_append_dev", d_qkv.ptr, d_b.ptr if bias else None, n, H, Hkv, hd, d_pos.ptr, d_r.ptr, dq.ptr,
         dK.ptr, dV.ptr, po.I8, d_t.ptr, max_pages, ps, None)
    call("qraf_hip_stream_synchronize", None)
    qo = dq.download(np.float32, n * H * hd).reshape(n, H * hd)
    kb, vb = dK.download(np.uint8, init.size), dV.download(np.uint8, init.size)
    wk, wv = init.copy().reshape(P, Hkv, blk), init[::-1].copy().reshape(P, Hkv, blk)
    fp = po._fp
    for s in range(n):
        r = qkv[s] + b if bias else qkv[s].copy()
        q, k, v = r[:H * hd].copy(), r[H * hd:(H + Hkv) * hd].copy(), r[(H + Hkv) * hd:].copy()
        for h in range(H):
            seg = np.ascontiguousarray(q[h * hd:(h + 1) * hd])
            L.or_rope(seg.ctypes.data_as(fp), hd, int(pos[s]), theta)
            q[h * hd:(h + 1) * hd] = seg
        for h in range(Hkv):
            seg = np.ascontiguousarray(k[h * hd:(h + 1) * hd])
            L.or_rope(seg.ctypes.data_as(fp), hd, int(pos[s]), theta)
            k[h * hd:(h + 1) * hd] = seg
        assert np.array_equal(qo[s].view(np.uint32), q.view(np.uint32))
        k8, ksc = po.kv_quant_heads(k, Hkv, hd)
        v8, vsc = po.kv_quant_heads(v, Hkv, hd)
        page, off = table[s, pos[s] // ps], pos[s] % ps
        for h in range(Hkv):
            wk[page, h, off * hd:(off + 1) * hd] = k8[h].view(np.uint8)
            wk[page, h, ps * hd + 4 * off:ps * hd + 4 * off + 4] = ksc[h:h + 1].view(np.uint8)
            wv[page, h, np.arange(hd) * ps + off] = v8[h].view(np.uint8)
            wv[page, h, ps * hd + 4 * off:ps * hd + 4 * off + 4] = vsc[h:h + 1].view(np.uint8)
    assert np.array_equal(kb, wk.reshape(-1)), "K pool differs from QuantizedKVCache::store"
    assert np.array_equal(vb, wv.reshape(-1)), "V pool differs from QuantizedKVCache::store"


def upload_i8(m, kw, max_batch=1, max_seq=None):
    from qraf_amd.engine import Engine
    e = Engine(engine_config(dict(kw, max_seq=max_seq or kw["max_seq"])), kv_dtype=po.I8, max_batch=max_batch)
    for name, dt, shape, data in m.tensors():
        e.set_tensor(name, dt, shape, data)
    e.finalize()
    return e


@pytest.mark.parametrize("name", ["q4_gqa8_hd128", "q8_hd64_gqa3"])
def test_engine_int8_logits_vs_oracle(hip, name):
    from qraf_amd.engine import Transformer
    kw, seed = SMALL[name]
    m = oracle_model(kw, seed)
    m.set_kv_int8()
    tf = Transformer(upload_i8(m, kw))
    prompt = [po.lib().or_gen_token(seed, i, kw["vocab"]) for i in range(40)]
    print(f"int8 engine forward {name}", flush=True)
    for pos, t in enumerate(prompt):
        got, want = tf.forward(t, pos), m.forward(t, pos)
        err = np.abs(got.astype(np.float64) - want).max() / np.abs(want).max()
        assert err <= 2e-3, f"{name} int8 pos {pos}: max err {err:.2e} of the logit range"
    tf.engine.close()
    m.close()


def test_engine_int8_greedy_and_continuous_batching(hip):
    from qraf_amd.engine import BatchScheduler, InferenceEngine, Transformer
    kw, seed = SMALL["q4_gqa8_hd128"]
    m = oracle_model(kw, seed)
    m.set_kv_int8()
    L = po.lib()
    prompt = [L.or_gen_token(seed + 1, i, kw["vocab"]) for i in range(16)]
    want = m.generate(prompt, 32, 1.0, eos=-1)
    tf = Transformer(upload_i8(m, kw))
    assert InferenceEngine(tf, eos_token=None).generate_tokens(prompt, 32, repetition_penalty=1.0) == want
    tf.engine.close()
    e = upload_i8(m, kw, max_batch=64)
    pool = e.free_pages()
    prompts = [[L.or_gen_token(300 + r, i, kw["vocab"]) for i in range(2 + 9 * r)] for r in range(7)]
    sched = BatchScheduler(e, max_batch=4, max_rows=64, prefill_chunk=16)
    ids = [sched.submit(p, 6 + 2 * r) for r, p in enumerate(prompts)]
    done = {r.id: r for r in sched.run()}
    for r, (i, p) in enumerate(zip(ids, prompts)):
        assert done[i].generated == m.generate(p, 6 + 2 * r, 1.0, eos=-1), f"request {r}"
    assert e.free_pages() == pool
    e.close()
    m.close()
