"""Device sampler against the compiled reference's Sampler on identical
logits: the repetition penalty bit for bit (logits penalised in place), the
greedy argmax, and temperature / top-k / top-p sampling token for token
(the uniforms are the reference's own draw stream, reproduced on the host).
Then InferenceEngine with sampling, end to end, against the reference's
InferenceEngine on the same .qraf file.

Sampling parity is exact on the same logits unless a uniform lands within a
rounding of a cumulative-probability boundary (device expf against glibc's
expf); with continuous random logits that has probability of order 1e-6 per
draw.  Ties between equal probabilities are not ordered by the reference
(std::sort), so the inputs here have none (tie_free).
"""
import ctypes as C

import numpy as np
import pytest

from oracle import pyoracle as po

pytestmark = [pytest.mark.gpu,
              pytest.mark.usefixtures("reference")]

u32p = C.POINTER(C.c_uint32)
fp = C.POINTER(C.c_float)


def device_sample(hip, logits_rows, params, recent=None, uniforms=None):
    from qraf_amd._lib import SamplingParams
    from qraf_amd.backend import DeviceBuffer
    rows, V = logits_rows.shape
    dl = DeviceBuffer.from_array(np.ascontiguousarray(logits_rows, np.float32))
    out = DeviceBuffer(rows * 4)
    rec = cnt = uni = None
    stride = 0
    if recent is not None:
        stride = max(1, max(len(r) for r in recent))
        a = np.zeros((rows, stride), np.uint32)
        c = np.zeros(rows, np.int32)
        for i, r in enumerate(recent):
            a[i, :len(r)] = r
            c[i] = len(r)
        rec, cnt = DeviceBuffer.from_array(a), DeviceBuffer.from_array(c)
    if uniforms is not None:
        uni = DeviceBuffer.from_array(np.ascontiguousarray(uniforms, np.float32))
    sp = SamplingParams(*params)
    hip._lib.call("qraf_hip_sample_dev", dl.ptr, rows, V, C.byref(sp), rec.ptr if rec else None,
                  cnt.ptr if cnt else None, stride, uni.ptr if uni else None, out.ptr, None)
    hip._lib.call("qraf_hip_stream_synchronize", None)
    return out.download(np.uint32, rows), dl.download(np.float32, rows * V).reshape(rows, V)


def tie_free(logits, T):
    """The logits with every p = logit / T (float32, as both samplers
    compute it) distinct: duplicates are moved up one ulp at a time.  The
    reference's std::sort leaves equal p in an unspecified order, which a
    large candidate list would otherwise reach."""
    x = np.array(logits, np.float32)
    for _ in range(64):
        q = x / np.float32(T)
        order = np.argsort(q, kind="stable")
        dup = order[1:][q[order[1:]] == q[order[:-1]]]
        if dup.size == 0:
            return x
        x[dup] = np.nextafter(x[dup], np.float32(np.inf))
    raise AssertionError("could not separate equal probabilities")


def ref_sample(logits, T, k, p, seed, n):
    out = np.zeros(n, np.uint32)
    l = np.ascontiguousarray(logits, np.float32)
    po.ref().ref_sample(l.ctypes.data_as(fp), l.size, T, k, p, seed, n, out.ctypes.data_as(u32p))
    return out


@pytest.mark.parametrize("V", [1000, 151936])
@pytest.mark.parametrize("cfg", [(0.8, 40, 0.9), (1.0, 1, 1.0), (0.7, 1024, 0.95), (1.3, 50, 0.0), (0.9, 200, 0.5),
                                 (2.0, 0, 0.8)], ids=lambda c: "T%g_k%d_p%g" % c)
def test_sampling_equals_reference_sampler(hip, V, cfg):
    from qraf_amd.engine import Sampler, SamplingConfig
    T, k, p = cfg
    rng = np.random.default_rng(V + int(T * 10) + k)
    n = 96
    logits = tie_free((rng.standard_normal(V) * 3.0).astype(np.float32), T)
    seed = 1000 + k
    print(f"sampler V={V} T={T} top_k={k} top_p={p}", flush=True)
    want = ref_sample(logits, T, k, p, seed, n)
    uni = Sampler(SamplingConfig(seed=seed)).uniforms(n)
    got, _ = device_sample(hip, np.tile(logits, (n, 1)), (T, k, p, 1.0), uniforms=uni)
    assert np.array_equal(got, want), f"{np.count_nonzero(got != want)} of {n} draws differ"
    assert len(set(want.tolist())) > (1 if k != 1 else 0)  # the draws do explore the candidates


@pytest.mark.parametrize("V,hist", [(1000, 40), (151936, 40), (1000, 3000), (151936, 5000)])
def test_penalty_and_greedy_equal_reference(hip, V, hist):
    """Histories up to 4096 tokens take the LDS-sorted kernel, longer ones
    the sequential one."""
    rng = np.random.default_rng(V + hist)
    rows = 6
    L = (rng.standard_normal((rows, V)) * 2.0).astype(np.float32)
    recent = [rng.integers(0, V, hist).tolist() + [5, 5, 5] for _ in range(rows)]  # repeats: applied per occurrence
    recent[1] = recent[1] + [V + 3]  # out of range: skipped
    got, pen = device_sample(hip, L, (0.0, 40, 0.9, 1.1), recent=recent)
    R = po.ref()
    for i in range(rows):
        w = L[i].copy()
        r = np.array(recent[i], np.uint32)
        R.ref_penalty(w.ctypes.data_as(fp), V, r.ctypes.data_as(u32p), r.size, 1.1)
        assert np.array_equal(pen[i], w), f"row {i}: penalised logits differ"
        assert got[i] == R.ref_argmax(w.ctypes.data_as(fp), V), f"row {i}"


def test_first_index_of_equal_maxima(hip):
    L = np.zeros((2, 4096), np.float32)
    L[0, [7, 100, 4000]] = 3.0
    L[1, [4095, 4094]] = 1.0
    got, _ = device_sample(hip, L, (0.0, 0, 1.0, 1.0))
    assert got.tolist() == [7, 4094]


@pytest.mark.parametrize("V,k,T,p", [(8192, 5000, 0.8, 0.9), (151936, 4097, 0.9, 0.95), (151936, 60000, 1.5, 0.0),
                                     (151936, 151935, 2.0, 0.8), (20000, 19999, 1.0, 0.999)])
def test_top_k_above_lds_limit_equals_reference_sampler(hip, V, k, T, p):
    """4096 < top_k < vocab: the top_k candidates are gathered and sorted in
    global sort storage (radix sort), then the reference's loops run over
    all of them."""
    from qraf_amd.engine import Sampler, SamplingConfig
    n = 24
    rng = np.random.default_rng(V + k)
    logits = tie_free((rng.standard_normal(V) * 3.0).astype(np.float32), T)
    print(f"sampler V={V} top_k={k} T={T} top_p={p}", flush=True)
    want = ref_sample(logits, T, k, p, 5 + k, n)
    uni = Sampler(SamplingConfig(seed=5 + k)).uniforms(n)
    got, _ = device_sample(hip, np.tile(logits, (n, 1)), (T, k, p, 1.0), uniforms=uni)
    assert np.array_equal(got, want), f"{np.count_nonzero(got != want)} of {n} draws differ"
    assert len(set(want.tolist())) > 3


def zipf_logits(rng, V, exponent, scale=1.0, head=20.0):
    """log of a Zipf-like law over a random permutation of the vocabulary:
    p ~ (1 + rank / head)^-exponent (a flat head of about `head` tokens)."""
    rank = rng.permutation(V).astype(np.float64)
    return (-exponent * np.log1p(rank / head) * scale + rng.standard_normal(V) * 1e-3).astype(np.float32)


@pytest.mark.parametrize("kind,T,p", [("zipf6", 1.0, 0.9), ("zipf6", 0.8, 0.0), ("zipf8", 1.3, 0.95),
                                      ("masked", 0.8, 0.9), ("masked", 1.0, 0.0)])
def test_whole_vocabulary_equals_reference_sampler(hip, kind, T, p):
    """top_k 0 over 151,936 tokens: the device gathers the tokens whose terms
    survive the reference's sequential sums (file comment of sampler.hip) and
    must pick the reference's token for every draw; "masked" rows hold 2,000
    N(0,3) logits and -inf elsewhere (the reference sorts those last)."""
    from qraf_amd.engine import Sampler, SamplingConfig
    V, n = 151936, 96
    rng = np.random.default_rng({"zipf6": 100, "zipf8": 200, "masked": 300}[kind] + int(T * 10))
    if kind == "masked":
        logits = np.full(V, -np.inf, np.float32)
        logits[rng.choice(V, 2000, replace=False)] = (rng.standard_normal(2000) * 3).astype(np.float32)
    else:
        logits = zipf_logits(rng, V, 6.0 if kind == "zipf6" else 8.0, T)
    seed = 77
    print(f"whole vocabulary {kind} T={T} top_p={p}", flush=True)
    want = ref_sample(logits, T, 0, p, seed, n)
    uni = Sampler(SamplingConfig(seed=seed)).uniforms(n)
    got, _ = device_sample(hip, np.tile(logits, (n, 1)), (T, 0, p, 1.0), uniforms=uni)
    assert np.array_equal(got, want), f"{np.count_nonzero(got != want)} of {n} draws differ"
    assert len(set(want.tolist())) > 3


@pytest.mark.parametrize("V,p", [(20000, 0.9), (20000, 0.0), (151936, 0.5)])
def test_flat_whole_vocabulary_equals_reference_sampler(hip, V, p):
    """Rows whose weight spreads over more than 4096 tokens (nearly flat
    logits): every pair of the row is sorted in global sort storage; the
    uniforms include values near 1, where the cumulative sum runs to the
    row's tail."""
    from qraf_amd.engine import Sampler, SamplingConfig
    n = 16
    rng = np.random.default_rng(V + int(p * 10))
    logits = tie_free((rng.standard_normal(V) * 0.1).astype(np.float32), 1.0)
    print(f"sampler flat V={V} top_p={p}", flush=True)
    want = ref_sample(logits, 1.0, 0, p, 9, n)
    uni = Sampler(SamplingConfig(seed=9)).uniforms(n)
    got, _ = device_sample(hip, np.tile(logits, (n, 1)), (1.0, 0, p, 1.0), uniforms=uni)
    assert np.array_equal(got, want), f"{np.count_nonzero(got != want)} of {n} draws differ"
    assert len(set(want.tolist())) > 3


@pytest.mark.parametrize("k", [1500, 3000, 4096])
def test_top_k_up_to_4096_equals_reference_sampler(hip, k):
    from qraf_amd.engine import Sampler, SamplingConfig
    V, n = 151936, 64
    rng = np.random.default_rng(k)
    logits = (rng.standard_normal(V) * 3.0).astype(np.float32)
    want = ref_sample(logits, 0.9, k, 0.95, 11, n)
    uni = Sampler(SamplingConfig(seed=11)).uniforms(n)
    got, _ = device_sample(hip, np.tile(logits, (n, 1)), (0.9, k, 0.95, 1.0), uniforms=uni)
    assert np.array_equal(got, want), f"{np.count_nonzero(got != want)} of {n} draws differ"


@pytest.mark.parametrize("cfg", [(0.8, 40, 0.9, 1.1, 7), (1.0, 10, 1.0, 1.0, 3), (0.0, 40, 0.9, 1.3, 1)],
                         ids=["default", "topk10", "greedy_penalty"])
def test_generate_with_sampling_equals_reference(hip, tmp_path, cfg):
    from qraf_amd.engine import InferenceEngine, SamplingConfig, Transformer
    from tests.test_gpu_engine import SMALL
    T, k, p, pen, seed = cfg
    kw, mseed = SMALL["q8_llama"]
    m = po.Model(po.make_config(**kw), mseed)
    path = str(tmp_path / "m.qraf")
    m.write_qraf(path)
    prompt = [po.lib().or_gen_token(mseed, i, kw["vocab"]) for i in range(8)]
    ref = po.RefEngine(path)
    want = ref.generate_sampled(prompt, 24, T, k, p, pen, seed)
    ref.close()
    tf = Transformer.from_file(path)
    got = InferenceEngine(tf).generate_tokens(prompt, 24, sampling=SamplingConfig(T, k, p, pen, seed))
    tf.engine.close()
    m.close()
    assert got == want
