"""Host side of the device sampler: the draw stream of the reference's
Sampler (std::mt19937 seeded as sampler.cpp:9-16, read through
std::uniform_real_distribution<float>(0, 1)) against the compiled reference,
and the parameter mapping of SamplingConfig.  No GPU use.
"""
import ctypes as C

import numpy as np
import pytest

from oracle import pyoracle as po

need_ref = pytest.mark.skipif(po.ref() is None, reason="oracle/_ref (the compiled reference) is not built")


@need_ref
@pytest.mark.parametrize("seed", [1, 42, 123456789, 0xFFFFFFFF, 2 ** 40 + 5])
def test_uniform_stream_equals_reference(seed):
    from qraf_amd.engine import Sampler, SamplingConfig
    n = 50000
    want = np.zeros(n, np.float32)
    po.ref().ref_uniforms(seed, n, want.ctypes.data_as(C.POINTER(C.c_float)))
    got = Sampler(SamplingConfig(seed=seed)).uniforms(n)
    assert np.array_equal(got, want)


def test_uniform_top_word_is_clamped_below_one():
    """libstdc++'s generate_canonical<float, 24>: float(x) / 2^32 rounds to 1
    for the top 128 words, which become the largest float below 1."""
    from qraf_amd.engine import Sampler, SamplingConfig
    s = Sampler(SamplingConfig(seed=7))
    for x, want in ((0xFFFFFFFF, np.nextafter(np.float32(1), np.float32(0))),
                    (0xFFFFFF80, np.nextafter(np.float32(1), np.float32(0))),
                    (0xFFFFFF7F, np.float32(0xFFFFFF00) / np.float32(2 ** 32)),
                    (0, np.float32(0)), (1 << 31, np.float32(0.5))):
        s._rng.getrandbits = lambda k, x=x: x
        assert np.float32(s.uniform()) == want, hex(x)


def test_greedy_mapping():
    from qraf_amd.engine import SamplingConfig
    assert SamplingConfig(temperature=0.0).greedy and SamplingConfig(deterministic=True).greedy
    assert not SamplingConfig().greedy
    p = SamplingConfig(deterministic=True, temperature=0.8).params()
    assert p.temperature == 0.0  # sampler.cpp:59-61: deterministic means argmax
    q = SamplingConfig(temperature=0.7, top_k=50, top_p=0.95, repetition_penalty=1.2).params()
    assert (q.top_k, round(q.temperature, 6), round(q.top_p, 6), round(q.repetition_penalty, 6)) == (50, 0.7, 0.95, 1.2)
