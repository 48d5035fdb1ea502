"""The device quantizer and synthetic-weight generator are bit-exact with
the oracle (and, through the golden fixtures, with the reference's
quantize_q8_0 / quantize_q4_0)."""
import numpy as np
import pytest

from oracle import pyoracle as po
from tests.conftest import golden

pytestmark = pytest.mark.gpu


def _dev_quantize(hip, x, dt):
    from qraf_amd.backend import DeviceBuffer
    src = DeviceBuffer.from_array(x.astype(np.float32))
    nbytes = po.lib().or_q_tensor_bytes(dt, x.size, 32)
    dst = DeviceBuffer(nbytes)
    dst.zero()
    hip._lib.call("qraf_hip_quantize_dev", src.ptr, x.size, dt, dst.ptr, None)
    hip._lib.call("qraf_hip_stream_synchronize", None)
    return dst.download(np.uint8, nbytes)


@pytest.mark.parametrize("dt", [po.Q8_0, po.Q4_0])
def test_device_quantizer_golden(hip, dt):
    g = golden("quant.npz")
    for tag in ("rand", "special"):  # special: zeros, +-1e-8, 3.4e38, denormal, NaN, +-inf, an all-zero block
        k = f"{dt}_32_{tag}"
        assert np.array_equal(_dev_quantize(hip, g["x_" + k], dt), g["q_" + k]), tag


@pytest.mark.parametrize("dt", [po.Q8_0, po.Q4_0])
@pytest.mark.parametrize("count", [32, 1000, 4096 * 3 + 17, 1 << 20])
def test_device_quantizer_vs_oracle(hip, dt, count):
    rng = np.random.default_rng(count)
    x = (rng.standard_normal(count) * rng.choice([1e-3, 0.02, 5.0], count)).astype(np.float32)
    assert np.array_equal(_dev_quantize(hip, x, dt), po.quantize(dt, x))


@pytest.mark.parametrize("dt", [po.F32, po.Q8_0, po.Q4_0])
@pytest.mark.parametrize("count", [64, 576 * 192, 2048 * 256 + 32])
def test_generator_matches_oracle(hip, dt, count):
    from qraf_amd.backend import DeviceBuffer
    name = b"model.layers.3.self_attn.k_proj.weight"
    sid = hip.lib.qraf_hip_name_hash(name)
    assert sid == po.fnv1a(name.decode())
    nbytes = count * 4 if dt == po.F32 else po.lib().or_q_tensor_bytes(dt, count, 32)
    dst = DeviceBuffer(nbytes)
    hip._lib.call("qraf_hip_gen_weights_dev", dst.ptr, dt, count, 77, sid, 0.02, None)
    hip._lib.call("qraf_hip_stream_synchronize", None)
    got = dst.download(np.uint8, nbytes)
    ref = po.gen_normal(77, sid, count, 0.02)
    want = ref.view(np.uint8) if dt == po.F32 else po.quantize(dt, ref)
    assert np.array_equal(got, want)
