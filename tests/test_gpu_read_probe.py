"""The plain-read probe the matvec benchmark reports its ceiling with: it must
read every byte it is given (the wave sums add up to the data's sum; small
integers, so every fp32 sum is exact) and refuse sizes it cannot read whole."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n", [4, 1000, 1 << 20, (1 << 22) + 12])
def test_read_probe_reads_every_byte(hip, n):
    from qraf_amd.backend import DeviceBuffer
    call, lib = hip._lib.call, hip._lib.lib
    data = np.random.default_rng(n).integers(-3, 4, n).astype(np.float32)
    d = DeviceBuffer.from_array(data)
    out = DeviceBuffer(lib.qraf_hip_read_probe_out_bytes())
    call("qraf_hip_read_probe_dev", d.ptr, n * 4, out.ptr, None)
    call("qraf_hip_stream_synchronize", None)
    sums = out.download(np.float32, lib.qraf_hip_read_probe_out_bytes() // 4)
    assert sums.astype(np.float64).sum() == data.astype(np.float64).sum()


def test_read_probe_refusals(hip):
    from qraf_amd.backend import DeviceBuffer
    from qraf_amd._lib import HipError
    call, lib = hip._lib.call, hip._lib.lib
    d = DeviceBuffer(64)
    out = DeviceBuffer(lib.qraf_hip_read_probe_out_bytes())
    for bad in (0, 20):
        with pytest.raises(HipError):
            call("qraf_hip_read_probe_dev", d.ptr, bad, out.ptr, None)


@pytest.mark.parametrize("wgs", [1, 256, 65536])
def test_launch_floor_runs_in_a_graph(hip, wgs):
    """The per-launch floor's empty kernel, as bench.py times it: launched
    eagerly and replayed in a captured graph on a stream of its own, every
    launch completing."""
    from qraf_amd.backend import Graph, Stream
    call = hip._lib.call
    s = Stream()
    call("qraf_hip_launch_floor_dev", wgs, s.h)
    call("qraf_hip_stream_synchronize", s.h)
    with Graph(s) as g:
        for _ in range(8):
            call("qraf_hip_launch_floor_dev", wgs, s.h)
    try:
        for _ in range(3):
            g.launch()
        call("qraf_hip_stream_synchronize", s.h)
    finally:
        g.destroy()
        s.destroy()
