"""GPU parity of the Q8_0/Q4_0 matvec and the op-level dispatch mirror
against the oracle (oracle/oracle.c) on the same seeded inputs.

Tolerance for every matvec output row i (floating point; the GPU sums in a
different order than the reference's sequential loop):
    |y_gpu[i] - y_oracle[i]| <= 2 * (K + 2) * 2^-24 * sum_j |w_ij * x_j|
i.e. twice the classical worst-case bound of a K-term fp32 dot product, which
both implementations satisfy with respect to the exact value.  A dropped
block, a wrong scale or a swapped nibble overshoots it by orders of magnitude.
"""
import ctypes as C

import numpy as np
import pytest

from oracle import pyoracle as po

pytestmark = pytest.mark.gpu

FP = C.POINTER(C.c_float)


def quantize_rows(dt, w, n, k, bs=32):
    if k % bs == 0:
        return po.quantize(dt, w, bs)
    return np.concatenate([po.quantize(dt, w[i * k:(i + 1) * k], bs) for i in range(n)])


def dequant_rows(dt, wq, n, k, bs=32):
    rb = len(wq) // n
    return np.stack([po.dequantize(dt, wq[i * rb:(i + 1) * rb], k, bs) for i in range(n)])


def tol_rows(dt, wq, n, k, x, bs=32):
    W = dequant_rows(dt, wq, n, k, bs).astype(np.float64)
    if dt == po.Q4_0 and k % 2:  # reference ignores the odd tail element
        W[:, -1] = 0
    return 2.0 * (k + 2) * 2.0 ** -24 * (np.abs(W) @ np.abs(x.astype(np.float64))) + 1e-30


def check(y, y_ref, tol):
    err = np.abs(y.astype(np.float64) - y_ref.astype(np.float64))
    bad = np.nonzero(err > tol)[0]
    assert bad.size == 0, f"{bad.size} rows out of tolerance, first {bad[:5]}: err {err[bad[:5]]} tol {tol[bad[:5]]}"


SHAPES = [
    # (N, K, bs): BASELINE matvec shapes, SmolLM2-135M and Qwen2.5-3B projection shapes, ragged cases
    (4096, 4096, 32), (11008, 4096, 32),
    (576, 576, 32), (192, 576, 32), (1536, 576, 32), (576, 1536, 32), (49152, 576, 32),
    (2048, 2048, 32), (256, 2048, 32), (11008, 2048, 32), (2048, 11008, 32),
    (1, 64, 32), (7, 100, 32), (13, 31, 32), (33, 96, 32), (5, 45, 8), (9, 19, 4), (3, 4000, 16),
]


@pytest.mark.parametrize("dt", [po.Q8_0, po.Q4_0])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_matvec_q_vs_oracle(hip, dt, shape):
    n, k, bs = shape
    print(f"matvec dt={dt} N={n} K={k} bs={bs}", flush=True)
    rng = np.random.default_rng(n * 131 + k * 7 + dt)
    w = (rng.standard_normal(n * k) * 0.02).astype(np.float32)
    wq = quantize_rows(dt, w, n, k, bs)
    x = rng.standard_normal(k).astype(np.float32)
    y_ref = po.matvec_q(wq, dt, n, k, x, bs)
    y = np.zeros(n, np.float32)
    hip.backend.dispatch_matvec_q(wq, wq.nbytes, dt, bs, n, k, x, y)
    check(y, y_ref, tol_rows(dt, wq, n, k, x, bs))


@pytest.mark.parametrize("kernel,rows,wgs", [(1, 1, 0), (1, 2, 0), (1, 4, 0), (1, 8, 0), (2, 1, 4), (2, 2, 2),
                                             (2, 4, 1), (2, 2, 8), (3, 1, 0), (3, 2, 1), (3, 1, 3), (4, 1, 2),
                                             (4, 2, 4), (4, 2, 16)])
@pytest.mark.parametrize("dt", [po.Q8_0, po.Q4_0])
@pytest.mark.parametrize("k", [2048, 11008])
@pytest.mark.parametrize("n", [1000, 999])
def test_matvec_kernel_variants(hip, kernel, rows, wgs, dt, k, n):
    rng = np.random.default_rng(rows + k)
    wq = po.quantize(dt, (rng.standard_normal(n * k) * 0.02).astype(np.float32))
    x = rng.standard_normal(k).astype(np.float32)
    y_ref = po.matvec_q(wq, dt, n, k, x)
    y = np.zeros(n, np.float32)
    hip.lib.qraf_hip_set_matvec_tuning(kernel, rows, wgs)
    try:
        hip.backend.dispatch_matvec_q(wq, 0, dt, 32, n, k, x, y)
    finally:
        hip.lib.qraf_hip_set_matvec_tuning(0, 0, 0)
    check(y, y_ref, tol_rows(dt, wq, n, k, x))


def test_matvec_golden_fixtures(hip):
    from tests.conftest import golden
    g = golden("matvec.npz")
    for key in [f[2:] for f in g.files if f.startswith("w_")]:
        dt, n, k, bs = (int(v) for v in key.split("_"))
        y = np.zeros(n, np.float32)
        hip.backend.dispatch_matvec_q(g["w_" + key], 0, dt, bs, n, k, g["x_" + key], y)
        check(y, g["y_" + key], tol_rows(dt, g["w_" + key], n, k, g["x_" + key], bs))
    y = np.zeros(40, np.float32)
    hip.backend.dispatch_matvec_opt(np.ascontiguousarray(g["f32_W"]), g["f32_x"], y, 40, 96)
    tol = 2 * 98 * 2.0 ** -24 * (np.abs(g["f32_W"]).astype(np.float64) @ np.abs(g["f32_x"]))
    check(y, g["f32_y"], tol)


def test_matvec_unaligned_and_registered(hip):
    n, k = 300, 4096
    rng = np.random.default_rng(11)
    for dt in (po.Q8_0, po.Q4_0):
        wq = po.quantize(dt, (rng.standard_normal(n * k) * 0.02).astype(np.float32))
        x = rng.standard_normal(k).astype(np.float32)
        y_ref = po.matvec_q(wq, dt, n, k, x)
        tol = tol_rows(dt, wq, n, k, x)
        # weights at an odd address take the general kernel
        buf = np.zeros(wq.nbytes + 3, np.uint8)
        buf[1:1 + wq.nbytes] = wq
        y = np.zeros(n, np.float32)
        hip.backend.dispatch_matvec_q(buf[1:], 0, dt, 32, n, k, x, y)
        check(y, y_ref, tol)
        # registered (HBM-resident) weights give the same bits as uploaded ones
        y2 = np.zeros(n, np.float32)
        hip.backend.dispatch_matvec_q(wq, 0, dt, 32, n, k, x, y2)
        hip.backend.register_weights(wq)
        y3 = np.zeros(n, np.float32)
        hip.backend.dispatch_matvec_q(wq, 0, dt, 32, n, k, x, y3)
        hip.backend.unregister_weights(wq)
        assert np.array_equal(y2.view(np.uint32), y3.view(np.uint32))


def test_matvec_device_level_matches_op_level(hip):
    from qraf_amd.backend import DeviceBuffer
    n, k = 2048, 11008
    rng = np.random.default_rng(12)
    for dt in (po.Q8_0, po.Q4_0):
        wq = po.quantize(dt, (rng.standard_normal(n * k) * 0.02).astype(np.float32))
        x = rng.standard_normal(k).astype(np.float32)
        y = np.zeros(n, np.float32)
        hip.backend.dispatch_matvec_q(wq, 0, dt, 32, n, k, x, y)
        dw, dx, dy = DeviceBuffer.from_array(wq), DeviceBuffer.from_array(x), DeviceBuffer(n * 4)
        hip._lib.call("qraf_hip_matvec_q_dev", dw.ptr, dt, 32, n, k, dx.ptr, dy.ptr, None)
        hip._lib.call("qraf_hip_stream_synchronize", None)
        assert np.array_equal(dy.download(np.float32, n).view(np.uint32), y.view(np.uint32))


def test_matvec_from_several_host_threads(hip):
    """Four host threads at once, each alternating the op-level matvec (host
    pointers, serialised inside the library) with the device-level one on the
    library's default stream (NULL stream) into buffers of its own: every
    result equals the single-threaded one bit for bit."""
    import threading
    from qraf_amd.backend import DeviceBuffer
    n, k = 1024, 2048
    rng = np.random.default_rng(21)
    wq = po.quantize(po.Q8_0, (rng.standard_normal(n * k) * 0.02).astype(np.float32))
    xs = [rng.standard_normal(k).astype(np.float32) for _ in range(4)]
    want = []
    for x in xs:
        y = np.zeros(n, np.float32)
        hip.backend.dispatch_matvec_q(wq, 0, po.Q8_0, 32, n, k, x, y)
        want.append(y)
    dw = DeviceBuffer.from_array(wq)
    bad = []

    def work(i):
        dx, dy = DeviceBuffer.from_array(xs[i]), DeviceBuffer(n * 4)
        for it in range(20):
            y = np.zeros(n, np.float32)
            hip.backend.dispatch_matvec_q(wq, 0, po.Q8_0, 32, n, k, xs[i], y)
            hip._lib.call("qraf_hip_matvec_q_dev", dw.ptr, po.Q8_0, 32, n, k, dx.ptr, dy.ptr, None)
            hip._lib.call("qraf_hip_stream_synchronize", None)
            got = dy.download(np.float32, n)
            if not (np.array_equal(y.view(np.uint32), want[i].view(np.uint32)) and
                    np.array_equal(got.view(np.uint32), want[i].view(np.uint32))):
                bad.append((i, it))

    threads = [threading.Thread(target=work, args=(i,)) for i in range(4)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=120)
    assert not any(th.is_alive() for th in threads)
    assert not bad, bad


def test_matvec_error_codes(hip):
    x = np.ones(64, np.float32)
    y = np.zeros(4, np.float32)
    with pytest.raises(hip.HipError) as e:
        hip.backend.dispatch_matvec_q(np.zeros(300, np.uint8), 0, 7, 32, 4, 64, x, y)
    assert e.value.code == -2


def test_elementwise_ops_vs_oracle(hip):
    rng = np.random.default_rng(13)
    L = po.lib()
    for n in (576, 2048, 3000):
        x = (rng.standard_normal(n) * 3).astype(np.float32)
        w = rng.uniform(0.5, 1.5, n).astype(np.float32)
        a, b = x.copy(), x.copy()
        L.or_rms_norm(a.ctypes.data_as(FP), w.ctypes.data_as(FP), n, 1e-5)
        hip.backend.dispatch_rms_norm(b, w, n, 1e-5)
        np.testing.assert_allclose(b, a, rtol=2e-6, atol=1e-7)
        a, b = x.copy(), x.copy()
        L.or_softmax(a.ctypes.data_as(FP), n)
        hip.backend.dispatch_softmax(b, n)
        np.testing.assert_allclose(b, a, rtol=1e-5, atol=1e-9)
        a, b = x.copy(), x.copy()
        L.or_silu(a.ctypes.data_as(FP), n)
        hip.backend.dispatch_silu(b, n)
        np.testing.assert_allclose(b, a, rtol=4e-7, atol=1e-30)
        y = rng.standard_normal(n).astype(np.float32)
        b = x.copy()
        hip.backend.dispatch_add(b, y, n)
        assert np.array_equal(b, x + y)
        b = x.copy()
        hip.backend.dispatch_mul(b, y, n)
        assert np.array_equal(b, x * y)
        b = x.copy()
        hip.backend.dispatch_scale(b, 0.37, n)
        assert np.array_equal(b, x * np.float32(0.37))
        d = hip.backend.dispatch_dot_f32(x, y, n)
        assert abs(d - float(np.dot(x.astype(np.float64), y))) <= 2 * n * 2.0 ** -24 * float(np.abs(x * y).sum())


def batch_covered(dt, k, nv):
    """The batch matvec's own coverage rule: K a multiple of 32 (64 for Q4_0),
    the batch rounded up to 2/4/8/16 vectors staged within 144 KB."""
    if k % (32 if dt == po.Q8_0 else 64):
        return False
    nvr = 2 if nv <= 2 else 4 if nv <= 4 else 8 if nv <= 8 else 16
    per = (k // 32) * 36 * 4 if dt == po.Q8_0 else (k // 64) * 76 * 4
    return nvr * per <= 144 * 1024


BATCH_SHAPES = [(576, 576), (1536, 576), (576, 1536), (2048, 2048), (256, 2048), (11008, 2048), (49152, 576),
                (999, 4096), (33, 128), (5, 2048)]


# every (shape, dtype, batch) the kernel covers; the others are refused (tested below)
BATCH_CASES = [(shape, dt, nv) for shape in BATCH_SHAPES for dt in (po.Q8_0, po.Q4_0) for nv in (1, 2, 3, 5, 8, 16)
               if batch_covered(dt, shape[1], nv)]


@pytest.mark.parametrize("shape,dt,nv", BATCH_CASES,
                         ids=lambda v: "x".join(map(str, v)) if isinstance(v, tuple) else str(v))
def test_matvec_batch_vs_oracle(hip, shape, dt, nv):
    """qraf_hip_matvec_q_batch_dev: every row of y = W x[b] against the
    oracle's matvec of that row within the bound above, and each row
    bit-identical to the same vector alone (nv = 1): the vectors' sums do not
    depend on the batch they ride in."""
    from qraf_amd.backend import DeviceBuffer
    n, k = shape
    print(f"batch matvec dt={dt} N={n} K={k} nv={nv}", flush=True)
    rng = np.random.default_rng(n * 17 + k * 3 + nv + dt)
    wq = po.quantize(dt, (rng.standard_normal(n * k) * 0.02).astype(np.float32))
    x = rng.standard_normal((nv, k)).astype(np.float32)
    dw, dx, dy = DeviceBuffer.from_array(wq), DeviceBuffer.from_array(x), DeviceBuffer(nv * n * 4)
    hip._lib.call("qraf_hip_matvec_q_batch_dev", dw.ptr, dt, n, k, dx.ptr, nv, dy.ptr, None)
    hip._lib.call("qraf_hip_stream_synchronize", None)
    y = dy.download(np.float32, nv * n).reshape(nv, n)
    for b in range(nv):
        check(y[b], po.matvec_q(wq, dt, n, k, x[b]), tol_rows(dt, wq, n, k, x[b]))
    d1, dy1 = DeviceBuffer.from_array(np.ascontiguousarray(x[nv - 1])), DeviceBuffer(n * 4)
    hip._lib.call("qraf_hip_matvec_q_batch_dev", dw.ptr, dt, n, k, d1.ptr, 1, dy1.ptr, None)
    hip._lib.call("qraf_hip_stream_synchronize", None)
    assert np.array_equal(dy1.download(np.float32, n).view(np.uint32), y[nv - 1].view(np.uint32))
    for d in (dw, dx, dy, d1, dy1):
        d.free()


def test_matvec_batch_refuses_what_it_does_not_cover(hip):
    from qraf_amd.backend import DeviceBuffer
    d = DeviceBuffer(1 << 20)
    for dt, n, k, nv in ((po.Q8_0, 64, 11008, 4), (po.Q4_0, 64, 96, 2), (po.Q8_0, 64, 100, 2), (po.Q8_0, 64, 64, 17),
                         (po.Q8_0, 64, 64, 0), (7, 64, 64, 2)):
        with pytest.raises(hip.HipError):
            hip._lib.call("qraf_hip_matvec_q_batch_dev", d.ptr, dt, n, k, d.ptr, nv, d.ptr, None)
    d.free()
