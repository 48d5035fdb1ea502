"""GPU parity of the large-batch GEMM on the MFMA-ready ("mx") weight copy
against the oracle's dispatch_matvec_q applied to every batch row, with the
bound of test_gpu_qgemm.py:
    |y_gpu - y_oracle| <= sum_k |w_k| (2^-20 |x_k| + 2^-25) + 2 (K + 2) 2^-24 sum_k |w_k x_k|.

The mx layout is pinned byte for byte against a numpy construction from the
reference bytes; for Q4_0 this also pins the hardware fp8 encoder's format
(OCP e4m3: 1 = 0x38, -8 = 0xD0) and byte order.  The SwiGLU epilogue
(silu(gate) * up of interleaved rows, written as bf16/fp16 planes) is checked
against the same GEMM's plain output put through SiLU-gate on the host.
"""
import numpy as np
import pytest

from oracle import pyoracle as po
from tests.test_gpu_qgemm import check

pytestmark = pytest.mark.gpu

# OCP fp8 e4m3 codes of the integers -8..7 (sign, 4-bit exponent with bias 7, 3-bit mantissa)
E4M3 = {0: 0x00, 1: 0x38, 2: 0x40, 3: 0x44, 4: 0x48, 5: 0x4A, 6: 0x4C, 7: 0x4E}
E4M3.update({-v: c | 0x80 for v, c in list(E4M3.items()) if v})
E4M3[-8] = 0xD0


def mx_reference(wq, dt, N, K):
    nb, nt = K // 32, (N + 15) // 16
    out = np.zeros((nt * 16, nb, 576 // 16), np.uint8)  # per row: 4 scale bytes + 32 values, reordered below
    scale = np.zeros((nt * 16, nb), np.float32)
    vals = np.zeros((nt * 16, nb, 32), np.uint8)
    if dt == po.Q8_0:
        b = wq.reshape(N, nb, 36)
        scale[:N] = b[..., :4].copy().view(np.float32)[..., 0]
        vals[:N] = b[..., 4:]
    else:
        b = wq.reshape(N, nb, 18)
        scale[:N] = b[..., :2].copy().view(np.float16)[..., 0].astype(np.float32)
        q = b[..., 2:]
        nib = np.stack([q & 15, q >> 4], axis=-1).reshape(N, nb, 32).astype(np.int32) - 8
        lut = np.array([E4M3[v] for v in range(-8, 8)], np.uint8)
        vals[:N] = lut[nib + 8]
    del out
    res = np.zeros((nb, nt, 576), np.uint8)  # block-major
    sc = scale.reshape(nt, 16, nb).transpose(2, 0, 1)  # block, tile, row
    res[..., :64] = sc.copy().view(np.uint8).reshape(nb, nt, 64)
    v = vals.reshape(nt, 16, nb, 4, 8).transpose(2, 0, 3, 1, 4)  # block, tile, seg, row, 8
    res[..., 64:] = v.reshape(nb, nt, 512)
    return res.reshape(-1)


@pytest.mark.parametrize("dt", [po.Q8_0, po.Q4_0])
@pytest.mark.parametrize("shape", [(2048, 2048), (100, 64), (65, 96)], ids=lambda c: "x".join(map(str, c)))
def test_repack_mx_layout(hip, dt, shape):
    from qraf_amd.backend import DeviceBuffer
    call, lib = hip._lib.call, hip._lib.lib
    N, K = shape
    rng = np.random.default_rng(N * K + dt + 1)
    wq = po.quantize(dt, rng.standard_normal(N * K).astype(np.float32))
    nbytes = lib.qraf_hip_mx_weight_bytes(dt, N, K)
    assert nbytes == ((N + 15) // 16) * (K // 32) * 576
    dw, dm = DeviceBuffer.from_array(wq), DeviceBuffer(nbytes)
    call("qraf_hip_repack_mx_dev", dw.ptr, dt, N, K, dm.ptr, None)
    call("qraf_hip_stream_synchronize", None)
    got = dm.download(np.uint8, nbytes)
    want = mx_reference(wq, dt, N, K)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} bytes differ, first at {bad[:8]}: got {got[bad[:8]]}, want {want[bad[:8]]}"


def run_mx(hip, wq, dt, N, K, X, shape=-1, splits=0, workspace=True, add=None, silu=False, repeats=1):
    from qraf_amd.backend import DeviceBuffer
    call, lib = hip._lib.call, hip._lib.lib
    M = X.shape[0]
    call("qraf_hip_set_mx_tuning", shape, splits)
    try:
        dw, dx = DeviceBuffer.from_array(wq), DeviceBuffer.from_array(X)
        dm = DeviceBuffer(lib.qraf_hip_mx_weight_bytes(dt, N, K))
        call("qraf_hip_repack_mx_dev", dw.ptr, dt, N, K, dm.ptr, None)
        dh, dl = DeviceBuffer(M * K * 2), DeviceBuffer(M * K * 2)
        call("qraf_hip_split_bf16_dev", dx.ptr, dh.ptr, dl.ptr, M, K, None)
        outs = []
        if silu:
            F = N // 2
            oh, ol = DeviceBuffer(M * F * 2), DeviceBuffer(M * F * 2)
            call("qraf_hip_qgemm_mx_silu_dev", dm.ptr, dt, N, K, dh.ptr, dl.ptr, M, oh.ptr, ol.ptr, None)
            call("qraf_hip_stream_synchronize", None)
            return oh.download(np.uint16, M * F).reshape(M, F), ol.download(np.uint16, M * F).reshape(M, F)
        wsb = lib.qraf_hip_qgemm_mx_workspace_bytes(dt, N, K, M) if workspace else 0
        ws = DeviceBuffer(wsb) if wsb else None
        dy = DeviceBuffer(M * N * 4)
        da = DeviceBuffer.from_array(add) if add is not None else None
        for _ in range(repeats):
            call("qraf_hip_qgemm_mx_dev", dm.ptr, dt, N, K, dh.ptr, dl.ptr, M, dy.ptr, da.ptr if da else None,
                 ws.ptr if ws else None, wsb, None)
            call("qraf_hip_stream_synchronize", None)
            outs.append(dy.download(np.float32, M * N).reshape(M, N))
        for o in outs[1:]:
            assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32)), "repeated GEMM differs"
        return outs[0]
    finally:
        call("qraf_hip_set_mx_tuning", -1, 0)


CASES = [
    # (N, K, batch): the continuous-batch projections at 128 rows, prefill-sized batches, ragged shapes
    (2560, 2048, 128), (2048, 2048, 128), (11008, 2048, 128), (2048, 11008, 128), (256, 2048, 64),
    (2048, 2048, 200), (513, 1024, 257), (1000, 576, 100), (100, 64, 1), (65, 96, 3), (300, 2048, 80),
    (2048, 2048, 512),
]


@pytest.mark.parametrize("dt", [po.Q8_0, po.Q4_0])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c)))
def test_qgemm_mx_vs_oracle(hip, dt, case):
    N, K, M = case
    print(f"qgemm mx dt={dt} N={N} K={K} M={M}", flush=True)
    rng = np.random.default_rng(N + K + M + dt + 7)
    wq = po.quantize(dt, (rng.standard_normal(N * K) * 0.02).astype(np.float32))
    X = rng.standard_normal((M, K)).astype(np.float32)
    Y = run_mx(hip, wq, dt, N, K, X, repeats=2)
    check(Y, wq, dt, N, K, X)
    Y1 = run_mx(hip, wq, dt, N, K, X, workspace=False)  # one split
    check(Y1, wq, dt, N, K, X)


@pytest.mark.parametrize("shape", [0, 1, 2, 3])
@pytest.mark.parametrize("splits", [1, 3, 7])
def test_qgemm_mx_forced_shapes_and_splits(hip, shape, splits):
    N, K, M = 1000, 2048, 150
    dt = po.Q4_0
    print(f"qgemm mx shape={shape} splits={splits}", flush=True)
    rng = np.random.default_rng(shape * 10 + splits)
    wq = po.quantize(dt, (rng.standard_normal(N * K) * 0.02).astype(np.float32))
    X = rng.standard_normal((M, K)).astype(np.float32)
    add = rng.standard_normal((M, N)).astype(np.float32)
    Y = run_mx(hip, wq, dt, N, K, X, shape=shape, splits=splits, add=add)
    check(Y, wq, dt, N, K, X, add=add)


def bf16_bits_to_f64(h):
    return (h.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


@pytest.mark.parametrize("dt", [po.Q8_0, po.Q4_0])
@pytest.mark.parametrize("case", [(2 * 1536, 576, 128), (2 * 11008, 2048, 128), (2 * 300, 1024, 70)],
                         ids=lambda c: "x".join(map(str, c)))
def test_qgemm_mx_silu_gate_epilogue(hip, dt, case):
    """Rows 2i (gate) and 2i+1 (up): the epilogue writes silu(g) * u as hi/lo
    planes.  The GEMM outputs are the plain mx GEMM's at one split (same
    kernel, same order: bit for bit), so the planes must hold silu_gate of
    those outputs to the planes' own precision (2^-20 relative + 2^-25) plus
    a few ulp of expf."""
    N, K, M = case
    print(f"qgemm mx silu dt={dt} N={N} K={K} M={M}", flush=True)
    rng = np.random.default_rng(N + K + M)
    wq = po.quantize(dt, (rng.standard_normal(N * K) * 0.02).astype(np.float32))
    X = rng.standard_normal((M, K)).astype(np.float32)
    Y = run_mx(hip, wq, dt, N, K, X, splits=1)
    check(Y, wq, dt, N, K, X)
    hi, lo = run_mx(hip, wq, dt, N, K, X, splits=1, silu=True)
    g, u = Y[:, 0::2].astype(np.float64), Y[:, 1::2].astype(np.float64)
    want = g / (1.0 + np.exp(-g)) * u
    got = bf16_bits_to_f64(hi) + lo.view(np.float16).astype(np.float64)
    tol = 2.0 ** -20 * np.abs(want) + 2.0 ** -25 + 8 * 2.0 ** -24 * np.abs(want)
    err = np.abs(got - want)
    assert np.all(err <= tol), f"max err {err.max():.3e}, worst ratio {(err / tol).max():.3f}"
