"""GPU parity of the batched Q8_0/Q4_0 GEMM (matrix cores) against the
oracle's dispatch_matvec_q applied to every batch row.

Tolerance per output (floating point): the GEMM's activation split (bf16 hi,
fp16 lo) leaves |r| <= 2^-20 |x| + 2^-25 per element and both sides
accumulate in fp32, so
    |y_gpu - y_oracle| <= sum_k |w_k| (2^-20 |x_k| + 2^-25) + 2 (K + 2) 2^-24 sum_k |w_k x_k|.
The split itself is pinned bit-exactly (numpy's correctly rounded bf16 and
fp16 conversions), and single-product GEMMs pin that the matrix cores add
the two planes exactly, fp16 subnormals included.
"""
import ctypes as C

import numpy as np
import pytest

from oracle import pyoracle as po

pytestmark = pytest.mark.gpu


def run_gemm(hip, wq, dt, N, K, X, add=None, split=True, in_place=False, repeats=1, tiled=False):
    """split: pass the split-K workspace (as the engine does); in_place: the
    residual is added into y itself (add == y); tiled: repack the weights
    tile-major on the device and use the tiled GEMM."""
    from qraf_amd.backend import DeviceBuffer
    call, lib = hip._lib.call, hip._lib.lib
    M = X.shape[0]
    dw, dx = DeviceBuffer.from_array(wq), DeviceBuffer.from_array(X)
    if tiled:
        dtl = DeviceBuffer(lib.qraf_hip_tiled_weight_bytes(dt, N, K))
        call("qraf_hip_repack_tiles_dev", dw.ptr, dt, N, K, dtl.ptr, None)
    dh, dl = DeviceBuffer(M * K * 2), DeviceBuffer(M * K * 2)
    dy = DeviceBuffer(M * N * 4)
    da = DeviceBuffer.from_array(add) if add is not None and not in_place else None
    wsq = lib.qraf_hip_qgemm_tiled_workspace_bytes if tiled else lib.qraf_hip_qgemm_workspace_bytes
    wsb = wsq(dt, N, K, M) if split else 0
    ws = DeviceBuffer(wsb) if wsb else None
    call("qraf_hip_split_bf16_dev", dx.ptr, dh.ptr, dl.ptr, M, K, None)
    outs = []
    for _ in range(repeats):
        if in_place:
            dy.upload(np.ascontiguousarray(add, np.float32))
        a = dy.ptr if in_place else (da.ptr if da else None)
        if tiled:
            call("qraf_hip_qgemm_tiled_dev", dtl.ptr, dt, N, K, dh.ptr, dl.ptr, M, dy.ptr, a, ws.ptr if ws else None,
                 wsb, None)
        else:
            call("qraf_hip_qgemm_dev", dw.ptr, dt, 32, N, K, dh.ptr, dl.ptr, M, dy.ptr, a, ws.ptr if ws else None, wsb,
                 None)
        call("qraf_hip_stream_synchronize", None)
        outs.append(dy.download(np.float32, M * N).reshape(M, N))
    Y = outs[0]
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), Y.view(np.uint32)), "repeated GEMM differs"
    return Y, dh.download(np.uint16, M * K), dl.download(np.uint16, M * K)


def check(Y, wq, dt, N, K, X, add=None):
    W = po.dequantize(dt, wq, N * K).reshape(N, K).astype(np.float64)
    absw = np.abs(W)
    for m in range(X.shape[0]):
        y_ref = po.matvec_q(wq, dt, N, K, X[m]).astype(np.float64)
        if add is not None:
            y_ref = y_ref + add[m]
        ax = np.abs(X[m].astype(np.float64))
        tol = 2.0 ** -20 * (absw @ ax) + 2.0 ** -25 * absw.sum(1) + 2 * (K + 2) * 2.0 ** -24 * (absw @ ax) + 1e-30
        if add is not None:
            tol += 2.0 ** -23 * np.abs(y_ref)
        err = np.abs(Y[m] - y_ref)
        assert np.all(err <= tol), f"row {m}: max err {err.max():.3e}, worst ratio {(err / tol).max():.3f}"


CASES = [
    # (N, K, batch): Qwen2.5-3B projection shapes at the continuous-batch sizes, ragged cases
    (2048, 2048, 128), (256, 2048, 64), (11008, 2048, 32), (2048, 11008, 8), (2048, 11008, 128),
    (2560, 2048, 17), (100, 64, 1), (65, 96, 3), (1000, 576, 100), (576, 1536, 16), (300, 2048, 80),
    (700, 4096, 48), (130, 128, 2), (2048, 2048, 200), (513, 1024, 257),
    # the largest steps the engine takes (max_batch up to 1024 rows)
    (2560, 2048, 512), (576, 1536, 1024),
]


@pytest.mark.parametrize("dt", [po.Q8_0, po.Q4_0])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c)))
def test_qgemm_vs_oracle(hip, dt, case):
    N, K, M = case
    print(f"qgemm dt={dt} N={N} K={K} M={M}", flush=True)
    rng = np.random.default_rng(N + K + M + dt)
    wq = po.quantize(dt, (rng.standard_normal(N * K) * 0.02).astype(np.float32))
    X = rng.standard_normal((M, K)).astype(np.float32)
    Y, _, _ = run_gemm(hip, wq, dt, N, K, X, repeats=2)
    check(Y, wq, dt, N, K, X)
    Y1, _, _ = run_gemm(hip, wq, dt, N, K, X, split=False)  # one split, no workspace
    check(Y1, wq, dt, N, K, X)
    # tile-major weights: up to 16 rows the same kernel and split, bit for bit;
    # larger batches run the wave-split or the pipelined kernel (own tiling and split)
    Yt, _, _ = run_gemm(hip, wq, dt, N, K, X, tiled=True, repeats=2)
    check(Yt, wq, dt, N, K, X)
    if M <= 16:
        assert np.array_equal(Yt.view(np.uint32), Y.view(np.uint32))
    Yt1, _, _ = run_gemm(hip, wq, dt, N, K, X, tiled=True, split=False)
    check(Yt1, wq, dt, N, K, X)


C3_SHAPES = [(2048, 2048), (256, 2048), (11008, 2048), (2048, 11008)]


@pytest.mark.parametrize("dt", [po.Q8_0, po.Q4_0])
@pytest.mark.parametrize("shape", C3_SHAPES, ids=lambda c: "x".join(map(str, c)))
@pytest.mark.parametrize("M", [8, 32, 64, 128])
def test_qgemm_c3_grid(hip, dt, shape, M):
    """The whole batched-GEMM grid of the benchmark: Qwen2.5-3B projection
    shapes at 8, 32, 64 and 128 activation rows, Q8_0 and Q4_0, through the
    tile-major path the engine uses (its automatic kernel and split choice,
    with the split-K workspace), against the oracle; repeated calls
    bit-identical."""
    N, K = shape
    print(f"qgemm C3 dt={dt} N={N} K={K} M={M}", flush=True)
    rng = np.random.default_rng(11 * N + K + M + dt)
    wq = po.quantize(dt, (rng.standard_normal(N * K) * 0.02).astype(np.float32))
    X = rng.standard_normal((M, K)).astype(np.float32)
    Y, _, _ = run_gemm(hip, wq, dt, N, K, X, tiled=True, repeats=2)
    check(Y, wq, dt, N, K, X)


KW_CASES = [
    # (N, K, batch): ragged tile groups, batch tiles and wave shares of the blocks
    (2048, 2048, 128), (11008, 2048, 32), (2048, 11008, 64), (2560, 2048, 17), (300, 512, 64), (1000, 576, 100),
    (513, 1024, 200), (100, 96, 33), (22016, 2048, 48),
]


@pytest.mark.parametrize("dt", [po.Q8_0, po.Q4_0])
@pytest.mark.parametrize("case", KW_CASES, ids=lambda c: "x".join(map(str, c)))
@pytest.mark.parametrize("tiles", [0, 2, 3, 4])
def test_qgemm_wave_split_kernel(hip, dt, case, tiles):
    """The wave-split tiled kernel (qraf_hip_set_qgemm_kw) forced on for every
    shape with 2, 3 or 4 weight tiles per workgroup or its automatic choice:
    the 4 waves' shares of the quant blocks (3 to 86 blocks a wave, shares
    that differ by one, waves without blocks when a split holds fewer than 4),
    batch tiles past the rows and weight tiles past the matrix, with split-K
    partials and without, against the oracle and bit-identical over repeats."""
    N, K, M = case
    rng = np.random.default_rng(3 * N + K + 7 * M + dt)
    wq = po.quantize(dt, (rng.standard_normal(N * K) * 0.02).astype(np.float32))
    X = rng.standard_normal((M, K)).astype(np.float32)
    call = hip._lib.call
    call("qraf_hip_set_qgemm_kw", 1, tiles)
    try:
        Y, _, _ = run_gemm(hip, wq, dt, N, K, X, tiled=True, repeats=2)
        Y1, _, _ = run_gemm(hip, wq, dt, N, K, X, tiled=True, split=False)
    finally:
        call("qraf_hip_set_qgemm_kw", 0, 0)
    check(Y, wq, dt, N, K, X)
    check(Y1, wq, dt, N, K, X)


@pytest.mark.parametrize("dt", [po.Q8_0, po.Q4_0])
@pytest.mark.parametrize("case", KW_CASES + [(15000, 512, 128), (2048, 11008, 256)],
                         ids=lambda c: "x".join(map(str, c)))
def test_qgemm_row_split_kernel(hip, dt, case):
    """The row-split tiled kernel with LDS-shared activations (forced on
    through qraf_hip_set_qgemm_tuning's pipe = 3): 192 weight rows per
    workgroup in 4 waves of 48, 64- or 128-row batch chunks, a 3-stage ring
    of direct-to-LDS loads (workgroups past the weight tiles, batch tiles past
    the rows, the last stage trip padded), with split-K partials and without,
    against the oracle and bit-identical over repeats."""
    N, K, M = case
    rng = np.random.default_rng(5 * N + K + 3 * M + dt)
    wq = po.quantize(dt, (rng.standard_normal(N * K) * 0.02).astype(np.float32))
    X = rng.standard_normal((M, K)).astype(np.float32)
    call = hip._lib.call
    call("qraf_hip_set_qgemm_tuning", 0, 0, 3, 0)
    try:
        Y, _, _ = run_gemm(hip, wq, dt, N, K, X, tiled=True, repeats=2)
        Y1, _, _ = run_gemm(hip, wq, dt, N, K, X, tiled=True, split=False)
    finally:
        call("qraf_hip_set_qgemm_tuning", 0, 0, 0, 0)
    check(Y, wq, dt, N, K, X)
    check(Y1, wq, dt, N, K, X)


@pytest.mark.parametrize("in_place", [True, False])
@pytest.mark.parametrize("split", [True, False])
def test_qgemm_wave_split_residual(hip, split, in_place):
    """The wave-split kernel's residual epilogue (y = W x + add, add == y in
    place) in the single-split form and through the split-K reduction."""
    rng = np.random.default_rng(9)
    N, K, M = 2048, 2048, 40
    wq = po.quantize(po.Q4_0, (rng.standard_normal(N * K) * 0.02).astype(np.float32))
    X = rng.standard_normal((M, K)).astype(np.float32)
    add = rng.standard_normal((M, N)).astype(np.float32)
    hip._lib.call("qraf_hip_set_qgemm_kw", 1, 0)
    try:
        Y, _, _ = run_gemm(hip, wq, po.Q4_0, N, K, X, add, split=split, in_place=in_place, tiled=True)
    finally:
        hip._lib.call("qraf_hip_set_qgemm_kw", 0, 0)
    check(Y, wq, po.Q4_0, N, K, X, add)


def tile_major_reference(wq, dt, N, K):
    """The documented tile-major layout, built from the reference bytes with numpy."""
    bb, sb = (36, 4) if dt == po.Q8_0 else (18, 2)
    nb, nt = K // 32, (N + 15) // 16
    rows = np.zeros((nt * 16, nb, bb), np.uint8)
    rows[:N] = wq.reshape(N, nb, bb)
    t = rows.reshape(nt, 16, nb, bb).transpose(0, 2, 1, 3)  # tile, block, row, bytes
    return np.concatenate([t[..., :sb].reshape(nt, nb, 16 * sb), t[..., sb:].reshape(nt, nb, 16 * (bb - sb))],
                          axis=2).reshape(-1)


@pytest.mark.parametrize("dt", [po.Q8_0, po.Q4_0])
@pytest.mark.parametrize("shape", [(2048, 2048), (100, 64), (65, 96), (1000, 576)], ids=lambda c: "x".join(map(str, c)))
def test_repack_tiles_layout(hip, dt, shape):
    from qraf_amd.backend import DeviceBuffer
    call, lib = hip._lib.call, hip._lib.lib
    N, K = shape
    rng = np.random.default_rng(N * K + dt)
    wq = po.quantize(dt, rng.standard_normal(N * K).astype(np.float32))
    nbytes = lib.qraf_hip_tiled_weight_bytes(dt, N, K)
    ref = tile_major_reference(wq, dt, N, K)
    assert nbytes == ref.size
    dw, dt_ = DeviceBuffer.from_array(wq), DeviceBuffer(nbytes)
    call("qraf_hip_repack_tiles_dev", dw.ptr, dt, N, K, dt_.ptr, None)
    call("qraf_hip_stream_synchronize", None)
    assert np.array_equal(dt_.download(np.uint8, nbytes), ref)


@pytest.mark.parametrize("dt", [po.Q8_0, po.Q4_0])
@pytest.mark.parametrize("case", [(8192, 1024, 100), (2048, 2048, 128), (300, 512, 64), (1000, 576, 33)],
                         ids=lambda c: "x".join(map(str, c)))
@pytest.mark.parametrize("form", [(1, 0), (2, 0), (2, 128)], ids=["wide", "narrow64", "narrow128"])
def test_qgemm_pipelined_kernel(hip, dt, case, form):
    """The pipelined tiled kernel (direct-to-LDS 3-stage ring), in its wide
    (8 waves, 256 weight rows) and narrow (4 waves, 128 weight rows; 64- or
    128-row batch chunks) forms, forced on for every shape, with and without
    split-K, against the oracle."""
    N, K, M = case
    rng = np.random.default_rng(N + 3 * K + M + dt)
    wq = po.quantize(dt, (rng.standard_normal(N * K) * 0.02).astype(np.float32))
    X = rng.standard_normal((M, K)).astype(np.float32)
    hip._lib.call("qraf_hip_set_qgemm_tuning", 0, 0, form[0], form[1])
    try:
        Y, _, _ = run_gemm(hip, wq, dt, N, K, X, tiled=True, repeats=2)
        Y1, _, _ = run_gemm(hip, wq, dt, N, K, X, tiled=True, split=False)
    finally:
        hip._lib.call("qraf_hip_set_qgemm_tuning", 0, 0, 0, 0)
    check(Y, wq, dt, N, K, X)
    check(Y1, wq, dt, N, K, X)


@pytest.mark.parametrize("case", [(16384, 2048, 128), (16384, 2048, 200)], ids=lambda c: "x".join(map(str, c)))
def test_qgemm_pipelined_384_row_tiles(hip, case):
    """Q4_0 wide products where the plan takes the 384-weight-row form of the
    pipelined kernel (8 waves of 128 batch rows x 48 weight rows; it fills more
    CUs than 256-row tiles at these shapes: four split-K slices at 128 rows,
    two at 200, the second batch chunk partial), against the oracle."""
    N, K, M = case
    lib = hip._lib.lib
    assert lib.qraf_hip_qgemm_tiled_workspace_bytes(po.Q4_0, N, K, M) == (4 if M == 128 else 2) * M * N * 4
    rng = np.random.default_rng(N + 7 * K + M)
    wq = po.quantize(po.Q4_0, (rng.standard_normal(N * K) * 0.02).astype(np.float32))
    X = rng.standard_normal((M, K)).astype(np.float32)
    print(f"qgemm 384-row tiles N={N} K={K} M={M}", flush=True)
    Y, _, _ = run_gemm(hip, wq, po.Q4_0, N, K, X, tiled=True, repeats=2)
    check(Y, wq, po.Q4_0, N, K, X)
    try:  # the same form under the stream-K schedule
        hip._lib.call("qraf_hip_set_qgemm_schedule", 1, 0)
        Ys, _, _ = run_gemm(hip, wq, po.Q4_0, N, K, X, tiled=True)
    finally:
        hip._lib.call("qraf_hip_set_qgemm_schedule", 0, 0)
    check(Ys, wq, po.Q4_0, N, K, X)


@pytest.mark.parametrize("dt", [po.Q8_0, po.Q4_0])
@pytest.mark.parametrize("case", [(8192, 1024, 100), (2560, 2048, 130), (300, 512, 64), (1000, 576, 33)],
                         ids=lambda c: "x".join(map(str, c)))
@pytest.mark.parametrize("form", [(1, 0), (2, 0), (2, 128)], ids=["wide", "narrow64", "narrow128"])
@pytest.mark.parametrize("min_blocks", [0, 5, 7])
def test_qgemm_stream_k(hip, dt, case, form, min_blocks):
    """The stream-K schedule of the pipelined kernel, forced on: equal shares
    of the (tile, block) pairs that start and end inside tiles (shares of 16,
    5 or 7 blocks, so segments of every length and position occur, batch
    chunks included), each tile's segments summed in order through the
    workspace, unused slices zeroed; against the oracle, deterministic over
    repeats, and within the tolerance of the uniform split-K grid."""
    N, K, M = case
    rng = np.random.default_rng(7 * N + K + M + dt)
    wq = po.quantize(dt, (rng.standard_normal(N * K) * 0.02).astype(np.float32))
    X = rng.standard_normal((M, K)).astype(np.float32)
    call = hip._lib.call
    call("qraf_hip_set_qgemm_tuning", 0, 0, form[0], form[1])
    try:
        call("qraf_hip_set_qgemm_schedule", 1, min_blocks)
        ws = hip._lib.lib.qraf_hip_qgemm_tiled_workspace_bytes(dt, N, K, M)
        Y, _, _ = run_gemm(hip, wq, dt, N, K, X, tiled=True, repeats=2)
        call("qraf_hip_set_qgemm_schedule", 2, 0)
        Yu, _, _ = run_gemm(hip, wq, dt, N, K, X, tiled=True)
    finally:
        call("qraf_hip_set_qgemm_schedule", 0, 0)
        call("qraf_hip_set_qgemm_tuning", 0, 0, 0, 0)
    if min_blocks:  # shares of 5 or 7 blocks, shorter than every tile here
        assert ws > 0, "stream-K with shares shorter than a tile must use partial slices"
    check(Y, wq, dt, N, K, X)
    check(Yu, wq, dt, N, K, X)


def test_qgemm_stream_k_plan(hip):
    """The schedule knob through the workspace query (host-side plan): the
    default keeps the uniform grid (the 128-row gate/up product in four
    split-K slices of 384-row tiles, 11008 rows in four slices of 256-row
    tiles, the LM head in whole tiles without partials); forced stream-K
    shares the head's tiles too."""
    lib, call = hip._lib.lib, hip._lib.call
    q = lib.qraf_hip_qgemm_tiled_workspace_bytes
    assert q(po.Q4_0, 22016, 2048, 128) == 4 * 128 * 22016 * 4
    assert q(po.Q4_0, 11008, 2048, 128) == 4 * 128 * 11008 * 4
    assert q(po.Q4_0, 151936, 2048, 128) == 0
    try:
        call("qraf_hip_set_qgemm_schedule", 1, 0)
        forced = q(po.Q4_0, 151936, 2048, 128)
    finally:
        call("qraf_hip_set_qgemm_schedule", 0, 0)
    assert forced > 0


@pytest.mark.parametrize("dt", [po.Q8_0, po.Q4_0])
@pytest.mark.parametrize("case", [(2 * 1536, 576, 128), (2 * 11008, 2048, 128), (2 * 300, 1024, 70),
                                  (2 * 11008, 2048, 200), (2 * 64, 64, 33), (2 * 11008, 2048, 32)],
                         ids=lambda c: "x".join(map(str, c)))
@pytest.mark.parametrize("form", ["pipelined", "wave_split", "row_split"])
def test_qgemm_tiled_silu_epilogue(hip, dt, case, form):
    """qraf_hip_qgemm_tiled_silu_dev: rows 2i (gate) and 2i+1 (up) summed
    unsplit by the pipelined kernel (narrow form, 64-row chunks) or the
    wave-split kernel, the epilogue writing silu(g) * u as hi/lo planes.  The
    plain tiled GEMM forced into the same form with one split gives the same
    sums bit for bit (the row-split kernel, pipe = 3, as a third form), which are checked against the oracle; the planes must
    hold silu_gate of those sums to the planes' own precision (2^-20 relative
    + 2^-25) plus a few ulp of expf."""
    from qraf_amd.backend import DeviceBuffer
    N, K, M = case
    print(f"qgemm tiled silu dt={dt} N={N} K={K} M={M} {form}", flush=True)
    rng = np.random.default_rng(N + 5 * K + M)
    wq = po.quantize(dt, (rng.standard_normal(N * K) * 0.02).astype(np.float32))
    X = rng.standard_normal((M, K)).astype(np.float32)
    call, lib = hip._lib.call, hip._lib.lib
    F = N // 2
    dw, dx = DeviceBuffer.from_array(wq), DeviceBuffer.from_array(X)
    dtl = DeviceBuffer(lib.qraf_hip_tiled_weight_bytes(dt, N, K))
    call("qraf_hip_repack_tiles_dev", dw.ptr, dt, N, K, dtl.ptr, None)
    dh, dl = DeviceBuffer(M * K * 2), DeviceBuffer(M * K * 2)
    call("qraf_hip_split_bf16_dev", dx.ptr, dh.ptr, dl.ptr, M, K, None)
    oh, ol = DeviceBuffer(M * F * 2), DeviceBuffer(M * F * 2)
    if form == "pipelined":
        call("qraf_hip_set_qgemm_tuning", 0, 1, 2, 0)
    elif form == "row_split":
        call("qraf_hip_set_qgemm_tuning", 0, 1, 3, 0)
    else:
        call("qraf_hip_set_qgemm_tuning", 0, 1, 0, 0)
        call("qraf_hip_set_qgemm_kw", 1, 0)
    try:
        Y, _, _ = run_gemm(hip, wq, dt, N, K, X, tiled=True, split=False)
        if form == "pipelined":  # the epilogue entry's own automatic choice is this form at these shapes
            call("qraf_hip_set_qgemm_tuning", 0, 0, 0, 0)
            call("qraf_hip_set_qgemm_kw", -1, 0)
        call("qraf_hip_qgemm_tiled_silu_dev", dtl.ptr, dt, N, K, dh.ptr, dl.ptr, M, oh.ptr, ol.ptr, None)
        call("qraf_hip_stream_synchronize", None)
    finally:
        call("qraf_hip_set_qgemm_tuning", 0, 0, 0, 0)
        call("qraf_hip_set_qgemm_kw", 0, 0)
    check(Y, wq, dt, N, K, X)
    hi = oh.download(np.uint16, M * F).reshape(M, F)
    lo = ol.download(np.uint16, M * F).reshape(M, F)
    g, u = Y[:, 0::2].astype(np.float64), Y[:, 1::2].astype(np.float64)
    want = g / (1.0 + np.exp(-g)) * u
    got = (hi.astype(np.uint32) << 16).view(np.float32).astype(np.float64) + lo.view(np.float16).astype(np.float64)
    tol = 2.0 ** -20 * np.abs(want) + 2.0 ** -25 + 8 * 2.0 ** -24 * np.abs(want)
    err = np.abs(got - want)
    assert np.all(err <= tol), f"max err {err.max():.3e}, worst ratio {(err / tol).max():.3f}"


def test_qgemm_split_k_is_used(hip):
    lib = hip._lib.lib
    # few 128-row tiles and a long K: the split-K path must be chosen
    assert lib.qraf_hip_qgemm_workspace_bytes(po.Q4_0, 2048, 11008, 128) > 0
    assert lib.qraf_hip_qgemm_workspace_bytes(po.Q8_0, 2048, 2048, 8) > 0
    # many tiles: no split
    assert lib.qraf_hip_qgemm_workspace_bytes(po.Q4_0, 151936, 2048, 128) == 0


@pytest.mark.parametrize("tiled", [False, True])
@pytest.mark.parametrize("split", [True, False])
@pytest.mark.parametrize("in_place", [True, False])
def test_qgemm_residual_epilogue(hip, split, in_place, tiled):
    rng = np.random.default_rng(5)
    N, K, M = 2048, 2048, 40
    wq = po.quantize(po.Q8_0, (rng.standard_normal(N * K) * 0.02).astype(np.float32))
    X = rng.standard_normal((M, K)).astype(np.float32)
    add = rng.standard_normal((M, N)).astype(np.float32)
    Y, _, _ = run_gemm(hip, wq, po.Q8_0, N, K, X, add, split=split, in_place=in_place, tiled=tiled)
    check(Y, wq, po.Q8_0, N, K, X, add)


def split_planes(X):
    """The planes the split must produce: hi = round-to-nearest-even bf16 of
    x, lo = round-to-nearest-even fp16 of x - hi clamped to +-65504."""
    b = X.view(np.uint32).astype(np.uint64)
    hi = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    hv = (hi.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    lo = np.clip(X.astype(np.float64) - hv, -65504, 65504).astype(np.float16)
    return hi, lo


def test_split_bf16_reconstruction(hip):
    rng = np.random.default_rng(6)
    X = (rng.standard_normal((7, 4096)) * np.exp(rng.uniform(-30, 30, (7, 4096)))).astype(np.float32)
    X[0, :4] = [0.0, -0.0, 1.0, -3.0]
    _, h, l = run_gemm(hip, np.zeros(36 * 4096 // 32, np.uint8), po.Q8_0, 1, 4096, X)
    ref_hi, ref_lo = split_planes(X)
    assert np.array_equal(h.reshape(X.shape), ref_hi)
    assert np.array_equal(l.reshape(X.shape), ref_lo.view(np.uint16))
    hi = (h.astype(np.uint32) << 16).view(np.float32).reshape(X.shape).astype(np.float64)
    lo = l.view(np.float16).reshape(X.shape).astype(np.float64)
    ax = np.abs(X.astype(np.float64))
    err = np.abs(hi + lo - X)
    small = ax < 2.0 ** 24
    assert np.all(err[small] <= 2.0 ** -20 * ax[small] + 2.0 ** -25)
    assert np.all(err[~small] <= 2.0 ** -8 * ax[~small])


@pytest.mark.parametrize("N,M,tiled", [(16, 5, False), (8192, 128, True)])
def test_planes_added_exactly(hip, N, M, tiled):
    """One product per output: weight row n is 1 at k = n % 32 (Q8_0, scale
    1), so y[m][n] = hi + lo of x[m][n % 32] exactly, for x from 1e-7 (fp16
    subnormal lo) to 1e6; N = 8192 at 128 rows runs the pipelined kernel."""
    K = 32
    rng = np.random.default_rng(N + M)
    X = (rng.choice([-1.0, 1.0], (M, K)) * 10.0 ** rng.uniform(-7, 6, (M, K))).astype(np.float32)
    wq = np.zeros((N, 36), np.uint8)
    wq[:, :4] = np.frombuffer(np.float32(1.0).tobytes(), np.uint8)
    wq[np.arange(N), 4 + np.arange(N) % K] = 1
    Y, h, l = run_gemm(hip, wq.reshape(-1), po.Q8_0, N, K, X, tiled=tiled)
    hi = (h.astype(np.uint32) << 16).view(np.float32).reshape(M, K).astype(np.float64)
    lo = l.view(np.float16).reshape(M, K).astype(np.float64)
    want = (hi + lo).astype(np.float32)[:, np.arange(N) % K]
    assert np.array_equal(Y.view(np.uint32), want.view(np.uint32))
    ax = np.abs(X.astype(np.float64))[:, np.arange(N) % K]
    assert np.all(np.abs(Y - X[:, np.arange(N) % K].astype(np.float64)) <= 2.0 ** -20 * ax + 2.0 ** -25)

ARGMAX_CASES = [
    # (distinct weight rows R, K, batch): the matrix holds them twice, [W; W], plus one more row
    (4100, 256, 100), (8192, 512, 65), (10000, 1024, 128), (16000, 2048, 200),  # wide pipelined form
    (2500, 2048, 130),                                                           # narrow pipelined form
    (150, 512, 64), (8192, 2048, 40),                                            # other forms: nothing fused
]


@pytest.mark.parametrize("dt", [po.Q8_0, po.Q4_0])
@pytest.mark.parametrize("case", ARGMAX_CASES, ids=lambda c: "x".join(map(str, c)))
def test_qgemm_tiled_argmax(hip, dt, case):
    """The greedy head's fused argmax (qraf_hip_qgemm_tiled_argmax_dev) equals
    Sampler::argmax (sampler.cpp:25-35, the first of the largest values:
    numpy's argmax) of the unsplit tiled GEMM's own product, where the plan
    is the pipelined form (fused = 1); elsewhere it launches nothing
    (fused = 0, the tokens untouched).  The weights hold every row twice, at
    i and R + i, so every logit ties with one 2R rows / many workgroups away
    and only the smaller index wins; a last extra row makes the row count
    ragged.  A keys buffer one entry short also launches nothing."""
    from qraf_amd.backend import DeviceBuffer
    call, lib = hip._lib.call, hip._lib.lib
    R, K, M = case
    N = 2 * R + 1
    rng = np.random.default_rng(R + 5 * K + M + dt)
    half = po.quantize(dt, (rng.standard_normal(R * K) * 0.02).astype(np.float32))
    extra = po.quantize(dt, (rng.standard_normal(K) * 0.02).astype(np.float32))
    wq = np.concatenate([half, half, extra])
    X = rng.standard_normal((M, K)).astype(np.float32)
    Y, _, _ = run_gemm(hip, wq, dt, N, K, X, tiled=True, split=False)
    assert np.array_equal(Y[:, :R].view(np.uint32), Y[:, R:2 * R].view(np.uint32)), "repeated rows differ"
    want = np.argmax(Y, axis=1)
    assert np.all(want < R) or np.any(want == 2 * R)
    dw, dx = DeviceBuffer.from_array(wq), DeviceBuffer.from_array(X)
    dtl = DeviceBuffer(lib.qraf_hip_tiled_weight_bytes(dt, N, K))
    call("qraf_hip_repack_tiles_dev", dw.ptr, dt, N, K, dtl.ptr, None)
    dh, dl = DeviceBuffer(M * K * 2), DeviceBuffer(M * K * 2)
    call("qraf_hip_split_bf16_dev", dx.ptr, dh.ptr, dl.ptr, M, K, None)
    kb = lib.qraf_hip_qgemm_tiled_argmax_keys_bytes(N, M)
    assert kb == -(-N // 128) * M * 8
    keys = DeviceBuffer(kb)
    sentinel = np.full(M, 0xFFFFFFFF, np.uint32)
    dtok = DeviceBuffer.from_array(sentinel)
    fused = C.c_int32(-1)
    print(f"qgemm argmax N={N} K={K} M={M} dt={dt}", flush=True)
    call("qraf_hip_qgemm_tiled_argmax_dev", dtl.ptr, dt, N, K, dh.ptr, dl.ptr, M, keys.ptr, kb, dtok.ptr,
         C.byref(fused), None)
    call("qraf_hip_stream_synchronize", None)
    got = dtok.download(np.uint32, M)
    pipelined = R != 150 and M > 64
    assert fused.value == (1 if pipelined else 0)
    if pipelined:
        assert np.array_equal(got, want.astype(np.uint32)), f"first mismatch at row {np.argmax(got != want)}"
        # a keys buffer too small for the plan's workgroups: nothing launched
        dtok.upload(sentinel)
        call("qraf_hip_qgemm_tiled_argmax_dev", dtl.ptr, dt, N, K, dh.ptr, dl.ptr, M, keys.ptr, 8, dtok.ptr,
             C.byref(fused), None)
        call("qraf_hip_stream_synchronize", None)
        assert fused.value == 0
    assert np.array_equal(dtok.download(np.uint32, M), sentinel)  # not fused: tokens untouched
    for d in (dw, dx, dtl, dh, dl, keys, dtok):
        d.free()
