"""qraf_hip_paged_attention_noalloc_dev, the no-allocation form of
qraf_hip_paged_attention_dev (its workspace is a file-scope device array),
against the allocating entry point on the same inputs: outputs bit for bit
equal, on two calls in a row (the second on a smaller batch, so it runs in
scratch that still holds the first call's partials), and a shape beyond the
scratch refused before any launch."""
import numpy as np
import pytest

from oracle import pyoracle as po
from tests.test_gpu_attention import build_cache, device_v

pytestmark = pytest.mark.gpu


def _inputs(rng, ctxs, H, Hkv, hd, ps, kv):
    table, K, V, _ = build_cache(rng, ctxs, Hkv, hd, ps, kv)
    q = rng.standard_normal((len(ctxs), H * hd)).astype(np.float32)
    return q, table, K, device_v(V, kv)


def _both(hip, q, table, K, V, ctxs, H, Hkv, hd, ps, kv, max_ctx):
    from qraf_amd.backend import DeviceBuffer
    call = hip._lib.call
    n = len(ctxs)
    dq, dK, dV = DeviceBuffer.from_array(q), DeviceBuffer.from_array(K), DeviceBuffer.from_array(V)
    dt, dc = DeviceBuffer.from_array(table), DeviceBuffer.from_array(np.array(ctxs, np.int32))
    scale = np.float32(1.0 / np.sqrt(np.float32(hd)))
    ws_bytes = hip.lib.qraf_hip_attention_workspace_bytes(n, H, Hkv, hd, max_ctx)
    assert ws_bytes <= hip.lib.qraf_hip_attention_noalloc_max_bytes()
    ws = DeviceBuffer(ws_bytes)
    out_a, out_b = DeviceBuffer(n * H * hd * 4), DeviceBuffer(n * H * hd * 4)
    call("qraf_hip_paged_attention_dev", dq.ptr, dK.ptr, dV.ptr, kv, dt.ptr, table.shape[1], dc.ptr, n, H, Hkv, hd, ps,
         scale, max_ctx, out_a.ptr, ws.ptr, ws_bytes, None)
    call("qraf_hip_paged_attention_noalloc_dev", dq.ptr, dK.ptr, dV.ptr, kv, dt.ptr, table.shape[1], dc.ptr, n, H, Hkv,
         hd, ps, scale, max_ctx, out_b.ptr, None)
    call("qraf_hip_stream_synchronize", None)
    return out_a.download(np.float32, n * H * hd), out_b.download(np.float32, n * H * hd)


def test_noalloc_attention_equals_allocating_entry_point(hip):
    rng = np.random.default_rng(77)
    # first call: the 128-sequence ragged batch (contexts U[128, 4096], 16 / 2 heads, head_dim 128, fp16 pages)
    H, Hkv, hd, ps = 16, 2, 128, 16
    ctxs = rng.integers(128, 4097, 128).tolist()
    print("call 1: 128 sequences, fp16 pages, max context", max(ctxs), flush=True)
    a, b = _both(hip, *_inputs(rng, ctxs, H, Hkv, hd, ps, po.F16), ctxs, H, Hkv, hd, ps, po.F16, 4096)
    assert np.isfinite(a).all()
    assert np.array_equal(a, b)
    # second call, smaller: 9 sequences of 1..700 positions, f32 pages, 8 / 2 heads of 64
    H, Hkv, hd = 8, 2, 64
    ctxs = [1, 5, 63, 64, 65, 256, 257, 511, 700]
    print("call 2: 9 sequences, f32 pages", flush=True)
    a, b = _both(hip, *_inputs(rng, ctxs, H, Hkv, hd, ps, po.F32), ctxs, H, Hkv, hd, ps, po.F32, 700)
    assert np.isfinite(a).all()
    assert np.array_equal(a, b)
