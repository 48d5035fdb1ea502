"""GPU parity of ragged paged decode attention and of the bias/RoPE/append
step against the oracle (attention.cpp:100-150 restated in oracle.c).

K/V live in randomly permuted physical pages; the oracle gathers each
sequence's rows in position order (fp16 pages converted to f32 first, the
same values the kernel reads) and runs the reference's per-head math.
fp16 pages hold V dimension-major ([page][kv head][dim][position]); the
tests keep the logical [page][kv head][position][dim] arrays and transpose
V when they upload it.

Tolerance (floating point, different summation order and chunked online
softmax instead of one sequential pass): |gpu - oracle| <= 1e-5 + 1e-4 |oracle|.
The fp32 score error is below 1e-5 relative for head_dim <= 128, which the
softmax passes through to the output; observed errors are ~1e-6.
"""
import numpy as np
import pytest

from oracle import pyoracle as po

pytestmark = pytest.mark.gpu


@pytest.fixture(params=[1, 2, 3], ids=["chunk", "split", "valu"])
def form(request, hip):
    """Both work decompositions of the matrix-core kernels (1: one workgroup
    per 256-position chunk, 2: balanced split) and the plain VALU kernel (3);
    the automatic choice is restored afterwards."""
    hip._lib.call("qraf_hip_set_attention_tuning", request.param)
    yield request.param
    hip._lib.call("qraf_hip_set_attention_tuning", 0)


def build_cache(rng, ctxs, Hkv, hd, page_size, kv_dtype, extra_pages=7, poison=False):
    """Logical [page][kv head][position][dim] K and V.  poison: positions at
    or past each sequence's context in its last page hold NaN, which the
    kernels must never let reach the output."""
    n = len(ctxs)
    max_ctx = max(ctxs)
    max_pages = (max_ctx + page_size - 1) // page_size
    need = sum((c + page_size - 1) // page_size for c in ctxs)
    num_pages = need + extra_pages
    perm = rng.permutation(num_pages)
    table = np.zeros((n, max_pages), np.int32)
    k = 0
    for s, c in enumerate(ctxs):
        for j in range((c + page_size - 1) // page_size):
            table[s, j] = perm[k]
            k += 1
    np_dt = np.float16 if kv_dtype == po.F16 else np.float32
    K = rng.standard_normal((num_pages, Hkv, page_size, hd)).astype(np_dt)
    V = rng.standard_normal((num_pages, Hkv, page_size, hd)).astype(np_dt)
    if poison:
        for s, c in enumerate(ctxs):
            if c % page_size:
                last = table[s, (c - 1) // page_size]
                K[last, :, c % page_size:, :] = np.nan
                V[last, :, c % page_size:, :] = np.nan
    return table, K, V, max_pages


def device_v(V, kv_dtype):
    return np.ascontiguousarray(V.transpose(0, 1, 3, 2)) if kv_dtype == po.F16 else V


def gather(table, cache, s, ctx, page_size):
    """[ctx][Hkv*hd] f32 rows of sequence s in position order."""
    t = np.arange(ctx)
    return cache[table[s, t // page_size], :, t % page_size, :].reshape(ctx, -1).astype(np.float32)


def run_attention(hip, q, table, K, V, ctxs, H, Hkv, hd, page_size, kv_dtype, max_ctx, repeats=1):
    from qraf_amd.backend import DeviceBuffer
    call = hip._lib.call
    n = len(ctxs)
    ws_bytes = hip.lib.qraf_hip_attention_workspace_bytes(n, H, Hkv, hd, max_ctx)
    ws = DeviceBuffer(ws_bytes)
    ws.zero()
    dq, dK, dV = DeviceBuffer.from_array(q), DeviceBuffer.from_array(K), DeviceBuffer.from_array(device_v(V, kv_dtype))
    dt, dc = DeviceBuffer.from_array(table), DeviceBuffer.from_array(np.array(ctxs, np.int32))
    out = DeviceBuffer(n * H * hd * 4)
    res = []
    for _ in range(repeats):
        call("qraf_hip_paged_attention_dev", dq.ptr, dK.ptr, dV.ptr, kv_dtype, dt.ptr, table.shape[1], dc.ptr, n, H, Hkv,
             hd, page_size, np.float32(1.0 / np.sqrt(np.float32(hd))), max_ctx, out.ptr, ws.ptr, ws_bytes, None)
        call("qraf_hip_stream_synchronize", None)
        res.append(out.download(np.float32, n * H * hd).reshape(n, H * hd))
    return res


def oracle_attention(q, table, K, V, ctxs, H, Hkv, hd, page_size):
    out = []
    for s, c in enumerate(ctxs):
        Ks = gather(table, K, s, c, page_size)
        Vs = gather(table, V, s, c, page_size)
        out.append(po.attention_decode(q[s].reshape(-1), Ks, Vs, H, Hkv, hd))
    return np.stack(out)


def check(got, want):
    err = np.abs(got.astype(np.float64) - want)
    tol = 1e-5 + 1e-4 * np.abs(want)
    assert np.all(err <= tol), f"max err {err.max():.3e}, worst ratio {(err / tol).max():.2f}"


@pytest.mark.parametrize("kv_dtype", [po.F16, po.F32])
def test_attention_ragged_batch_config(hip, form, kv_dtype):
    # 128 sequences, context lengths U[128, 4096] from a seed, 16 q / 2 kv
    # heads, head_dim 128, fp16 (and f32) K/V ~ N(0,1), one query per sequence
    rng = np.random.default_rng(2024)
    ctxs = rng.integers(128, 4097, 128).tolist()
    H, Hkv, hd, ps = 16, 2, 128, 16
    print(f"attention n=128 H={H} Hkv={Hkv} hd={hd} kv_dtype={kv_dtype} sum_ctx={sum(ctxs)}", flush=True)
    table, K, V, _ = build_cache(rng, ctxs, Hkv, hd, ps, kv_dtype)
    q = rng.standard_normal((128, H * hd)).astype(np.float32)
    got = run_attention(hip, q, table, K, V, ctxs, H, Hkv, hd, ps, kv_dtype, 4096, repeats=2)
    assert np.array_equal(got[0], got[1])  # merge counters are reset: repeat launches agree bit for bit
    check(got[0], oracle_attention(q, table, K, V, ctxs, H, Hkv, hd, ps))


@pytest.mark.parametrize("H,Hkv,hd", [(9, 3, 64), (16, 16, 64), (8, 4, 64), (16, 4, 64), (4, 1, 128), (32, 4, 128),
                                     (12, 2, 64), (16, 1, 128), (4, 1, 16), (8, 2, 32)])
@pytest.mark.parametrize("kv_dtype", [po.F16, po.F32])
def test_attention_edge_lengths(hip, form, H, Hkv, hd, kv_dtype):
    # head_dim 16 and 32 take the VALU kernel for fp16 pages too
    rng = np.random.default_rng(H * 7 + hd)
    ctxs = [1, 2, 15, 16, 17, 255, 256, 257, 511, 512, 513, 1000, 3]
    ps = 16
    table, K, V, _ = build_cache(rng, ctxs, Hkv, hd, ps, kv_dtype, poison=True)
    q = (rng.standard_normal((len(ctxs), H * hd)) * 2).astype(np.float32)
    got = run_attention(hip, q, table, K, V, ctxs, H, Hkv, hd, ps, kv_dtype, max(ctxs))
    check(got[0], oracle_attention(q, table, K, V, ctxs, H, Hkv, hd, ps))


@pytest.mark.parametrize("ps", [4, 8, 32, 64])
@pytest.mark.parametrize("kv_dtype", [po.F16, po.F32])
def test_attention_page_sizes(hip, form, ps, kv_dtype):
    rng = np.random.default_rng(ps)
    ctxs = [1, 5, 33, 64, 100, 257, 700]
    H, Hkv, hd = 16, 2, 128
    table, K, V, _ = build_cache(rng, ctxs, Hkv, hd, ps, kv_dtype, poison=True)
    q = rng.standard_normal((len(ctxs), H * hd)).astype(np.float32)
    got = run_attention(hip, q, table, K, V, ctxs, H, Hkv, hd, ps, kv_dtype, max(ctxs))
    check(got[0], oracle_attention(q, table, K, V, ctxs, H, Hkv, hd, ps))


def test_attention_single_position_is_v(hip):
    # softmax over one position is 1: the output is that position's V row
    rng = np.random.default_rng(3)
    table, K, V, _ = build_cache(rng, [1, 1], 2, 128, 16, po.F32)
    q = rng.standard_normal((2, 16 * 128)).astype(np.float32)
    got = run_attention(hip, q, table, K, V, [1, 1], 16, 2, 128, 16, po.F32, 16)[0]
    for s in range(2):
        v = V[table[s, 0], :, 0, :]
        want = np.concatenate([v[h // 8] for h in range(16)])
        assert np.array_equal(got[s], want)


@pytest.mark.parametrize("kv_dtype", [po.F32, po.F16])
def test_rope_append_vs_oracle(hip, kv_dtype):
    from qraf_amd.backend import DeviceBuffer
    call = hip._lib.call
    L = po.lib()
    rng = np.random.default_rng(9)
    H, Hkv, hd, ps, theta = 16, 2, 128, 16, 1e6
    n = 5
    pos = np.array([0, 1, 17, 1000, 4095], np.int32)
    max_pages = 4096 // ps
    table = rng.permutation(n * max_pages).reshape(n, max_pages).astype(np.int32)
    num_pages = n * max_pages
    np_dt = np.float16 if kv_dtype == po.F16 else np.float32
    qkv = rng.standard_normal((n, (H + 2 * Hkv) * hd)).astype(np.float32)
    bias = (rng.standard_normal((H + 2 * Hkv) * hd) * 0.02).astype(np.float32)
    dK = DeviceBuffer(num_pages * Hkv * ps * hd * np.dtype(np_dt).itemsize)
    dV = DeviceBuffer(dK.nbytes)
    dK.zero()
    dV.zero()
    dq = DeviceBuffer(n * H * hd * 4)
    rope = np.zeros(4096 * hd, np.float32)
    call("qraf_hip_rope_table_host", 4096, hd, np.float32(theta), rope.ctypes.data_as(po._fp))
    d_qkv, d_b, d_pos, d_t, d_r = (DeviceBuffer.from_array(a) for a in (qkv, bias, pos, table, rope))
    call("qraf_hip_rope_append_dev", d_qkv.ptr, d_b.ptr, n, H, Hkv, hd, d_pos.ptr, d_r.ptr, dq.ptr, dK.ptr,
         dV.ptr, kv_dtype, d_t.ptr, max_pages, ps, None)
    call("qraf_hip_stream_synchronize", None)
    qo = dq.download(np.float32, n * H * hd).reshape(n, H * hd)
    Kc = dK.download(np_dt, num_pages * Hkv * ps * hd).reshape(num_pages, Hkv, ps, hd)
    Vc = dV.download(np_dt, num_pages * Hkv * ps * hd)
    Vc = (Vc.reshape(num_pages, Hkv, hd, ps).transpose(0, 1, 3, 2) if kv_dtype == po.F16
          else Vc.reshape(num_pages, Hkv, ps, hd))
    fp = po._fp
    for s in range(n):
        row = qkv[s] + bias  # attention.cpp:100-102 (dispatch_add)
        q = row[:H * hd].copy()
        k = row[H * hd:(H + Hkv) * hd].copy()
        v = row[(H + Hkv) * hd:].copy()
        for h in range(H):
            seg = np.ascontiguousarray(q[h * hd:(h + 1) * hd])
            L.or_rope(seg.ctypes.data_as(fp), hd, int(pos[s]), theta)
            q[h * hd:(h + 1) * hd] = seg
        for h in range(Hkv):
            seg = np.ascontiguousarray(k[h * hd:(h + 1) * hd])
            L.or_rope(seg.ctypes.data_as(fp), hd, int(pos[s]), theta)
            k[h * hd:(h + 1) * hd] = seg
        page, off = table[s, pos[s] // ps], pos[s] % ps
        # angles come from the host-libm table and products are not fused:
        # bit-exact with the reference's rope (ops.cpp:158-177) on this host
        assert np.array_equal(qo[s].view(np.uint32), q.view(np.uint32))
        assert np.array_equal(Kc[page, :, off, :].reshape(-1), k.astype(np_dt))
        assert np.array_equal(Vc[page, :, off, :].reshape(-1), v.astype(np_dt))



def test_attention_split_shares_over_many_sequences(hip, form):
    """Batches whose 64-position tiles outnumber the workgroups: shares span
    several sequences and sequences span several shares (merged in order);
    fewer tiles than workgroups: one tile per share."""
    for n, lo, hi, Hkv in [(300, 1, 700, 2), (40, 128, 4096, 2), (7, 1, 90, 16)]:
        rng = np.random.default_rng(n + lo)
        ctxs = rng.integers(lo, hi + 1, n).tolist()
        H, hd = 8 * Hkv if Hkv < 16 else 16, 128 if Hkv < 16 else 64
        print(f"split n={n} ctx {lo}..{hi} Hkv={Hkv}", flush=True)
        table, K, V, _ = build_cache(rng, ctxs, Hkv, hd, 16, po.F16, poison=True)
        q = rng.standard_normal((n, H * hd)).astype(np.float32)
        got = run_attention(hip, q, table, K, V, ctxs, H, Hkv, hd, 16, po.F16, max(ctxs), repeats=2)
        assert np.array_equal(got[0], got[1])
        check(got[0], oracle_attention(q, table, K, V, ctxs, H, Hkv, hd, 16))


@pytest.mark.parametrize("ps", [12, 20])
def test_attention_page_size_not_power_of_two(hip, ps):
    """fp16 pages of such sizes take the VALU kernel (the matrix-core ones
    address pages by shifts)."""
    rng = np.random.default_rng(ps)
    ctxs = [1, 13, 100, 300]
    H, Hkv, hd = 8, 2, 128
    table, K, V, _ = build_cache(rng, ctxs, Hkv, hd, ps, po.F16, poison=True)
    q = rng.standard_normal((len(ctxs), H * hd)).astype(np.float32)
    got = run_attention(hip, q, table, K, V, ctxs, H, Hkv, hd, ps, po.F16, max(ctxs))
    check(got[0], oracle_attention(q, table, K, V, ctxs, H, Hkv, hd, ps))
