"""End-to-end parity of the GPU decode engine against the oracle's
Transformer::forward / generate_tokens restatement on identical weights.

Bars (floating point): logits within 1e-3 relative + 1e-4 absolute of the
oracle at every position; greedy token streams identical (first 32 tokens).
Weights generated on the device must equal the oracle's byte for byte, which
the bit-identical logits of the generated and the uploaded engine show.
"""
import numpy as np
import pytest

from oracle import pyoracle as po
from tests.conftest import golden

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-3, 1e-4


def oracle_model(kw, seed):
    return po.Model(po.make_config(**kw), seed)


def engine_config(kw):
    from qraf_amd.engine import model_config
    return model_config(kw["vocab"], kw["hidden"], kw["layers"], kw["heads"], kw["kv_heads"], kw["inter"],
                        kw.get("max_seq", 2048), kw.get("rope_theta", 1e4), kw.get("eps", 1e-5))


def upload(m, kw, kv_dtype=po.F32, max_batch=1, num_pages=0):
    from qraf_amd.engine import Transformer
    return Transformer.from_tensors(engine_config(kw), m.tensors(), kv_dtype=kv_dtype, max_batch=max_batch,
                                    num_pages=num_pages)


def check_logits(got, want, what=""):
    err = np.abs(got.astype(np.float64) - want)
    tol = ATOL + RTOL * np.abs(want)
    assert np.all(err <= tol), f"{what}: max err {err.max():.3e}, worst ratio {(err / tol).max():.3f}"


def gap(logits):
    s = np.sort(logits)
    return float(s[-1] - s[-2])


SMALL = {
    "q8_llama": (dict(vocab=512, hidden=64, layers=2, heads=4, kv_heads=2, inter=128, max_seq=128, rope_theta=1e5,
                      eps=1e-5, wdtype=po.Q8_0), 11),
    "q4_qwen2_tied_bias": (dict(vocab=640, hidden=128, layers=2, heads=4, kv_heads=1, inter=160, max_seq=128,
                                rope_theta=1e6, eps=1e-6, wdtype=po.Q4_0, tied=True, qkv_bias=True), 12),
    "f32_llama": (dict(vocab=300, hidden=64, layers=2, heads=2, kv_heads=2, inter=96, max_seq=128, rope_theta=1e4,
                       eps=1e-5, wdtype=po.F32), 13),
    "q4_gqa8_hd128": (dict(vocab=1000, hidden=512, layers=3, heads=4, kv_heads=1, inter=1024, max_seq=256,
                           rope_theta=1e6, eps=1e-6, wdtype=po.Q4_0, tied=True, qkv_bias=True), 14),
    "q8_hd64_gqa3": (dict(vocab=800, hidden=576, layers=2, heads=9, kv_heads=3, inter=1536, max_seq=256,
                          rope_theta=1e5, eps=1e-5, wdtype=po.Q8_0), 15),
    "q4_hd64_gqa2": (dict(vocab=700, hidden=256, layers=2, heads=4, kv_heads=2, inter=512, max_seq=256,
                          rope_theta=1e4, eps=1e-5, wdtype=po.Q4_0), 16),
}


@pytest.mark.parametrize("name", list(SMALL))
def test_forward_logits_vs_oracle(hip, name):
    kw, seed = SMALL[name]
    print(f"engine forward {name}", flush=True)
    m = oracle_model(kw, seed)
    tf = upload(m, kw)
    L = po.lib()
    prompt = [L.or_gen_token(seed, i, kw["vocab"]) for i in range(12)]
    m.reset()
    tf.reset()
    for pos, t in enumerate(prompt):
        check_logits(tf.forward(t, pos), m.forward(t, pos), f"{name} pos {pos}")
    tf.engine.close()


@pytest.mark.parametrize("tuning", [(3, 1, 0), (3, 2, 0), (4, 1, 2), (4, 2, 4), (1, 0, 0), (2, 0, 0)],
                         ids=lambda t: "k%d_r%d_w%d" % t)
@pytest.mark.parametrize("name", ["q8_hd64_gqa3", "q4_gqa8_hd128"])
def test_forward_logits_matvec_kernels(hip, name, tuning):
    """Every batch-1 matvec of the decode forced onto one kernel variant: the
    ring kernels (3, 4) also take the in-place residual of the O and down
    projections through their preloaded residual values."""
    kw, seed = SMALL[name]
    print(f"engine forward {name} matvec tuning {tuning}", flush=True)
    m = oracle_model(kw, seed)
    tf = upload(m, kw)
    L = po.lib()
    prompt = [L.or_gen_token(seed, i, kw["vocab"]) for i in range(6)]
    hip.lib.qraf_hip_set_matvec_tuning(*tuning)
    try:
        m.reset()
        tf.reset()
        for pos, t in enumerate(prompt):
            check_logits(tf.forward(t, pos), m.forward(t, pos), f"{name} {tuning} pos {pos}")
    finally:
        hip.lib.qraf_hip_set_matvec_tuning(0, 0, 0)
        tf.engine.close()


@pytest.mark.parametrize("name", ["q8_llama", "q4_qwen2_tied_bias", "f32_llama"])
def test_golden_logits_and_streams(hip, name):
    # the fixtures were written by the compiled reference itself
    from qraf_amd.engine import InferenceEngine
    from tests.golden.gen_golden import MODELS
    key = {"q8_llama": "model_q8_llama", "q4_qwen2_tied_bias": "model_q4_qwen2", "f32_llama": "model_f32_llama"}[name]
    g = golden(key + ".npz")
    kw, seed, np_, nlog, ngen = MODELS[key]
    m = oracle_model(kw, seed)
    tf = upload(m, kw)
    prompt = g["prompt"].tolist()
    tf.reset()
    for i in range(nlog):
        check_logits(tf.forward(prompt[i], i), g["logits"][i], f"{key} pos {i}")
    eng = InferenceEngine(tf, eos_token=2)
    assert eng.generate_tokens(prompt, ngen, repetition_penalty=1.0) == g["stream"].tolist()
    assert eng.generate_tokens(prompt, ngen, repetition_penalty=1.1) == g["stream_pen"].tolist()
    tf.engine.close()


@pytest.mark.parametrize("name", ["q8_llama", "q4_qwen2_tied_bias", "q4_gqa8_hd128"])
def test_device_generated_weights_match_oracle(hip, name):
    from qraf_amd.engine import Transformer
    kw, seed = SMALL[name]
    m = oracle_model(kw, seed)
    up = upload(m, kw)
    gen = Transformer.synthetic(engine_config(kw), kw["wdtype"], seed, tied=kw.get("tied", False),
                                qkv_bias=kw.get("qkv_bias", False))
    for pos, t in enumerate([3, 1, 4, 1, 5]):
        a, b = up.forward(t, pos), gen.forward(t, pos)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"pos {pos}"
    up.engine.close()
    gen.engine.close()


@pytest.mark.parametrize("kv", [po.F32, po.F16])
def test_greedy_streams_32_tokens(hip, kv):
    from qraf_amd.engine import InferenceEngine
    kw, seed = SMALL["q4_gqa8_hd128"]
    m = oracle_model(kw, seed)
    tf = upload(m, kw, kv_dtype=kv)
    prompt = [po.lib().or_gen_token(seed + 1, i, kw["vocab"]) for i in range(16)]
    want = m.generate(prompt, 32, 1.0, eos=-1)
    got = InferenceEngine(tf, eos_token=None).generate_tokens(prompt, 32, repetition_penalty=1.0)
    assert got == want
    tf.engine.close()


@pytest.mark.parametrize("pipeline", [False, True])
def test_batched_step_equals_single_sequence_decode(hip, pipeline):
    """Several sequences of different lengths advanced together (GEMM path,
    several rows per step) produce each sequence's own greedy stream, and
    logits within tolerance of the oracle; pipelined (step N+1 issued before
    step N's tokens reach the host) or not."""
    from qraf_amd.engine import BatchScheduler, Engine
    kw, seed = SMALL["q4_gqa8_hd128"]
    m = oracle_model(kw, seed)
    L = po.lib()
    e = Engine(engine_config(kw), kv_dtype=po.F32, max_batch=8)
    for name, dt, shape, data in m.tensors():
        e.set_tensor(name, dt, shape, data)
    e.finalize()
    pool = e.free_pages()
    prompts = [[L.or_gen_token(100 + r, i, kw["vocab"]) for i in range(3 + 5 * r)] for r in range(6)]
    sched = BatchScheduler(e, max_batch=4, pipeline=pipeline)  # 6 requests, 4 slots: admission as others finish
    ids = [sched.submit(p, 10 + 3 * r) for r, p in enumerate(prompts)]
    done = {r.id: r for r in sched.run()}
    for r, (i, p) in enumerate(zip(ids, prompts)):
        assert done[i].generated == m.generate(p, 10 + 3 * r, 1.0, eos=-1), f"request {r}"
    assert e.free_pages() == pool  # every retired request returned its pages
    e.close()


@pytest.mark.parametrize("pipeline", [False, True])
@pytest.mark.parametrize("chunk,max_rows,plen", [(7, 32, 9), (64, 40, 9), (3, 4, 9), (512, 512, 31), (300, 300, 33)])
def test_scheduler_chunked_prefill_streams(hip, chunk, max_rows, plen, pipeline):
    """Continuous batching with prompts entering in chunks of up to `chunk`
    tokens per step within a `max_rows` row budget (decode rows first; the
    last two cases run steps of several hundred rows, over the GEMM's
    128-row batch chunk): every request's stream equals its independent
    greedy decode, and every page comes back."""
    from qraf_amd.engine import BatchScheduler, Engine
    kw, seed = SMALL["q4_gqa8_hd128"]
    m = oracle_model(kw, seed)
    L = po.lib()
    e = Engine(engine_config(kw), kv_dtype=po.F16, max_batch=max_rows)
    for name, dt, shape, data in m.tensors():
        e.set_tensor(name, dt, shape, data)
    e.finalize()
    pool = e.free_pages()
    prompts = [[L.or_gen_token(300 + r, i, kw["vocab"]) for i in range(2 + plen * r)] for r in range(7)]
    sched = BatchScheduler(e, max_batch=4, max_rows=max_rows, prefill_chunk=chunk, pipeline=pipeline)
    ids = [sched.submit(p, 6 + 2 * r) for r, p in enumerate(prompts)]
    done = {r.id: r for r in sched.run()}
    for r, (i, p) in enumerate(zip(ids, prompts)):
        assert done[i].generated == m.generate(p, 6 + 2 * r, 1.0, eos=-1), f"request {r}"
    rows_token_by_token = sum(len(p) + 6 + 2 * r - 1 for r, p in enumerate(prompts))
    assert sched.rows == rows_token_by_token  # every prompt token and fed-back token exactly once
    if chunk > 1 and max_rows > 4:
        assert sched.steps < 25 + 6 * plen  # prompts entered in chunks
    assert e.free_pages() == pool
    e.close()


def test_pipelined_scheduler_eos_retirement(hip):
    """Requests that stop on EOS: the pipelined run finds EOS a step late and
    drops the row it had issued past it; every stream equals the unpipelined
    run's (and each request's independent greedy decode cut at EOS), and
    every page comes back."""
    from qraf_amd.engine import BatchScheduler, Engine
    kw, seed = SMALL["q8_llama"]
    m = oracle_model(kw, seed)
    L = po.lib()
    prompts = [[L.or_gen_token(500 + r, i, kw["vocab"]) for i in range(3 + 4 * r)] for r in range(8)]
    full = [m.generate(p, 24, 1.0, eos=-1) for p in prompts]
    # an EOS id that cuts several streams early: the token (past the first)
    # found in the most streams
    streams = {}
    for k, f in enumerate(full):
        for t in set(f[1:]):
            streams.setdefault(t, set()).add(k)
    eos = max(sorted(streams), key=lambda t: len(streams[t]))
    want = [f[:f.index(eos)] if eos in f else f for f in full]
    assert sum(len(w) < 24 for w in want) >= 2, "the EOS id should end at least two streams early"
    runs = {}
    for stop in (None, eos):
        for pipeline in (False, True):
            e = Engine(engine_config(kw), kv_dtype=po.F32, max_batch=16)
            for name, dt, shape, data in m.tensors():
                e.set_tensor(name, dt, shape, data)
            e.finalize()
            pool = e.free_pages()
            sched = BatchScheduler(e, max_batch=3, max_rows=16, prefill_chunk=4, pipeline=pipeline)
            ids = [sched.submit(p, 24, eos=stop) for p in prompts]
            done = {r.id: r for r in sched.run()}
            runs[stop, pipeline] = ([done[i].generated for i in ids], sched.steps, sched.rows)
            assert e.free_pages() == pool
            assert all(r.inflight == 0 for r in done.values())
            e.close()
    # without EOS the pipelined run issues the same steps, row for row
    assert runs[None, True] == runs[None, False]
    assert runs[None, True][0] == full
    assert runs[eos, False][0] == want
    assert runs[eos, True][0] == want
    # with EOS it runs one dropped row per request that stopped on it before
    # its last allowed token (a row past the EOS it had not yet seen)
    dropped = sum(len(w) < 23 for w in want)
    assert runs[eos, True][2] == runs[eos, False][2] + dropped


def test_async_step_token_sources_and_states(hip):
    """Engine.step_async / collect: decode rows fed from the previous step's
    argmax on the device give the host-fed greedy streams; a third step in
    flight, a synchronous step while steps are in flight and a token source
    past the previous step's logit rows are refused."""
    from qraf_amd._lib import HipError
    from qraf_amd.engine import Engine
    kw, seed = SMALL["q4_qwen2_tied_bias"]
    m = oracle_model(kw, seed)
    L = po.lib()
    e = Engine(engine_config(kw), kv_dtype=po.F32, max_batch=32)
    for name, dt, shape, data in m.tensors():
        e.set_tensor(name, dt, shape, data)
    e.finalize()
    prompts = [[L.or_gen_token(700 + r, i, kw["vocab"]) for i in range(5 + 3 * r)] for r in range(3)]
    want = [m.generate(p, 12, 1.0, eos=-1) for p in prompts]
    seqs = [e.seq_create() for _ in prompts]
    # prefill: every prompt in one step, the last row of each wants logits
    rows = [(s, t, i, i == len(p) - 1) for s, p in zip(seqs, prompts) for i, t in enumerate(p)]
    e.step_async([r[0] for r in rows], [r[1] for r in rows], [r[2] for r in rows], want_logits=[r[3] for r in rows])
    got = [[] for _ in prompts]
    src = list(range(len(prompts)))
    for k in range(11):
        pos = [len(p) + k for p in prompts]
        e.step_async(seqs, [0] * len(seqs), pos, token_src=src)
        if k == 0:
            with pytest.raises(HipError):
                e.step_async(seqs, [0] * len(seqs), [x + 1 for x in pos], token_src=src)
            with pytest.raises(HipError):
                e.step(seqs, [0] * len(seqs), [x + 1 for x in pos])
        for j, t in enumerate(e.collect()):
            got[j].append(int(t))
    for j, t in enumerate(e.collect()):
        got[j].append(int(t))
    assert got == want
    with pytest.raises(HipError):
        e.collect()  # nothing in flight
    with pytest.raises(HipError):  # the last step left 3 logit rows
        e.step_async(seqs, [0] * 3, [len(p) + 11 for p in prompts], token_src=[0, 1, 3])
    # a synchronous step works again once everything is collected
    _, nx = e.step(seqs, [w[-1] for w in want], [len(p) + 11 for p in prompts])
    assert len(nx) == 3
    e.close()


def test_batched_logits_and_chunked_prefill(hip):
    from qraf_amd.engine import Engine
    kw, seed = SMALL["q8_hd64_gqa3"]
    m = oracle_model(kw, seed)
    e = Engine(engine_config(kw), kv_dtype=po.F32, max_batch=16)
    for name, dt, shape, data in m.tensors():
        e.set_tensor(name, dt, shape, data)
    e.finalize()
    L = po.lib()
    prompt = [L.or_gen_token(7, i, kw["vocab"]) for i in range(11)]
    a, b = e.seq_create(), e.seq_create()
    # sequence a: the whole prompt in one step (11 rows); b: two rows per step
    lg, _ = e.step([a] * 11, prompt, list(range(11)), logits=True, argmax=False)
    m.reset()
    for i, t in enumerate(prompt):
        check_logits(lg[i], m.forward(t, i), f"chunked prefill row {i}")
    for i in range(0, 10, 2):
        lg2, _ = e.step([b, b], prompt[i:i + 2], [i, i + 1], want_logits=[0, 1], logits=True, argmax=False)
    m.reset()
    for i in range(10):
        ref = m.forward(prompt[i], i)
    check_logits(lg2[0], ref, "two-row steps")
    assert e.seq_length(a) == 11 and e.seq_length(b) == 10
    e.close()


@pytest.mark.parametrize("name,kv", [("q8_llama", "F32"), ("q4_qwen2_tied_bias", "F32"), ("q8_hd64_gqa3", "F16"),
                                     ("q4_gqa8_hd128", "F16")])
def test_fused_qkv_epilogue_equals_separate_launch(hip, name, kv):
    """One-row steps with the QKV bias, RoPE and K/V store fused into the QKV
    matvec (the default) against the separate RoPE/append launch: logits
    bit-identical at every position, so the pages hold the same values."""
    from qraf_amd.engine import Engine
    kw, seed = SMALL[name]
    m = oracle_model(kw, seed)
    L = po.lib()
    toks = [L.or_gen_token(seed + 9, i, kw["vocab"]) for i in range(40)]
    runs = []
    for flags in (1, 0):
        e = Engine(engine_config(kw), kv_dtype=getattr(po, kv), max_batch=4)
        for tname, dt, shape, data in m.tensors():
            e.set_tensor(tname, dt, shape, data)
        e.finalize()
        e.set_fusion(flags)
        a = e.seq_create()
        runs.append([e.step([a], [toks[p]], [p], logits=True, argmax=False)[0].copy() for p in range(40)])
        e.close()
    for p, (x, y) in enumerate(zip(*runs)):
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32)), f"position {p}"
    m.close()


@pytest.mark.parametrize("name", ["q8_hd64_gqa3", "q4_gqa8_hd128", "q4_qwen2_tied_bias", "q4_hd64_gqa2"])
def test_small_steps_on_batch_matvec(hip, name):
    """Steps of 2-8 rows run their projections on the multi-vector matvec
    (fusion bit 2, the default): a seeded schedule of steps mixing prefill
    chunks and single rows of 8 sequences, every row's logits within the
    oracle bar of its own sequence's decode; the same steps with bit 2 off
    run on the batched GEMM, within the bar too and not bit-identical (so the
    matvec path did run)."""
    from qraf_amd.engine import Engine
    kw, seed = SMALL[name]
    m = oracle_model(kw, seed)
    L = po.lib()
    nseq, npos = 8, 12
    toks = [[L.or_gen_token(seed + 40 + s, i, kw["vocab"]) for i in range(npos)] for s in range(nseq)]
    want = []
    for sq in range(nseq):
        m.reset()
        want.append([m.forward(toks[sq][p], p) for p in range(npos)])
    rng = np.random.default_rng(seed)
    nxt, steps = [0] * nseq, []
    while any(v < npos for v in nxt):
        target = int(rng.choice([2, 3, 5, 8]))
        rows = []
        for sq in rng.permutation(nseq):
            while nxt[sq] < npos and len(rows) < target and rng.random() < 0.6:
                rows.append((int(sq), nxt[sq]))
                nxt[sq] += 1
        if rows:
            steps.append(rows)
    assert any(len(r) >= 2 for r in steps)
    runs = []
    for flags in (7, 3):
        print(f"small steps {name}: fusion flags {flags}, {len(steps)} steps", flush=True)
        e = Engine(engine_config(kw), kv_dtype=po.F32, max_batch=8)
        for tname, dt, shape, data in m.tensors():
            e.set_tensor(tname, dt, shape, data)
        e.finalize()
        e.set_fusion(flags)
        ids = [e.seq_create() for _ in range(nseq)]
        out = []
        for rows in steps:
            lg, _ = e.step([ids[sq] for sq, _ in rows], [toks[sq][p] for sq, p in rows], [p for _, p in rows],
                           logits=True, argmax=False)
            for i, (sq, p) in enumerate(rows):
                check_logits(lg[i], want[sq][p], f"{name} flags {flags}, sequence {sq} position {p}")
            out.append(lg.copy())
        runs.append(out)
        e.close()
    assert any(not np.array_equal(a, b) for a, b, rows in zip(runs[0], runs[1], steps) if len(rows) >= 2)
    m.close()


@pytest.mark.parametrize("name", ["q4_gqa8_hd128", "q8_hd64_gqa3"])
def test_swiglu_epilogue_batched_steps(hip, name):
    """Steps over 256 rows with the SiLU-gate in the gate/up GEMM's epilogue
    (fusion bit 1, the default) and with the split-K GEMM plus a separate
    SiLU/split launch: 100 sequences of 3 prompt tokens in one 300-row step,
    then two 100-row decode steps; every logit row of both runs within the
    bar of the oracle's single-sequence decode (the two GEMM forms sum in
    different orders, so they are not bit-identical)."""
    from qraf_amd.engine import Engine
    kw, seed = SMALL[name]
    m = oracle_model(kw, seed)
    L = po.lib()
    prompts = [[L.or_gen_token(seed + 40 + r, i, kw["vocab"]) for i in range(3)] for r in range(100)]
    want, fed = [], []
    for p in prompts:  # the oracle: each sequence alone, 3 prompt tokens then two greedy tokens (fed to both)
        m.reset()
        lg = [m.forward(t, i) for i, t in enumerate(p)][-1]
        rows, toks = [lg], []
        for k in range(2):
            toks.append(int(np.argmax(lg)))
            lg = m.forward(toks[-1], 3 + k)
            rows.append(lg)
        want.append(rows)
        fed.append(toks)
    for flags in (3, 1):
        e = Engine(engine_config(kw), kv_dtype=po.F32, max_batch=320)
        for tname, dt, shape, data in m.tensors():
            e.set_tensor(tname, dt, shape, data)
        e.finalize()
        e.set_fusion(flags)
        seqs = [e.seq_create() for _ in prompts]
        rows = [(s, t, i) for s, p in zip(seqs, prompts) for i, t in enumerate(p)]
        lg, nx = e.step([r[0] for r in rows], [r[1] for r in rows], [r[2] for r in rows],
                        want_logits=[r[2] == 2 for r in rows], logits=True, argmax=True)
        got = [[lg[j]] for j in range(len(prompts))]
        for k in range(2):
            lg, nx = e.step(seqs, [f[k] for f in fed], [3 + k] * len(seqs), logits=True, argmax=True)
            for j in range(len(prompts)):
                got[j].append(lg[j])
        e.close()
        for j in range(len(prompts)):
            for k in range(3):
                check_logits(got[j][k], want[j][k].astype(np.float64), f"flags {flags} sequence {j} row {k}")
    m.close()


def test_attention_form_change_reaches_captured_steps(hip):
    """Changing the attention form (qraf_hip_set_attention_tuning) between
    replayed step graphs: the engine captures new graphs in the new form, so
    every step's logits equal an eager run that changes the form at the same
    steps, bit for bit (the forms themselves round differently)."""
    from qraf_amd.engine import Engine
    kw, seed = SMALL["q4_gqa8_hd128"]
    m = oracle_model(kw, seed)
    L = po.lib()
    toks = [L.or_gen_token(seed + 3, i, kw["vocab"]) for i in range(40)]
    runs = []
    try:
        # graphs with the form switched, eager with the form switched, eager in form 1 throughout
        for graphs, switch in ((True, True), (False, True), (False, False)):
            e = Engine(engine_config(kw), kv_dtype=po.F16, max_batch=4)
            for tname, dt, shape, data in m.tensors():
                e.set_tensor(tname, dt, shape, data)
            e.finalize()
            e.set_graphs(graphs)
            a, b = e.seq_create(), e.seq_create()
            out = []
            for form, steps in ((1, range(0, 12)), (2, range(12, 24)), (3, range(24, 36))):
                hip._lib.call("qraf_hip_set_attention_tuning", form if switch else 1)
                for i in steps:
                    lg, _ = e.step([a, b], [toks[i], toks[i + 1]], [i, i], logits=True, argmax=False)
                    out.append(lg.copy())
            runs.append(out)
            e.close()
    finally:
        hip._lib.call("qraf_hip_set_attention_tuning", 0)
    for i, (x, y) in enumerate(zip(runs[0], runs[1])):
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32)), f"step {i}"
    # the forms do round differently, so a graph left in form 1 would have failed above
    assert any(not np.array_equal(x, y) for x, y in zip(runs[1][12:], runs[2][12:]))
    m.close()


@pytest.mark.parametrize("name", ["q8_hd64_gqa3", "q4_gqa8_hd128"])
def test_step_graph_replay_equals_eager(hip, name):
    """Captured step graphs (the default) against eager launches of the same
    steps: bit-identical logits, for batch-1 decode across context buckets
    (positions up to 300 cross the 256-position bound) and for batched
    chunked-prefill steps; every graph is replayed several times with eager
    steps and host synchronisation in between."""
    from qraf_amd.engine import Engine
    kw, seed = SMALL[name]
    m = oracle_model(kw, seed)
    L = po.lib()
    toks = [L.or_gen_token(seed + 5, i, kw["vocab"]) for i in range(300)]
    runs = []
    for graphs in (True, False):
        e = Engine(engine_config(dict(kw, max_seq=512)), kv_dtype=po.F16, max_batch=8)
        for tname, dt, shape, data in m.tensors():
            e.set_tensor(tname, dt, shape, data)
        e.finalize()
        e.set_graphs(graphs)
        a, b = e.seq_create(), e.seq_create()
        out = []
        # b: prefill in 4-row chunks alongside a's single rows (mixed shapes)
        for i in range(0, 40, 4):
            lg, _ = e.step([a] + [b] * 4, [toks[i // 4]] + toks[i:i + 4], [i // 4] + list(range(i, i + 4)),
                           logits=True, argmax=False)
            out.append(lg.copy())
        # a: batch-1 decode to position 300 (graph replays within each bucket)
        for p in range(10, 300):
            lg, _ = e.step([a], [toks[p]], [p], logits=True, argmax=False)
            if p % 7 == 0 or p in (255, 256, 257):
                out.append(lg.copy())
        runs.append(out)
        e.close()
    assert len(runs[0]) == len(runs[1])
    for k, (g, x) in enumerate(zip(*runs)):
        assert np.array_equal(g.view(np.uint32), x.view(np.uint32)), f"{name}: step {k} differs"


def test_page_exhaustion_is_clean(hip):
    from qraf_amd.engine import Engine
    kw, seed = SMALL["q8_llama"]
    m = oracle_model(kw, seed)
    e = Engine(engine_config(kw), kv_dtype=po.F32, max_batch=4, num_pages=3, page_size=16)
    for name, dt, shape, data in m.tensors():
        e.set_tensor(name, dt, shape, data)
    e.finalize()
    s = e.seq_create()
    e.step([s] * 4, [1, 2, 3, 4], [0, 1, 2, 3])
    free = e.free_pages()
    t = e.seq_create()
    with pytest.raises(hip.HipError) as err:
        e.step([t, t, t, t], [1, 2, 3, 4], [0, 16, 32, 48])  # gaps are refused before any allocation
    assert err.value.code == -1
    for p in range(4, 64, 4):
        try:
            e.step([s] * 4, [5] * 4, [p, p + 1, p + 2, p + 3])
        except hip.HipError as x:
            assert x.code == -4  # KV page pool exhausted
            break
    else:
        raise AssertionError("pool never ran out")
    assert e.free_pages() == 0 and e.seq_length(s) == p  # the failed step changed nothing
    e.seq_release(s)
    assert e.free_pages() == 3
    e.close()


def test_smollm2_135m_architecture_q8_streams(hip):
    """SmolLM2-135M architecture (30 layers, hidden 576, 9/3 heads, FFN 1536,
    vocab 49152, theta 1e5), Q8 weights: logits and the first 32 greedy tokens
    of a seeded prompt against the oracle."""
    from qraf_amd.engine import InferenceEngine
    kw = dict(vocab=49152, hidden=576, layers=30, heads=9, kv_heads=3, inter=1536, max_seq=2048, rope_theta=1e5,
              eps=1e-5, wdtype=po.Q8_0)
    seed = 1
    m = oracle_model(kw, seed)
    tf = upload(m, kw)
    prompt = [po.lib().or_gen_token(seed, i, kw["vocab"]) for i in range(8)]
    m.reset()
    tf.reset()
    for i, t in enumerate(prompt):
        ref = m.forward(t, i)
        check_logits(tf.forward(t, i), ref, f"pos {i}")
    want = m.generate(prompt, 32, 1.0, eos=-1)
    got = InferenceEngine(tf, eos_token=None).generate_tokens(prompt, 32, repetition_penalty=1.0)
    assert got == want
    tf.engine.close()


def c1_prompt(vocab=49152):
    """The benchmark's batch-1 workload prompt: 32 tokens uniform over the
    vocabulary from numpy's default generator seeded with 1 (bench.py draws
    the same)."""
    return np.random.default_rng(1).integers(0, vocab, 32).tolist()


def test_smollm2_135m_c1_workload(hip):
    """The batch-1 benchmark workload exactly: SmolLM2-135M architecture, Q8_0
    weights of seed 1, the benchmark's 32-token prompt fed token by token, then
    128 greedy tokens.  Every logit vector of the prompt and of the first 32
    generated tokens within 1e-3 relative / 1e-4 absolute of the oracle's,
    those 32 tokens identical; the whole 128-token stream equal to the
    oracle's, or (were float ordering ever to flip a near-tie) first differing
    past token 32 at a position where the oracle's own top-2 gap is under
    1e-3 of its top logit."""
    from qraf_amd.engine import InferenceEngine
    kw = dict(vocab=49152, hidden=576, layers=30, heads=9, kv_heads=3, inter=1536, max_seq=2048, rope_theta=1e5,
              eps=1e-5, wdtype=po.Q8_0)
    m = oracle_model(kw, 1)
    tf = upload(m, kw)
    prompt = c1_prompt(kw["vocab"])
    print("C1 workload: 32-token prompt, 128 greedy tokens", flush=True)
    m.reset()
    tf.reset()
    toks = []
    ref = None
    for i, t in enumerate(prompt):
        ref = m.forward(t, i)
        check_logits(tf.forward(t, i), ref, f"prompt pos {i}")
    for j in range(32):  # the first 32 generated tokens, each from logits checked against the oracle's
        nxt = int(np.argmax(ref))
        toks.append(nxt)
        ref = m.forward(nxt, len(prompt) + j)
        check_logits(tf.forward(nxt, len(prompt) + j), ref, f"generated token {j}")
    want = m.generate(prompt, 128, 1.0, eos=-1)
    assert want[:32] == toks
    got = InferenceEngine(tf, eos_token=None).generate_tokens(prompt, 128, repetition_penalty=1.0)
    assert len(got) == 128 and got[:32] == want[:32]
    if got != want:
        d = next(i for i in range(128) if got[i] != want[i])
        m.reset()
        for i, t in enumerate(prompt + want[:d]):
            lg = m.forward(t, i)
        assert d >= 32 and gap(lg) <= 1e-3 * float(np.abs(lg).max()), f"streams differ at {d}, gap {gap(lg):.3e}"
    tf.engine.close()


def test_greedy_only_head_same_streams(hip):
    """keep_logits off (qraf_engine_set_keep_logits): greedy-only steps take
    the head's argmax in its GEMM's epilogue and write no logits.  With 96
    requests decoding together the head runs at 96-112 logit rows on a 16385-row
    vocabulary (the pipelined form, fused), at fewer rows as requests finish
    (not fused); every stream equals the run that keeps its logits, pipelined
    and not, and a greedy-only step refuses sample / read_logits."""
    from qraf_amd._lib import F32, HipError, Q4_0
    from qraf_amd.engine import BatchScheduler, Engine, SamplingParams, model_config
    cfg = model_config(16385, 256, 2, 4, 2, 512, 256, 1e6, 1e-6)
    e = Engine(cfg, kv_dtype=F32, max_batch=128)
    try:
        e.generate_weights(Q4_0, Q4_0, Q4_0, True, True, 77)
        e.finalize()
        rng = np.random.default_rng(5)
        work = [([int(t) for t in rng.integers(0, 16385, 4 + r % 5)], 6 + r % 7) for r in range(96)]
        runs = {}
        for keep in (True, False):
            for pipeline in (False, True):
                sched = BatchScheduler(e, max_batch=96, max_rows=128, prefill_chunk=8, pipeline=pipeline,
                                       keep_logits=keep)
                ids = [sched.submit(p, o) for p, o in work]
                done = {r.id: r for r in sched.run()}
                runs[keep, pipeline] = [done[i].generated for i in ids]
        want = runs[True, False]
        assert all(len(g) == o for g, (_, o) in zip(want, work))
        for k, v in runs.items():
            assert v == want, f"keep_logits={k[0]} pipeline={k[1]}: streams differ"
        # a greedy-only step (80 logit rows) keeps no logits
        seqs = [e.seq_create() for _ in range(80)]
        e.set_keep_logits(False)
        _, nx = e.step(seqs, [3] * 80, [0] * 80, logits=False, argmax=True)
        with pytest.raises(HipError):
            e.read_logits(0)
        with pytest.raises(HipError):
            e.sample(SamplingParams(0.0, 0, 1.0, 1.0), row0=0, rows=1)
        # the same step with logits kept: the same tokens, and its logits readable
        e.set_keep_logits(True)
        seqs2 = [e.seq_create() for _ in range(80)]
        lg, nx2 = e.step(seqs2, [3] * 80, [0] * 80, logits=True, argmax=True)
        assert np.array_equal(nx, nx2)
        assert np.array_equal(nx2, np.argmax(lg, axis=1).astype(np.uint32))
        e.read_logits(0)
        for s in seqs + seqs2:
            e.seq_release(s)
    finally:
        e.close()


@pytest.mark.parametrize("bs,dt", [(8, po.Q8_0), (16, po.Q4_0), (4, po.Q4_0)])
def test_quant_block_sizes(hip, bs, dt):
    """Models quantized in blocks of 4, 8 or 16 (the reference reads the block
    size from the file's quant scheme, backend.cpp:135 and quantize.cpp:105-183):
    every projection on the matvec (the batched GEMM's tiles are 32 wide), the
    embedding dequantized at that size.  One sequence decoded position by
    position: logits within the bar of the oracle's model of the same block
    size; three requests through the scheduler (steps of several rows, one
    matvec per row): each stream equal to its independent greedy decode; a
    tensor of another block size, or a size the engine does not take, refused."""
    from qraf_amd._lib import HipError
    from qraf_amd.engine import BatchScheduler, Engine
    kw = dict(vocab=300, hidden=128, layers=2, heads=4, kv_heads=2, inter=192, max_seq=64, rope_theta=1e5, eps=1e-5,
              wdtype=dt, tied=(dt == po.Q4_0))
    m = po.Model(po.make_config(**kw, block_size=bs), 40 + bs)
    e = Engine(engine_config(kw), kv_dtype=po.F32, max_batch=8)
    try:
        tensors = m.tensors()
        for name, tdt, shape, data in tensors:
            e.set_tensor(name, tdt, shape, data, block_size=bs)
        # another block size, or one the engine does not take: refused
        name, tdt, shape, data = next(t for t in tensors if t[0].endswith("mlp.down_proj.weight"))
        for bad in (32 if bs != 32 else 8, 12):
            with pytest.raises(HipError) as x:
                e.set_tensor(name, tdt, shape, data, block_size=bad)
            assert x.value.code == -2  # QRAF_HIP_ERR_DTYPE
        e.finalize()
        s = e.seq_create()
        prompt = [5, 299, 0, 42, 42, 7]
        for pos, tok in enumerate(prompt):
            lg, _ = e.step([s], [tok], [pos], logits=True, argmax=False)
            check_logits(lg[0], m.forward(tok, pos).astype(np.float64), f"block size {bs}, position {pos}")
        e.seq_release(s)
        L = po.lib()
        prompts = [[L.or_gen_token(700 + r, i, kw["vocab"]) for i in range(3 + 2 * r)] for r in range(3)]
        sched = BatchScheduler(e, max_batch=3, max_rows=8, prefill_chunk=4)
        ids = [sched.submit(p, 6) for p in prompts]
        done = {r.id: r for r in sched.run()}
        for i, p in zip(ids, prompts):
            assert done[i].generated == m.generate(p, 6, 1.0, eos=-1), f"block size {bs}"
    finally:
        e.close()
        m.close()



@pytest.mark.parametrize("graphs", [True, False])
def test_long_context_batch1_decode(hip, graphs):
    """One sequence decoded token by token to 1,100 positions (f32 pages,
    Q8 weights, head_dim 64, 2 KV heads): one-row steps whose attention
    leaves the single-chunk kernel at 256 positions for the chunked form and
    its merge, with step graphs captured at each context bound (256, 512,
    1,024, 2,048) or every step eager.  Logits at every position within the
    1e-3 / 1e-4 bar of the oracle's forward on the same tokens."""
    from qraf_amd.engine import Engine
    kw = dict(vocab=500, hidden=256, layers=2, heads=4, kv_heads=2, inter=512, max_seq=2048, rope_theta=1e4,
              eps=1e-5, wdtype=po.Q8_0)
    m = oracle_model(kw, 61)
    e = Engine(engine_config(kw), kv_dtype=po.F32, max_batch=1)
    try:
        for name, dt, shape, data in m.tensors():
            e.set_tensor(name, dt, shape, data)
        e.finalize()
        e.set_graphs(graphs)
        L = po.lib()
        s = e.seq_create()
        m.reset()
        print(f"long context decode, graphs {graphs}", flush=True)
        for pos in range(1100):
            tok = L.or_gen_token(61, pos, kw["vocab"])
            lg, _ = e.step([s], [tok], [pos], logits=True, argmax=False)
            check_logits(lg[0], m.forward(tok, pos), f"pos {pos}")
        assert e.seq_length(s) == 1100
    finally:
        e.close()
        m.close()


def test_two_engines_in_two_threads(hip):
    """Two engines (different models, each with its own stream, pages and
    step graphs) decoding at the same time from two host threads (ctypes
    releases the interpreter lock in every library call): each thread's
    greedy stream and final logits equal the same engine's run alone."""
    import threading
    from qraf_amd.engine import InferenceEngine
    names = ["q8_hd64_gqa3", "q4_gqa8_hd128"]
    models = {n: oracle_model(*SMALL[n]) for n in names}
    prompts = {n: [po.lib().or_gen_token(SMALL[n][1] + 3, i, SMALL[n][0]["vocab"]) for i in range(10)] for n in names}

    def run(n, out):
        tf = upload(models[n], SMALL[n][0])
        try:
            toks = InferenceEngine(tf, eos_token=None).generate_tokens(prompts[n], 48, repetition_penalty=1.0)
            tf.reset()
            lg = None
            for i, t in enumerate(prompts[n] + toks[:16]):
                lg = tf.forward(t, i)
            out[n] = (toks, lg.copy())
        finally:
            tf.engine.close()

    alone = {}
    for n in names:
        run(n, alone)
    together = {}
    threads = [threading.Thread(target=run, args=(n, together)) for n in names]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=120)
    for n in names:
        assert n in together, f"{n}: thread did not finish"
        assert together[n][0] == alone[n][0], n
        assert np.array_equal(together[n][1].view(np.uint32), alone[n][1].view(np.uint32)), n
    for m in models.values():
        m.close()


def test_1024_row_prefill_step(hip):
    """The engine's largest step: four 256-token prompts as one 1,024-row step
    (the gate/up GEMM with the SiLU-gate epilogue, every projection at 1,024
    rows), then eight 4-row decode steps.  Each sequence's last prompt row's
    logits within the 1e-3 / 1e-4 bar of the oracle's forward of that prompt
    alone, and its nine greedy tokens equal to the oracle's decode of it."""
    from qraf_amd.engine import Engine
    kw, seed = SMALL["q4_gqa8_hd128"]
    kw = dict(kw, max_seq=512)
    m = oracle_model(kw, seed)
    e = Engine(engine_config(kw), kv_dtype=po.F32, max_batch=1024)
    try:
        for name, dt, shape, data in m.tensors():
            e.set_tensor(name, dt, shape, data)
        e.finalize()
        L = po.lib()
        prompts = [[L.or_gen_token(seed + 50 + r, i, kw["vocab"]) for i in range(256)] for r in range(4)]
        sids = [e.seq_create() for _ in range(4)]
        rows_s, rows_t, rows_p, want = [], [], [], []
        for s, p in zip(sids, prompts):
            rows_s += [s] * 256
            rows_t += p
            rows_p += list(range(256))
            want += [0] * 255 + [1]
        lg, nx = e.step(rows_s, rows_t, rows_p, want_logits=want, logits=True, argmax=True)
        refs = []
        for r, p in enumerate(prompts):
            m.reset()
            for i, t in enumerate(p):
                ref = m.forward(t, i)
            check_logits(lg[r], ref, f"sequence {r} prompt end")
            assert int(nx[r]) == int(np.argmax(ref)), f"sequence {r} first token"
            refs.append(m.generate(p, 9, 1.0, eos=-1))
        toks = [int(t) for t in nx]
        streams = [[t] for t in toks]
        for k in range(8):
            lg, nx = e.step(sids, toks, [256 + k] * 4, logits=True, argmax=True)
            toks = [int(t) for t in nx]
            for r in range(4):
                streams[r].append(toks[r])
        for r in range(4):
            assert streams[r] == refs[r], f"sequence {r}"
    finally:
        e.close()
        m.close()


@pytest.mark.parametrize("name,penalty", [("q8_hd64_gqa3", 1.1), ("q4_gqa8_hd128", 1.3), ("q4_hd64_gqa2", 0.9),
                                          ("q4_qwen2_tied_bias", 1.1)])
def test_penalised_greedy_on_device(hip, name, penalty):
    """Greedy decoding with a repetition penalty, pipelined with the penalty
    applied on the device from counts of the fed tokens
    (qraf_engine_set_repetition_penalty), against the unpipelined loop that
    penalises on the host-built recent list (qraf_engine_sample) and against
    the oracle's generate: the same tokens, for prompts that repeat tokens
    (counts above 1), with a stop token met and without; the engine's
    penalty slots all returned."""
    from qraf_amd.engine import InferenceEngine
    kw, seed = SMALL[name]
    m = oracle_model(kw, seed)
    tf = upload(m, kw)
    try:
        L = po.lib()
        base = [L.or_gen_token(seed + 17, i, kw["vocab"]) for i in range(9)]
        prompts = [base, base[:3] * 4, [base[0]] * 6 + base]
        for p in prompts:
            want = m.generate(p, 40, penalty, eos=-1)
            got = InferenceEngine(tf, eos_token=None).generate_tokens(p, 40, repetition_penalty=penalty)
            host = InferenceEngine(tf, eos_token=None).generate_tokens(p, 40, repetition_penalty=penalty,
                                                                      pipeline=False)
            assert got == host == want, name
            # a stop token met part-way: the stream up to it, the same either way
            stop = want[len(want) // 2]
            got_s = InferenceEngine(tf, eos_token=stop).generate_tokens(p, 40, repetition_penalty=penalty)
            host_s = InferenceEngine(tf, eos_token=stop).generate_tokens(p, 40, repetition_penalty=penalty,
                                                                        pipeline=False)
            assert got_s == host_s == want[:want.index(stop)], name
    finally:
        tf.engine.close()
        m.close()


def test_device_penalty_refusals(hip):
    """qraf_engine_set_repetition_penalty: refused for a sequence that already
    holds positions, an unknown sequence, a penalty that is not positive and
    finite; more penalised sequences than 2 * max_batch run out of slots, and
    a released sequence's slot is reused."""
    from qraf_amd._lib import HipError
    from qraf_amd.engine import Engine
    kw, seed = SMALL["q8_llama"]
    m = oracle_model(kw, seed)
    e = Engine(engine_config(kw), kv_dtype=po.F32, max_batch=1)
    try:
        for tname, dt, shape, data in m.tensors():
            e.set_tensor(tname, dt, shape, data)
        e.finalize()
        a, b, c = e.seq_create(), e.seq_create(), e.seq_create()
        e.step([a], [5], [0])
        with pytest.raises(HipError) as x:
            e.set_repetition_penalty(a, 1.1)
        assert x.value.code == -5  # QRAF_HIP_ERR_STATE
        for bad in (0.0, -1.0, float("inf"), float("nan")):
            with pytest.raises(HipError):
                e.set_repetition_penalty(b, bad)
        with pytest.raises(HipError):
            e.set_repetition_penalty(999, 1.1)
        e.set_repetition_penalty(b, 1.1)
        e.set_repetition_penalty(c, 1.2)
        d = e.seq_create()
        with pytest.raises(HipError) as x:
            e.set_repetition_penalty(d, 1.1)
        assert x.value.code == -4  # QRAF_HIP_ERR_NOMEM: both slots (2 * max_batch) in use
        e.seq_release(b)
        e.set_repetition_penalty(d, 1.1)  # b's slot
        e.set_repetition_penalty(c, 1.0)  # off: its slot back
        e.set_repetition_penalty(e.seq_create(), 1.5)
    finally:
        e.close()
        m.close()


def test_scheduler_penalties_on_device(hip):
    """Requests with repetition penalties 1.0, 1.1 and 1.3 side by side through
    the scheduler, with chunked prefill and admission as others finish: with
    the penalty on the device (pipelined and not) and on the host-built recent
    lists (unpipelined), every request's stream equals the oracle's decode of
    it alone with its penalty, with an EOS token and without."""
    from qraf_amd.engine import BatchScheduler, Engine
    kw, seed = SMALL["q4_gqa8_hd128"]
    m = oracle_model(kw, seed)
    L = po.lib()
    prompts = [[L.or_gen_token(300 + r, i, kw["vocab"]) for i in range(3 + 4 * r)] * (1 + r % 2) for r in range(7)]
    pens = [1.0, 1.1, 1.3, 1.1, 1.0, 1.3, 1.1]
    want = {None: [m.generate(p, 20, pen, eos=-1) for p, pen in zip(prompts, pens)]}
    eos = want[None][1][5]
    want[eos] = [m.generate(p, 20, pen, eos=eos) for p, pen in zip(prompts, pens)]
    e = Engine(engine_config(kw), kv_dtype=po.F32, max_batch=16)
    try:
        for name, dt, shape, data in m.tensors():
            e.set_tensor(name, dt, shape, data)
        e.finalize()
        pool = e.free_pages()
        for stop in (None, eos):
            for device_penalty, pipeline in ((True, True), (True, False), (False, False)):
                sched = BatchScheduler(e, max_batch=4, max_rows=16, prefill_chunk=5, pipeline=pipeline,
                                       device_penalty=device_penalty)
                ids = [sched.submit(p, 20, repetition_penalty=pen, eos=stop) for p, pen in zip(prompts, pens)]
                done = {r.id: r for r in sched.run()}
                got = [done[i].generated for i in ids]
                assert got == want[stop], (stop, device_penalty, pipeline)
                assert e.free_pages() == pool
    finally:
        e.close()
        m.close()
