"""Host-side mirror of the reference's engine API over the HIP C ABI.

    Transformer      Transformer::init / forward / reset (transformer.h:55-90)
    InferenceEngine  InferenceEngine::generate_tokens (inference.cpp:68-159), greedy
    BatchScheduler   the continuous-batching contract of batch_scheduler.h:54-283:
                     requests queue, are admitted into max_batch slots as others
                     finish, and retire on EOS or max_tokens; every active
                     request advances one token per step, all in one batched
                     device step

    SamplingConfig   SamplingConfig (sampler.h:10-17)
    Sampler          a Sampler's draw stream: std::mt19937 seeded as
                     Sampler::Sampler (sampler.cpp:9-16) and libstdc++'s
                     uniform_real_distribution<float>(0, 1)

Sampling runs on the device (qraf_engine_sample): the repetition penalty
(sampler.cpp:37-49), then greedy argmax (:25-35) or temperature / top-k /
top-p sampling (:57-128) on the step's logits where they lie in HBM; only
token ids (and the uniform of each sampled row) cross PCIe.
"""
from __future__ import annotations

import ctypes as C
import os
import random
import time
from collections import deque
from dataclasses import dataclass, field

import numpy as np

from ._lib import (F16, F32, Q4_0, Q8_0, EngineOptions, EngineStats, ModelConfig, SamplingParams, call, fp, i32p, lib,
                   u32p)

__all__ = ["Engine", "Transformer", "InferenceEngine", "BatchScheduler", "Request", "model_config",
           "read_file_config", "SamplingConfig", "Sampler"]


def model_config(vocab, hidden, layers, heads, kv_heads, inter, max_seq=2048, rope_theta=1e4, eps=1e-5):
    return ModelConfig(vocab, hidden, layers, heads, kv_heads, inter, max_seq, rope_theta, eps)


def read_file_config(path: str) -> ModelConfig:
    """The model config stored in a .qraf file (QrafModel::parse_config,
    loader.cpp:133-177); host only."""
    cfg = ModelConfig()
    call("qraf_file_read_config", os.fsencode(path), C.byref(cfg), None)
    return cfg


@dataclass
class SamplingConfig:
    """SamplingConfig (sampler.h:10-17), with the reference's defaults."""
    temperature: float = 0.8
    top_k: int = 40
    top_p: float = 0.9
    repetition_penalty: float = 1.1
    seed: int = 0  # 0: a random seed
    deterministic: bool = False

    @property
    def greedy(self) -> bool:
        return self.deterministic or self.temperature <= 0.0  # sampler.cpp:59-61

    def params(self) -> SamplingParams:
        return SamplingParams(0.0 if self.greedy else self.temperature, self.top_k, self.top_p,
                              self.repetition_penalty)


def _mt19937_state(seed: int):
    """std::mt19937::seed(seed): the 624-word state before the first twist."""
    mt = [seed & 0xFFFFFFFF]
    for i in range(1, 624):
        mt.append((1812433253 * (mt[-1] ^ (mt[-1] >> 30)) + i) & 0xFFFFFFFF)
    return mt


class Sampler:
    """The draw stream of the reference's Sampler (sampler.cpp:9-16): a
    std::mt19937 seeded with the config's seed (truncated to unsigned; 0 ->
    random_device), read through uniform_real_distribution<float>(0, 1) as
    libstdc++ computes it: float(x) / 2^32, 1.0 replaced by the largest float
    below it.  Python's Mersenne Twister core is the same generator, so the
    state is installed directly.  One draw per sampled (non-greedy) token, as
    Sampler::sample makes."""

    def __init__(self, config: SamplingConfig):
        self.config = config
        seed = config.seed if config.seed != 0 else int.from_bytes(os.urandom(4), "little")
        self._rng = random.Random()
        self._rng.setstate((3, tuple(_mt19937_state(seed & 0xFFFFFFFF)) + (624,), None))

    def uniform(self) -> float:
        r = np.float32(self._rng.getrandbits(32)) / np.float32(4294967296.0)
        if r >= np.float32(1.0):
            r = np.nextafter(np.float32(1.0), np.float32(0.0))
        return float(r)

    def uniforms(self, n: int) -> np.ndarray:
        return np.array([self.uniform() for _ in range(n)], np.float32)


class Engine:
    """qraf_engine: device-resident weights, paged KV cache, batched steps."""

    def __init__(self, config: ModelConfig, kv_dtype=F32, page_size=16, max_batch=1, num_pages=0):
        self.config = config
        self.max_batch = max_batch
        opt = EngineOptions(kv_dtype, page_size, max_batch, num_pages)
        h = C.c_void_p()
        call("qraf_engine_create", C.byref(config), C.byref(opt), C.byref(h))
        self.h = h.value
        self.vocab = config.vocab_size

    @classmethod
    def from_file(cls, path: str, kv_dtype=F32, page_size=16, max_batch=1, num_pages=0) -> "Engine":
        """QrafModel::load + Transformer::init in one call: a .qraf file's
        config and tensors straight into HBM (qraf_engine_create_from_file)."""
        cfg = read_file_config(path)
        self = cls.__new__(cls)
        self.config = cfg
        self.max_batch = max_batch
        opt = EngineOptions(kv_dtype, page_size, max_batch, num_pages)
        h = C.c_void_p()
        call("qraf_engine_create_from_file", os.fsencode(path), C.byref(opt), C.byref(h))
        self.h = h.value
        self.vocab = cfg.vocab_size
        return self

    def close(self):
        if getattr(self, "h", None):
            lib.qraf_engine_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_tensor(self, name: str, dtype: int, shape, data: np.ndarray, block_size: int = 32):
        data = np.ascontiguousarray(data)
        sh = np.ascontiguousarray(shape, dtype=np.uint32)
        call("qraf_engine_set_tensor", self.h, name.encode(), dtype, block_size, sh.ctypes.data_as(u32p), sh.size,
             data.ctypes.data, data.nbytes)

    def generate_weights(self, weight_dtype, embed_dtype, head_dtype, tied, qkv_bias, seed):
        call("qraf_engine_generate_weights", self.h, weight_dtype, embed_dtype, head_dtype, int(tied), int(qkv_bias),
             seed)

    def finalize(self):
        call("qraf_engine_finalize", self.h)

    def set_graphs(self, on: bool):
        """Replay captured step graphs (default) or launch every step eagerly."""
        call("qraf_engine_set_graphs", self.h, int(bool(on)))

    def set_keep_logits(self, keep: bool):
        """False: steps that want only greedy tokens (step(..., logits=False),
        step_async) take the head's argmax inside its GEMM and write no logits
        (sample() and read_logits() then fail for such a step); True (default):
        every step leaves its logits in HBM."""
        call("qraf_engine_set_keep_logits", self.h, int(bool(keep)))

    def seq_create(self) -> int:
        i = C.c_int32()
        call("qraf_engine_seq_create", self.h, C.byref(i))
        return i.value

    def seq_release(self, seq_id: int):
        call("qraf_engine_seq_release", self.h, seq_id)

    def set_repetition_penalty(self, seq_id: int, penalty: float):
        """Greedy tokens of this sequence (set before its first step) taken
        after Sampler::apply_repetition_penalty with every token it was fed,
        counted on the device (qraf_engine_set_repetition_penalty)."""
        call("qraf_engine_set_repetition_penalty", self.h, seq_id, C.c_float(penalty))

    def seq_length(self, seq_id: int) -> int:
        i = C.c_int32()
        call("qraf_engine_seq_length", self.h, seq_id, C.byref(i))
        return i.value

    def free_pages(self) -> int:
        i = C.c_int32()
        call("qraf_engine_free_pages", self.h, C.byref(i))
        return i.value

    def step(self, seq_ids, tokens, positions, want_logits=None, logits=False, argmax=True):
        """One batched step.  Returns (logits [k][vocab] or None, next tokens [k] or None)
        for the k rows that want logits (all rows by default)."""
        sid = np.ascontiguousarray(seq_ids, dtype=np.int32)
        tok = np.ascontiguousarray(tokens, dtype=np.uint32)
        pos = np.ascontiguousarray(positions, dtype=np.int32)
        n = sid.size
        if want_logits is None:
            k, wl = n, None
        else:
            wl = np.ascontiguousarray(want_logits, dtype=np.uint8)
            k = int(np.count_nonzero(wl))
        lg = np.empty((k, self.vocab), np.float32) if logits else None
        nx = np.empty(k, np.uint32) if argmax else None
        call("qraf_engine_step", self.h, n, sid.ctypes.data_as(i32p), tok.ctypes.data_as(u32p),
             pos.ctypes.data_as(i32p), wl.ctypes.data_as(C.POINTER(C.c_uint8)) if wl is not None else None,
             lg.ctypes.data_as(fp) if lg is not None else None, nx.ctypes.data_as(u32p) if nx is not None else None)
        return lg, nx

    def step_async(self, seq_ids, tokens, positions, want_logits=None, token_src=None):
        """Issue one greedy step without waiting for it (at most two in
        flight).  token_src[i] >= 0: row i feeds the greedy token of logit
        row token_src[i] of the step issued just before, taken on the device
        (tokens[i] is then ignored).  collect() returns the steps' tokens in
        issue order."""
        sid = np.ascontiguousarray(seq_ids, dtype=np.int32)
        tok = np.ascontiguousarray(tokens, dtype=np.uint32)
        pos = np.ascontiguousarray(positions, dtype=np.int32)
        src = None if token_src is None else np.ascontiguousarray(token_src, dtype=np.int32)
        wl = None if want_logits is None else np.ascontiguousarray(want_logits, dtype=np.uint8)
        call("qraf_engine_step_async", self.h, sid.size, sid.ctypes.data_as(i32p), tok.ctypes.data_as(u32p),
             src.ctypes.data_as(i32p) if src is not None else None, pos.ctypes.data_as(i32p),
             wl.ctypes.data_as(C.POINTER(C.c_uint8)) if wl is not None else None)

    def collect(self) -> np.ndarray:
        """Wait for the oldest step in flight; its greedy tokens [k]."""
        out = np.empty(self.max_batch, np.uint32)
        k = C.c_int32()
        call("qraf_engine_step_collect", self.h, out.ctypes.data_as(u32p), C.byref(k))
        return out[:k.value]

    def read_logits(self, row0: int, rows: int = 1) -> np.ndarray:
        """Logit rows row0 .. row0+rows-1 of the last step (in the order of the
        rows that wanted logits), read back from HBM."""
        out = np.empty((rows, self.vocab), np.float32)
        call("qraf_engine_read_logits", self.h, row0, rows, out.ctypes.data_as(fp))
        return out

    def stats(self, reset: bool = False) -> dict:
        """Host-side time of the steps so far: host_us until every launch was
        issued, wait_us blocked on the device at the step's end; and how the
        steps ran (eager, captured, graph launches; pad rows)."""
        st = EngineStats()
        call("qraf_engine_get_stats", self.h, C.byref(st), int(bool(reset)))
        return {k: getattr(st, k) for k, _ in EngineStats._fields_}

    def set_fusion(self, flags: int) -> None:
        """Bit 0: one-row steps fuse the QKV bias, RoPE and K/V store into the
        QKV matvec (default on; bit-identical either way).  Bit 1: steps of
        more than 256 rows run the gate/up GEMM with the SiLU-gate in its
        epilogue (default on; the same sums in another order).  Bit 2: steps
        of 2-8 rows run their projections on the multi-vector matvec where
        it covers them (default on; batch-1 arithmetic instead of the GEMM's)."""
        call("qraf_engine_set_fusion", self.h, int(flags))

    def set_row_padding(self, rows: int) -> None:
        """Steps of more than 8 rows run padded to a multiple of `rows` (with
        step graphs on), so nearby step sizes share a graph; 1 turns it off."""
        call("qraf_engine_set_row_padding", self.h, int(rows))

    def sample(self, params: SamplingParams, recent=None, uniforms=None, row0=0, rows=None) -> np.ndarray:
        """Sampler::apply_repetition_penalty + Sampler::sample on rows row0.. of
        the last step's logit rows, on the device.  recent: one token list per
        row (the penalty's history); uniforms: one draw per row when sampling."""
        n = rows if rows is not None else (len(recent) if recent is not None else len(uniforms))
        rec = cnt = None
        stride = 0
        if recent is not None and params.repetition_penalty != 1.0:
            stride = max(1, max(len(r) for r in recent))
            rec = np.zeros((n, stride), np.uint32)
            cnt = np.zeros(n, np.int32)
            for i, r in enumerate(recent):
                rec[i, :len(r)] = r
                cnt[i] = len(r)
        uni = None if uniforms is None else np.ascontiguousarray(uniforms, dtype=np.float32)
        out = np.empty(n, np.uint32)
        call("qraf_engine_sample", self.h, row0, n, C.byref(params),
             rec.ctypes.data_as(u32p) if rec is not None else None,
             cnt.ctypes.data_as(i32p) if cnt is not None else None, stride,
             uni.ctypes.data_as(fp) if uni is not None else None, out.ctypes.data_as(u32p))
        return out


class Transformer:
    """Transformer::init / forward / reset (transformer.h:55-90) on the GPU."""

    def __init__(self, engine: Engine):
        self.engine = engine
        self._logits = np.empty(engine.vocab, np.float32)

    @classmethod
    def from_tensors(cls, config: ModelConfig, tensors, kv_dtype=F32, max_batch=1, num_pages=0, page_size=16):
        """tensors: iterable of (name, dtype, shape, bytes ndarray) as a QRAF
        model exposes them (TensorView, loader.h:12-27)."""
        e = Engine(config, kv_dtype=kv_dtype, max_batch=max_batch, num_pages=num_pages, page_size=page_size)
        for name, dt, shape, data in tensors:
            e.set_tensor(name, dt, shape, data)
        e.finalize()
        return cls(e)

    @classmethod
    def from_file(cls, path: str, kv_dtype=F32, max_batch=1, num_pages=0, page_size=16):
        """A .qraf file (QrafModel::load + Transformer::init) straight into HBM."""
        return cls(Engine.from_file(path, kv_dtype=kv_dtype, page_size=page_size, max_batch=max_batch,
                                    num_pages=num_pages))

    @classmethod
    def synthetic(cls, config: ModelConfig, weight_dtype, seed, embed_dtype=None, head_dtype=None, tied=False,
                  qkv_bias=False, kv_dtype=F32, max_batch=1, num_pages=0, page_size=16):
        e = Engine(config, kv_dtype=kv_dtype, max_batch=max_batch, num_pages=num_pages, page_size=page_size)
        e.generate_weights(weight_dtype, weight_dtype if embed_dtype is None else embed_dtype,
                           weight_dtype if head_dtype is None else head_dtype, tied, qkv_bias, seed)
        e.finalize()
        return cls(e)

    def forward(self, token: int, pos: int) -> np.ndarray:
        out = np.empty(self.engine.vocab, np.float32)
        call("qraf_engine_forward", self.engine.h, int(token), int(pos), out.ctypes.data_as(fp))
        return out

    def reset(self):
        call("qraf_engine_reset", self.engine.h)


def apply_repetition_penalty(logits: np.ndarray, recent, penalty: float):
    """Sampler::apply_repetition_penalty (sampler.cpp:37-49), once per occurrence."""
    if penalty == 1.0:
        return
    p = np.float32(penalty)
    n = logits.shape[0]
    for t in recent:
        if t >= n:
            continue
        v = logits[t]
        logits[t] = v / p if v > 0 else v * p


def argmax(logits: np.ndarray) -> int:
    """Sampler::argmax: numpy's argmax also returns the lowest index of the max."""
    return int(np.argmax(logits))


class InferenceEngine:
    """InferenceEngine::generate_tokens (inference.cpp:68-159)."""

    def __init__(self, transformer: Transformer, eos_token: int | None = 2):
        self.transformer = transformer
        self.eos = eos_token  # tokenizer.h:62 default when the file has no tokenizer

    def generate_tokens(self, prompt_tokens, max_tokens=256, repetition_penalty=1.1, stop_tokens=(),
                        sampling: SamplingConfig | None = None, pipeline: bool = True):
        """Greedy with `repetition_penalty` unless a SamplingConfig is given.
        The prompt is fed token by token (inference.cpp:90-99); then every
        token is the device sampler's pick from the last logits, penalised
        with the prompt and every generated token so far (inference.cpp:104-
        116), and is fed back until a stop token or max_tokens.  Greedy with
        a penalty (and pipeline, vocabularies a multiple of 4) runs
        pipelined: the penalty is applied on the device from counts of the
        tokens fed (qraf_engine_set_repetition_penalty) and each step takes
        its token from the previous step's argmax on the device, a stop token
        being seen one step late; the same tokens."""
        if len(prompt_tokens) == 0:
            raise ValueError("empty prompt")
        if sampling is None:
            sampling = SamplingConfig(temperature=0.0, top_k=0, top_p=1.0, repetition_penalty=repetition_penalty,
                                      deterministic=True)
        sampler = Sampler(sampling) if not sampling.greedy else None
        params = sampling.params()
        e = self.transformer.engine
        stops = set(stop_tokens) | ({self.eos} if self.eos is not None else set())
        self.transformer.reset()  # frees the default sequence's pages
        seq = e.seq_create()
        if pipeline and sampler is None and params.repetition_penalty != 1.0 and e.vocab % 4 == 0:
            try:
                return self._penalised_greedy_pipelined(e, seq, list(prompt_tokens), max_tokens, stops,
                                                        params.repetition_penalty)
            finally:
                e.seq_release(seq)
        try:
            last = len(prompt_tokens) - 1
            for i, t in enumerate(prompt_tokens):
                e.step([seq], [t], [i], want_logits=[i == last], logits=False, argmax=i == last)
            pos = len(prompt_tokens)
            recent = list(prompt_tokens)
            out = []
            for _ in range(max_tokens):
                uni = None if sampler is None else [sampler.uniform()]
                nxt = int(e.sample(params, [recent], uni, rows=1)[0])
                if nxt in stops:
                    break
                out.append(nxt)
                recent.append(nxt)
                e.step([seq], [nxt], [pos], logits=False, argmax=True)
                pos += 1
        finally:
            e.seq_release(seq)
        return out

    @staticmethod
    def _penalised_greedy_pipelined(e, seq, prompt, max_tokens, stops, penalty):
        e.set_repetition_penalty(seq, penalty)
        for i, t in enumerate(prompt[:-1]):
            e.step([seq], [t], [i], want_logits=[0], logits=False, argmax=False)
        e.step_async([seq], [prompt[-1]], [len(prompt) - 1])  # its argmax is the first token
        pending, out = 1, []
        try:
            while len(out) < max_tokens:
                if len(out) + 1 < max_tokens:  # the next step feeds this step's token, taken on the device
                    e.step_async([seq], [0], [len(prompt) + len(out)], token_src=[0])
                    pending += 1
                tok = int(e.collect()[0])
                pending -= 1
                if tok in stops:
                    break
                out.append(tok)
        finally:
            while pending:  # a step issued past a stop token or the last token: its token is not used
                e.collect()
                pending -= 1
        return out


@dataclass
class Request:
    """BatchRequest (batch_scheduler.h:23-37)."""
    id: int
    prompt: list
    max_tokens: int
    penalty: float = 1.0
    eos: int | None = None
    generated: list = field(default_factory=list)
    state: str = "QUEUED"  # QUEUED -> PREFILLING -> DECODING -> DONE
    seq: int = -1
    next_prompt: int = 0
    admit_step: int = -1  # scheduler step at which the request took a slot
    inflight: int = 0     # pipelined runs: tokens issued and not yet collected
    lrow: int = -1        # its logit row in step lrow_step (the source of its next decode row's token)
    lrow_step: int = -1


class BatchScheduler:
    """Continuous batching over one Engine (batch_scheduler.h:54-283 contract).

    Each step admits queued requests into free slots (max_batch concurrent
    requests), then builds the step's rows within a budget of max_rows (at
    most the engine's rows per step): every DECODING request feeds its last
    generated token, then PREFILLING requests, in admission order, feed their
    next prompt tokens, up to prefill_chunk consecutive positions each, while
    the budget lasts (chunked prefill: a prompt enters the cache as a
    batched projection instead of token by token).  A request whose last
    prompt token was just fed, or that is decoding, gets its next token from
    this step's logits; it retires on EOS or after max_tokens generated
    tokens and frees its KV pages for the next admission.  Every request's
    token stream equals an independent greedy decode of its prompt (the
    reference's scheduler runs requests one at a time over one shared cache,
    batch_scheduler.h:187-228, so it offers no batched numerics to mirror).  With the
    defaults (prefill_chunk 1, max_rows = max_batch) every active request
    feeds exactly one token per step.

    Requests with a repetition penalty take it on the device (device_penalty,
    vocabularies a multiple of 4: qraf_engine_set_repetition_penalty at
    admission, counts of every token fed), so their greedy tokens come from
    the step's own argmax like the others'; otherwise each step re-samples
    their logit rows with the penalty on the host-built recent lists
    (qraf_engine_sample).

    pipeline=True (unless some request's penalty is taken on the host): run() issues
    step N+1 before it collects step N's tokens (Engine.step_async), each
    decode row taking its token from step N's argmax on the device, so the
    host builds the next step while the device runs this one.  A request
    whose last token (by max_tokens) is in flight gets no further row and its
    slot goes to the next queued request at once, as the unpipelined run
    retires it before building that step: without EOS both runs issue the
    same steps, row for row.  A request that emits EOS is found a step late:
    the row it had in the next step is dropped (its cache writes land in
    pages it then releases, which later steps, ordered after it on the
    stream, may reuse) and its slot is refilled a step later.  The observer
    sees tokens only (the logits in HBM already belong to the next step)."""

    def __init__(self, engine: Engine, max_batch: int | None = None, max_rows: int | None = None,
                 prefill_chunk: int = 1, pipeline: bool = False, keep_logits: bool = True,
                 device_penalty: bool = True):
        self.engine = engine
        self.device_penalty = device_penalty and getattr(engine, "vocab", 1) % 4 == 0
        # False: a run whose requests are all greedy without penalty keeps no
        # logits (the engine's greedy-only head); the observer then sees tokens only
        self.keep_logits = keep_logits
        self.max_batch = max_batch or engine.max_batch
        self.max_rows = min(max_rows or self.max_batch, engine.max_batch)
        if self.max_rows < self.max_batch:
            raise ValueError(f"max_rows {self.max_rows} below max_batch {self.max_batch}: "
                             "every decoding request needs its row")
        if prefill_chunk < 1:
            raise ValueError("prefill_chunk must be >= 1")
        self.prefill_chunk = prefill_chunk
        self.pipeline = pipeline
        self.pending = deque()
        self.active = []
        self.done = []
        self._next_id = 1
        self.steps = 0
        self.rows = 0
        self.host_s = 0.0    # time in step() outside the engine's calls (admission, row building, retirement)
        self.engine_s = 0.0  # time inside the engine's step and sample calls
        self.observer = None  # observer(scheduler, requests of this step's logit rows, next tokens) after each step

    def submit(self, prompt_tokens, max_tokens, repetition_penalty=1.0, eos=None) -> int:
        if len(prompt_tokens) == 0:
            raise ValueError("empty prompt")
        r = Request(self._next_id, list(prompt_tokens), max_tokens, repetition_penalty, eos)
        self._next_id += 1
        self.pending.append(r)
        return r.id

    def _new_seq(self, r):
        r.seq = self.engine.seq_create()
        if self.device_penalty and r.penalty != 1.0:
            self.engine.set_repetition_penalty(r.seq, r.penalty)

    def _host_penalty(self, r) -> bool:
        return r.penalty != 1.0 and not self.device_penalty

    def _admit(self):
        while self.pending and len(self.active) < self.max_batch:
            r = self.pending.popleft()
            self._new_seq(r)
            r.state = "PREFILLING"
            r.admit_step = self.steps
            self.active.append(r)

    def _finish(self, r):
        r.state = "DONE"
        self.engine.seq_release(r.seq)
        self.done.append(r)

    def step(self) -> bool:
        """One scheduler iteration (process_step, batch_scheduler.h:239-273)."""
        t_start = time.perf_counter()
        self._admit()
        if not self.active:
            return False
        rows = []  # (request, token, position, wants logits)
        for r in self.active:
            if r.state == "DECODING":
                pos = len(r.prompt) + len(r.generated) - 1
                rows.append((r, r.generated[-1], pos, True))
        budget = self.max_rows - len(rows)
        for r in self.active:
            if r.state != "PREFILLING" or budget <= 0:
                continue
            c = min(self.prefill_chunk, len(r.prompt) - r.next_prompt, budget)
            for i in range(r.next_prompt, r.next_prompt + c):
                rows.append((r, r.prompt[i], i, i == len(r.prompt) - 1))
            budget -= c
        want = np.array([w for (_, _, _, w) in rows], np.uint8)
        t_eng = time.perf_counter()
        lg, nx = self.engine.step([r.seq for (r, _, _, _) in rows], [t for (_, t, _, _) in rows],
                                  [p for (_, _, p, _) in rows], want_logits=want, logits=False, argmax=True)
        # rows with a repetition penalty: penalty + argmax again on the device,
        # per run of consecutive logit rows that share a penalty value
        lrows = [r for (r, _, _, w) in rows if w]
        i = 0
        while i < len(lrows):
            j = i + 1
            while j < len(lrows) and lrows[j].penalty == lrows[i].penalty:
                j += 1
            if self._host_penalty(lrows[i]):
                gp = SamplingParams(0.0, 0, 1.0, lrows[i].penalty)
                nx[i:j] = self.engine.sample(gp, [r.prompt + r.generated for r in lrows[i:j]], row0=i)
            i = j
        t_eng_end = time.perf_counter()
        self.engine_s += t_eng_end - t_eng
        if self.observer is not None:
            self.observer(self, lrows, nx)
        t_obs = time.perf_counter() - t_eng_end
        self.steps += 1
        self.rows += len(rows)
        k = 0
        retire = []
        for (r, tok, pos, w) in rows:
            if r.state == "PREFILLING":
                r.next_prompt += 1
                if r.next_prompt == len(r.prompt):
                    r.state = "DECODING"
            if not w:
                continue
            t = int(nx[k])
            k += 1
            if (r.eos is not None and t == r.eos) or len(r.generated) >= r.max_tokens:
                retire.append(r)
                continue
            r.generated.append(t)
            if len(r.generated) >= r.max_tokens:
                retire.append(r)
        for r in retire:
            self.active.remove(r)
            self._finish(r)
        self.host_s += time.perf_counter() - t_start - (t_eng_end - t_eng) - t_obs
        return True

    def run(self):
        no_penalty = not any(self._host_penalty(r) for r in list(self.pending) + self.active)
        greedy_only = not self.keep_logits and no_penalty
        if greedy_only:
            self.engine.set_keep_logits(False)
        try:
            if self.pipeline and no_penalty:
                self._run_pipelined()
            while self.step():
                pass
        finally:
            if greedy_only:
                self.engine.set_keep_logits(True)
        return self.done

    def _run_pipelined(self):
        inflight = deque()  # per issued step: the requests of its logit rows
        while True:
            lrows = self._issue()
            if lrows is not None:
                inflight.append(lrows)
                if len(inflight) < 2:
                    continue
            if not inflight:
                if self.active:
                    raise RuntimeError("scheduler: active requests but no rows to run")
                return
            self._collect(inflight.popleft())

    def _issue(self):
        """Build and issue the next step without waiting; the requests of its
        logit rows, or None when there is nothing to run."""
        t_start = time.perf_counter()
        # a request whose last token is in flight no longer holds its slot
        held = sum(1 for r in self.active
                   if r.state != "DECODING" or len(r.generated) + r.inflight < r.max_tokens)
        while self.pending and held < self.max_batch:
            r = self.pending.popleft()
            self._new_seq(r)
            r.state = "PREFILLING"
            r.admit_step = self.steps
            self.active.append(r)
            held += 1
        rows = []  # (request, token, position, wants logits, token source)
        for r in self.active:
            if r.state != "DECODING":
                continue
            g = len(r.generated) + r.inflight
            if g >= r.max_tokens:
                continue  # its last token is in flight
            if r.inflight:
                assert r.lrow_step == self.steps - 1, "decode row without a token in the previous step"
                rows.append((r, 0, len(r.prompt) + g - 1, True, r.lrow))
            else:
                rows.append((r, r.generated[-1], len(r.prompt) + g - 1, True, -1))
        budget = self.max_rows - len(rows)
        for r in self.active:
            if r.state != "PREFILLING" or budget <= 0:
                continue
            c = min(self.prefill_chunk, len(r.prompt) - r.next_prompt, budget)
            for i in range(r.next_prompt, r.next_prompt + c):
                rows.append((r, r.prompt[i], i, i == len(r.prompt) - 1, -1))
            budget -= c
        if not rows:
            self.host_s += time.perf_counter() - t_start
            return None
        t_eng = time.perf_counter()
        self.engine.step_async([r.seq for (r, *_) in rows], [t for (_, t, *_) in rows], [p for (_, _, p, _, _) in rows],
                               want_logits=np.array([w for (_, _, _, w, _) in rows], np.uint8),
                               token_src=[s for (*_, s) in rows])
        t_eng_end = time.perf_counter()
        lrows = []
        for (r, _, _, w, _) in rows:
            if r.state == "PREFILLING":
                r.next_prompt += 1
                if r.next_prompt == len(r.prompt):
                    r.state = "DECODING"
            if w:
                r.lrow, r.lrow_step = len(lrows), self.steps
                r.inflight += 1
                lrows.append(r)
        self.steps += 1
        self.rows += len(rows)
        self.engine_s += t_eng_end - t_eng
        self.host_s += time.perf_counter() - t_start - (t_eng_end - t_eng)
        return lrows

    def _collect(self, lrows):
        """Wait for the oldest issued step and apply its tokens."""
        t_eng = time.perf_counter()
        nx = self.engine.collect()
        t_eng_end = time.perf_counter()
        self.engine_s += t_eng_end - t_eng
        if self.observer is not None:
            self.observer(self, lrows, nx)
        t_obs = time.perf_counter()
        retire = []
        for k, r in enumerate(lrows):
            r.inflight -= 1
            if r.state == "DONE":
                continue  # retired on EOS a step ago: this row ran past it
            t = int(nx[k])
            if (r.eos is not None and t == r.eos) or len(r.generated) >= r.max_tokens:
                retire.append(r)
                continue
            r.generated.append(t)
            if len(r.generated) >= r.max_tokens:
                retire.append(r)
        for r in retire:
            self.active.remove(r)
            self._finish(r)
        self.host_s += time.perf_counter() - t_obs
