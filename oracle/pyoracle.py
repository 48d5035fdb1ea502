"""ctypes access to the test oracle (liboracle.so) and, where it was built, the
compiled reference (_ref/libqraf_ref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() and
by the cpu_baseline leg of bench.py, never by the product package.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
F32, F16, Q8_0, Q4_0, I8 = 0, 1, 10, 20, 102

_fp = C.POINTER(C.c_float)
_u8p = C.POINTER(C.c_uint8)
_u32p = C.POINTER(C.c_uint32)


def _f(a):
    return a.ctypes.data_as(_fp)


def _u8(a):
    return a.ctypes.data_as(_u8p)


def _u32(a):
    return a.ctypes.data_as(_u32p)


class OrConfig(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("vocab", "hidden", "layers", "heads", "kv_heads", "inter", "max_seq")] + [
        ("rope_theta", C.c_float), ("eps", C.c_float),
        ("wdtype", C.c_uint32), ("embed_dtype", C.c_uint32), ("head_dtype", C.c_uint32),
        ("tied", C.c_int32), ("qkv_bias", C.c_int32), ("block_size", C.c_int32)]


def _load(path):
    if not os.path.exists(path):
        return None
    return C.CDLL(path)


_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        _lib = _load(os.path.join(HERE, "liboracle.so"))
        if _lib is None:
            raise RuntimeError("oracle/liboracle.so is not built (run __graft_entry__.build())")
        L = _lib
        L.or_fp16_to_fp32.restype = C.c_float
        L.or_fp16_to_fp32.argtypes = [C.c_uint16]
        L.or_fp32_to_fp16.restype = C.c_uint16
        L.or_fp32_to_fp16.argtypes = [C.c_float]
        L.or_q_tensor_bytes.restype = C.c_size_t
        L.or_q_tensor_bytes.argtypes = [C.c_uint32, C.c_size_t, C.c_int]
        for n in ("or_quantize_q8_0", "or_quantize_q4_0"):
            getattr(L, n).restype = C.c_size_t
            getattr(L, n).argtypes = [_fp, C.c_size_t, C.c_int, _u8p]
        L.or_dequantize.argtypes = [C.c_void_p, C.c_uint32, C.c_size_t, C.c_int, _fp]
        for n in ("or_dot_q8_0_f32", "or_dot_q4_0_f32"):
            getattr(L, n).restype = C.c_float
            getattr(L, n).argtypes = [C.c_void_p, _fp, C.c_size_t, C.c_int]
        L.or_matvec_q.argtypes = [C.c_void_p, C.c_uint32, C.c_int, C.c_uint32, C.c_uint32, _fp, _fp]
        L.or_matvec_f32.argtypes = [_fp, _fp, _fp, C.c_uint32, C.c_uint32]
        L.or_dot_f32.restype = C.c_float
        L.or_dot_f32.argtypes = [_fp, _fp, C.c_int]
        L.or_rms_norm.argtypes = [_fp, _fp, C.c_int, C.c_float]
        L.or_rope.argtypes = [_fp, C.c_int, C.c_int, C.c_float]
        for n in ("or_silu", "or_softmax"):
            getattr(L, n).argtypes = [_fp, C.c_int]
        L.or_attention_decode.argtypes = [_fp, _fp, _fp, C.c_int, C.c_int, C.c_int, C.c_int, _fp]
        L.or_kv_quant_head.argtypes = [_fp, C.c_int, C.c_void_p, _fp]
        L.or_kv_dot_key.restype = C.c_float
        L.or_kv_dot_key.argtypes = [C.c_void_p, C.c_float, _fp, C.c_int]
        L.or_attention_decode_i8.argtypes = [_fp, C.c_void_p, _fp, C.c_void_p, _fp, C.c_int, C.c_int, C.c_int,
                                             C.c_int, _fp]
        L.or_argmax.restype = C.c_uint32
        L.or_argmax.argtypes = [_fp, C.c_int]
        L.or_repetition_penalty.argtypes = [_fp, C.c_int, _u32p, C.c_int, C.c_float]
        L.or_mix64.restype = C.c_uint64
        L.or_mix64.argtypes = [C.c_uint64]
        L.or_fnv1a.restype = C.c_uint64
        L.or_fnv1a.argtypes = [C.c_char_p]
        L.or_gen_scale.restype = C.c_float
        L.or_gen_scale.argtypes = [C.c_float]
        L.or_gen_normal.argtypes = [C.c_uint64, C.c_uint64, C.c_size_t, C.c_float, _fp]
        L.or_gen_token.restype = C.c_uint32
        L.or_gen_token.argtypes = [C.c_uint64, C.c_uint64, C.c_uint32]
        L.or_model_generate.restype = C.c_void_p
        L.or_model_generate.argtypes = [C.POINTER(OrConfig), C.c_uint64]
        L.or_model_free.argtypes = [C.c_void_p]
        L.or_model_num_tensors.argtypes = [C.c_void_p]
        L.or_model_tensor.argtypes = [C.c_void_p, C.c_int, C.POINTER(C.c_char_p), _u32p, _u32p, _u32p,
                                      C.POINTER(C.c_void_p), C.POINTER(C.c_uint64)]
        L.or_model_reset.argtypes = [C.c_void_p]
        L.or_model_set_kv_int8.argtypes = [C.c_void_p]
        L.or_model_forward.argtypes = [C.c_void_p, C.c_uint32, C.c_int, _fp]
        L.or_generate.argtypes = [C.c_void_p, _u32p, C.c_int, C.c_int, C.c_float, C.c_int, _u32p]
    return _lib


def ref():
    """The compiled reference, or None when oracle/_ref was not built."""
    global _ref
    if _ref is None:
        _ref = _load(os.path.join(HERE, "_ref", "libqraf_ref.so"))
        if _ref is None:
            return None
        R = _ref
        R.ref_fp16_to_fp32.restype = C.c_float
        R.ref_fp16_to_fp32.argtypes = [C.c_uint16]
        R.ref_fp32_to_fp16.restype = C.c_uint16
        R.ref_fp32_to_fp16.argtypes = [C.c_float]
        R.ref_quantize.restype = C.c_size_t
        R.ref_quantize.argtypes = [C.c_uint32, _fp, C.c_size_t, C.c_int, _u8p]
        R.ref_dot.restype = C.c_float
        R.ref_dot.argtypes = [C.c_uint32, C.c_void_p, _fp, C.c_size_t, C.c_int]
        R.ref_matvec_q.argtypes = [C.c_void_p, C.c_uint32, C.c_int, C.c_uint32, C.c_uint32, _fp, _fp]
        R.ref_matvec_f32.argtypes = [_fp, _fp, _fp, C.c_uint32, C.c_uint32]
        R.ref_rms_norm.argtypes = [_fp, _fp, C.c_int, C.c_float]
        R.ref_softmax.argtypes = [_fp, C.c_int]
        R.ref_silu.argtypes = [_fp, C.c_int]
        R.ref_rope.argtypes = [_fp, _fp, C.c_int, C.c_int, C.c_float]
        R.ref_dequantize.argtypes = [C.c_void_p, C.c_uint32, C.c_size_t, C.c_int, _fp]
        R.ref_argmax.restype = C.c_uint32
        R.ref_argmax.argtypes = [_fp, C.c_int]
        R.ref_penalty.argtypes = [_fp, C.c_int, _u32p, C.c_int, C.c_float]
        R.ref_sample.argtypes = [_fp, C.c_int, C.c_float, C.c_int, C.c_float, C.c_uint64, C.c_int, _u32p]
        R.ref_uniforms.argtypes = [C.c_uint64, C.c_int, _fp]
        R.ref_kv_quant.argtypes = [_fp, _fp, C.c_int, C.c_int, _fp, C.c_void_p, _fp, C.c_void_p, _fp, _fp, _fp]
        R.ref_engine_generate_sampled.argtypes = [C.c_void_p, _u32p, C.c_int, C.c_int, C.c_float, C.c_int,
                                                  C.c_float, C.c_float, C.c_uint64, _u32p]
        R.ref_writer_new.restype = C.c_void_p
        R.ref_writer_free.argtypes = [C.c_void_p]
        R.ref_writer_config_u32.argtypes = [C.c_void_p, C.c_char_p, C.c_uint32]
        R.ref_writer_config_f32.argtypes = [C.c_void_p, C.c_char_p, C.c_float]
        R.ref_writer_config_str.argtypes = [C.c_void_p, C.c_char_p, C.c_char_p]
        R.ref_writer_quant_scheme.restype = C.c_uint32
        R.ref_writer_quant_scheme.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32]
        R.ref_writer_tensor.argtypes = [C.c_void_p, C.c_char_p, _u32p, C.c_uint32, C.c_uint32, C.c_void_p,
                                        C.c_uint64, C.c_uint32]
        R.ref_writer_write.argtypes = [C.c_void_p, C.c_char_p]
        R.ref_model_load.restype = C.c_void_p
        R.ref_model_load.argtypes = [C.c_char_p]
        R.ref_model_free.argtypes = [C.c_void_p]
        R.ref_model_reset.argtypes = [C.c_void_p]
        R.ref_model_forward.argtypes = [C.c_void_p, C.c_uint32, C.c_int, _fp]
        R.ref_engine_load.restype = C.c_void_p
        R.ref_engine_load.argtypes = [C.c_char_p]
        R.ref_engine_free.argtypes = [C.c_void_p]
        R.ref_engine_generate.argtypes = [C.c_void_p, _u32p, C.c_int, C.c_int, C.c_float, _u32p,
                                          C.POINTER(C.c_double)]
    return _ref


# ---------------------------------------------------------------- op helpers

def quantize(dtype, x, bs=32):
    x = np.ascontiguousarray(x, dtype=np.float32)
    L = lib()
    out = np.zeros(L.or_q_tensor_bytes(dtype, x.size, bs), dtype=np.uint8)
    fn = L.or_quantize_q8_0 if dtype == Q8_0 else L.or_quantize_q4_0
    fn(_f(x), x.size, bs, _u8(out))
    return out


def dequantize(dtype, q, count, bs=32):
    out = np.zeros(count, dtype=np.float32)
    q = np.ascontiguousarray(q)
    if lib().or_dequantize(q.ctypes.data, dtype, count, bs, _f(out)) != 0:
        raise ValueError("unsupported dtype")
    return out


def dot(dtype, q, x, bs=32):
    x = np.ascontiguousarray(x, dtype=np.float32)
    fn = lib().or_dot_q8_0_f32 if dtype == Q8_0 else lib().or_dot_q4_0_f32
    return fn(np.ascontiguousarray(q).ctypes.data, _f(x), x.size, bs)


def matvec_q(w, dtype, out_dim, in_dim, x, bs=32):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros(out_dim, dtype=np.float32)
    lib().or_matvec_q(np.ascontiguousarray(w).ctypes.data, dtype, bs, out_dim, in_dim, _f(x), _f(y))
    return y


def matvec_f32(W, x):
    W = np.ascontiguousarray(W, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros(W.shape[0], dtype=np.float32)
    lib().or_matvec_f32(_f(W), _f(x), _f(y), W.shape[0], W.shape[1])
    return y


def gen_normal(seed, stream, n, std=0.02):
    out = np.zeros(n, dtype=np.float32)
    lib().or_gen_normal(seed, stream, n, std, _f(out))
    return out


def fnv1a(name: str) -> int:
    return lib().or_fnv1a(name.encode())


def attention_decode(q, K, V, H, Hkv, hd):
    q = np.ascontiguousarray(q, dtype=np.float32)
    K = np.ascontiguousarray(K, dtype=np.float32)
    V = np.ascontiguousarray(V, dtype=np.float32)
    out = np.zeros(H * hd, dtype=np.float32)
    lib().or_attention_decode(_f(q), _f(K), _f(V), K.shape[0], H, Hkv, hd, _f(out))
    return out


def kv_quant_heads(x, Hkv, hd):
    """QuantizedKVCache::store of one position's [Hkv][hd] values: (int8 [Hkv][hd], f32 scales [Hkv])."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(Hkv, hd)
    q = np.zeros((Hkv, hd), np.int8)
    s = np.zeros(Hkv, np.float32)
    for h in range(Hkv):
        lib().or_kv_quant_head(_f(x[h]), hd, q[h].ctypes.data, _f(s[h:h + 1]))
    return q, s


def attention_decode_i8(q, K8, Ks, V8, Vs, H, Hkv, hd):
    """K8, V8: int8 [ctx][Hkv][hd]; Ks, Vs: f32 [ctx][Hkv]."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    K8, V8 = np.ascontiguousarray(K8, dtype=np.int8), np.ascontiguousarray(V8, dtype=np.int8)
    Ks, Vs = np.ascontiguousarray(Ks, dtype=np.float32), np.ascontiguousarray(Vs, dtype=np.float32)
    out = np.zeros(H * hd, dtype=np.float32)
    lib().or_attention_decode_i8(_f(q), K8.ctypes.data, _f(Ks), V8.ctypes.data, _f(Vs), K8.shape[0], H, Hkv, hd,
                                 _f(out))
    return out


# ---------------------------------------------------------------- model

def make_config(vocab, hidden, layers, heads, kv_heads, inter, max_seq=2048, rope_theta=1e4, eps=1e-5,
                wdtype=Q8_0, embed_dtype=None, head_dtype=None, tied=False, qkv_bias=False, block_size=32):
    return OrConfig(vocab, hidden, layers, heads, kv_heads, inter, max_seq, rope_theta, eps, wdtype,
                    wdtype if embed_dtype is None else embed_dtype,
                    wdtype if head_dtype is None else head_dtype, int(tied), int(qkv_bias), block_size)


class Model:
    """or_model: synthetic weights, scalar forward and greedy generate."""

    def __init__(self, cfg: OrConfig, seed: int):
        self.cfg = cfg
        self.seed = seed
        self.h = lib().or_model_generate(C.byref(cfg), seed)

    def close(self):
        if self.h:
            lib().or_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensors(self):
        """list of (name, dtype, shape, numpy uint8 view of the bytes)."""
        L = lib()
        out = []
        for i in range(L.or_model_num_tensors(self.h)):
            name = C.c_char_p()
            dt, nd = C.c_uint32(), C.c_uint32()
            shape = (C.c_uint32 * 2)()
            data = C.c_void_p()
            size = C.c_uint64()
            L.or_model_tensor(self.h, i, C.byref(name), C.byref(dt), C.byref(nd), shape, C.byref(data),
                              C.byref(size))
            buf = np.ctypeslib.as_array(C.cast(data, _u8p), shape=(size.value,)) if size.value else \
                np.zeros(0, np.uint8)
            out.append((name.value.decode(), dt.value, tuple(shape[: nd.value]), buf))
        return out

    def reset(self):
        lib().or_model_reset(self.h)

    def set_kv_int8(self):
        """Use QuantizedKVCache (int8 K/V, a scale per position and KV head) from here on."""
        if lib().or_model_set_kv_int8(self.h) != 0:
            raise MemoryError("int8 KV cache allocation failed")

    def forward(self, token, pos):
        logits = np.zeros(self.cfg.vocab, dtype=np.float32)
        if lib().or_model_forward(self.h, token, pos, _f(logits)) != 0:
            raise ValueError("forward failed (token/pos out of range)")
        return logits

    def generate(self, prompt, max_tokens, penalty=1.0, eos=-1):
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.zeros(max_tokens, dtype=np.uint32)
        n = lib().or_generate(self.h, _u32(p), p.size, max_tokens, penalty, eos, _u32(out))
        return out[:n].tolist()

    def write_qraf(self, path, arch=None):
        """Write this model as a .qraf file with the reference's QrafWriter
        (architecture "qwen2" with q/k/v biases, else "llama", unless given)."""
        R = ref()
        if R is None:
            raise RuntimeError("oracle/_ref not built")
        c = self.cfg
        w = R.ref_writer_new()
        if arch is None:
            arch = "qwen2" if c.qkv_bias else "llama"
        R.ref_writer_config_str(w, b"architecture", arch.encode())
        for k in ("vocab", "hidden", "layers", "heads", "kv_heads", "inter", "max_seq"):
            key = {"vocab": "vocab_size", "hidden": "hidden_size", "layers": "num_layers", "heads": "num_heads",
                   "kv_heads": "num_kv_heads", "inter": "intermediate_size", "max_seq": "max_seq_len"}[k]
            R.ref_writer_config_u32(w, key.encode(), getattr(c, k))
        R.ref_writer_config_f32(w, b"rope_theta", c.rope_theta)
        R.ref_writer_config_f32(w, b"rms_norm_eps", c.eps)
        schemes = {}
        for dt in (Q8_0, Q4_0):
            schemes[dt] = R.ref_writer_quant_scheme(w, dt, c.block_size)
        for name, dt, shape, buf in self.tensors():
            sh = np.array(shape, dtype=np.uint32)
            R.ref_writer_tensor(w, name.encode(), _u32(sh), len(shape), dt, buf.ctypes.data, buf.size,
                                schemes.get(dt, 0xFFFFFFFF))
        rc = R.ref_writer_write(w, path.encode())
        R.ref_writer_free(w)
        if rc != 0:
            raise RuntimeError("QrafWriter::write failed")


class RefModel:
    """QrafModel::load + Transformer::init / forward / reset (the reference)."""

    def __init__(self, path, vocab):
        self.R = ref()
        self.vocab = vocab
        self.h = self.R.ref_model_load(path.encode())
        if not self.h:
            raise RuntimeError("reference failed to load " + path)

    def close(self):
        if self.h:
            self.R.ref_model_free(self.h)
            self.h = None

    def reset(self):
        self.R.ref_model_reset(self.h)

    def forward(self, token, pos):
        logits = np.zeros(self.vocab, dtype=np.float32)
        if self.R.ref_model_forward(self.h, token, pos, _f(logits)) != 0:
            raise ValueError("reference forward failed")
        return logits


class RefEngine:
    """InferenceEngine::generate_tokens, greedy (the reference)."""

    def __init__(self, path):
        self.R = ref()
        self.h = self.R.ref_engine_load(path.encode())
        if not self.h:
            raise RuntimeError("reference engine failed to load " + path)

    def close(self):
        if self.h:
            self.R.ref_engine_free(self.h)
            self.h = None

    def generate(self, prompt, max_tokens, penalty=1.0):
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.zeros(max_tokens, dtype=np.uint32)
        ms = C.c_double()
        n = self.R.ref_engine_generate(self.h, _u32(p), p.size, max_tokens, penalty, _u32(out), C.byref(ms))
        return out[:n].tolist(), ms.value

    def generate_sampled(self, prompt, max_tokens, temperature, top_k, top_p, penalty, seed):
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.zeros(max_tokens, dtype=np.uint32)
        n = self.R.ref_engine_generate_sampled(self.h, _u32(p), p.size, max_tokens, temperature, top_k, top_p,
                                               penalty, seed, _u32(out))
        return out[:n].tolist()
