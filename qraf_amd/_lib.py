"""ctypes binding of libqraf_hip.so (include/qraf_hip.h).

The library is loaded from this package directory only.  There is no CPU
fallback: if the shared object is missing or fails to load, importing
qraf_amd raises.
"""
from __future__ import annotations

import ctypes as C
import os

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libqraf_hip.so")

OK = 0
ERR_INVALID, ERR_DTYPE, ERR_HIP, ERR_NOMEM, ERR_STATE, ERR_FORMAT = -1, -2, -3, -4, -5, -6
F32, F16, Q8_0, Q4_0, I8 = 0, 1, 10, 20, 102

vp = C.c_void_p
fp = C.POINTER(C.c_float)
u32p = C.POINTER(C.c_uint32)
i32p = C.POINTER(C.c_int32)

# name -> (restype, argtypes); every function returns int status unless noted
SIGNATURES = {
    "qraf_hip_last_error": (C.c_char_p, []),
    "qraf_hip_version": (C.c_char_p, []),
    "qraf_hip_init": (C.c_int, [C.c_int]),
    "qraf_hip_device_count": (C.c_int, [C.POINTER(C.c_int)]),
    "qraf_hip_malloc": (C.c_int, [C.POINTER(vp), C.c_uint64]),
    "qraf_hip_free": (C.c_int, [vp]),
    "qraf_hip_memcpy_h2d": (C.c_int, [vp, vp, C.c_uint64]),
    "qraf_hip_memcpy_d2h": (C.c_int, [vp, vp, C.c_uint64]),
    "qraf_hip_memcpy_d2d": (C.c_int, [vp, vp, C.c_uint64, vp]),
    "qraf_hip_read_probe_dev": (C.c_int, [vp, C.c_uint64, vp, vp]),
    "qraf_hip_read_probe_out_bytes": (C.c_uint64, []),
    "qraf_hip_launch_floor_dev": (C.c_int, [C.c_int32, vp]),
    "qraf_hip_memset": (C.c_int, [vp, C.c_int, C.c_uint64]),
    "qraf_hip_stream_create": (C.c_int, [C.POINTER(vp)]),
    "qraf_hip_stream_destroy": (C.c_int, [vp]),
    "qraf_hip_stream_synchronize": (C.c_int, [vp]),
    "qraf_hip_device_synchronize": (C.c_int, []),
    "qraf_hip_event_create": (C.c_int, [C.POINTER(vp)]),
    "qraf_hip_event_destroy": (C.c_int, [vp]),
    "qraf_hip_event_record": (C.c_int, [vp, vp]),
    "qraf_hip_event_elapsed_ms": (C.c_int, [vp, vp, fp]),
    "qraf_hip_graph_begin": (C.c_int, [vp]),
    "qraf_hip_graph_end": (C.c_int, [vp, C.POINTER(vp)]),
    "qraf_hip_graph_launch": (C.c_int, [vp, vp]),
    "qraf_hip_graph_destroy": (C.c_int, [vp]),
    "qraf_hip_register_weights": (C.c_int, [vp, C.c_uint64]),
    "qraf_hip_unregister_weights": (C.c_int, [vp]),
    "qraf_hip_matvec_q": (C.c_int, [vp, C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, fp, fp]),
    "qraf_hip_matvec_f32": (C.c_int, [fp, fp, fp, C.c_uint32, C.c_uint32]),
    "qraf_hip_dot_f32": (C.c_int, [fp, fp, C.c_int, fp]),
    "qraf_hip_rms_norm": (C.c_int, [fp, fp, C.c_int, C.c_float]),
    "qraf_hip_softmax": (C.c_int, [fp, C.c_int]),
    "qraf_hip_silu": (C.c_int, [fp, C.c_int]),
    "qraf_hip_add": (C.c_int, [fp, fp, C.c_int]),
    "qraf_hip_mul": (C.c_int, [fp, fp, C.c_int]),
    "qraf_hip_scale": (C.c_int, [fp, C.c_float, C.c_int]),
    "qraf_hip_matvec_q_dev": (C.c_int, [vp, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, vp, vp, vp]),
    "qraf_hip_matvec_q_batch_dev": (C.c_int, [vp, C.c_uint32, C.c_uint32, C.c_uint32, vp, C.c_int32, vp, vp]),
    "qraf_hip_matvec_f32_dev": (C.c_int, [vp, vp, vp, C.c_uint32, C.c_uint32, vp]),
    "qraf_hip_set_matvec_tuning": (C.c_int, [C.c_int, C.c_int, C.c_int]),
    "qraf_hip_quantize_dev": (C.c_int, [vp, C.c_uint64, C.c_uint32, vp, vp]),
    "qraf_hip_gen_weights_dev": (C.c_int, [vp, C.c_uint32, C.c_uint64, C.c_uint64, C.c_uint64, C.c_float, vp]),
    "qraf_hip_name_hash": (C.c_uint64, [C.c_char_p]),
    "qraf_hip_attention_workspace_bytes": (C.c_uint64, [C.c_int32] * 5),
    "qraf_hip_set_attention_tuning": (C.c_int, [C.c_int32]),
    "qraf_hip_paged_attention_dev": (C.c_int, [vp, vp, vp, C.c_uint32, vp, C.c_int32, vp] + [C.c_int32] * 5 +
                                     [C.c_float, C.c_int32, vp, vp, C.c_uint64, vp]),
    "qraf_hip_paged_attention_noalloc_dev": (C.c_int, [vp, vp, vp, C.c_uint32, vp, C.c_int32, vp] + [C.c_int32] * 5 +
                                             [C.c_float, C.c_int32, vp, vp]),
    "qraf_hip_attention_noalloc_max_bytes": (C.c_uint64, []),
    "qraf_hip_split_bf16_dev": (C.c_int, [vp, vp, vp, C.c_int32, C.c_int32, vp]),
    "qraf_hip_set_qgemm_tuning": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int]),
    "qraf_hip_set_qgemm_schedule": (C.c_int, [C.c_int32, C.c_int32]),
    "qraf_hip_set_qgemm_kw": (C.c_int, [C.c_int32, C.c_int32]),
    "qraf_hip_tiled_weight_bytes": (C.c_uint64, [C.c_uint32, C.c_uint32, C.c_uint32]),
    "qraf_hip_repack_tiles_dev": (C.c_int, [vp, C.c_uint32, C.c_uint32, C.c_uint32, vp, vp]),
    "qraf_hip_qgemm_tiled_dev": (C.c_int, [vp, C.c_uint32, C.c_uint32, C.c_uint32, vp, vp, C.c_int32, vp, vp, vp,
                                           C.c_uint64, vp]),
    "qraf_hip_qgemm_tiled_argmax_keys_bytes": (C.c_uint64, [C.c_uint32, C.c_int32]),
    "qraf_hip_qgemm_tiled_argmax_dev": (C.c_int, [vp, C.c_uint32, C.c_uint32, C.c_uint32, vp, vp, C.c_int32, vp,
                                                  C.c_uint64, vp, vp, vp]),
    "qraf_hip_qgemm_tiled_silu_dev": (C.c_int, [vp, C.c_uint32, C.c_uint32, C.c_uint32, vp, vp, C.c_int32, vp, vp, vp]),
    "qraf_hip_qgemm_tiled_workspace_bytes": (C.c_uint64, [C.c_uint32, C.c_uint32, C.c_uint32, C.c_int32]),
    "qraf_hip_qgemm_workspace_bytes": (C.c_uint64, [C.c_uint32, C.c_uint32, C.c_uint32, C.c_int32]),
    "qraf_hip_qgemm_dev": (C.c_int, [vp, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, vp, vp, C.c_int32, vp, vp,
                                     vp, C.c_uint64, vp]),
    "qraf_hip_rope_table_host": (C.c_int, [C.c_int32, C.c_int32, C.c_float, fp]),
    "qraf_hip_rope_append_dev": (C.c_int, [vp, vp] + [C.c_int32] * 4 + [vp, vp, vp, vp, vp, C.c_uint32, vp,
                                                                       C.c_int32, C.c_int32, vp]),
}


class ModelConfig(C.Structure):
    """qraf_model_config (include/qraf_hip.h)."""
    _fields_ = [(n, C.c_uint32) for n in ("vocab_size", "hidden_size", "num_layers", "num_heads", "num_kv_heads",
                                          "intermediate_size", "max_seq_len")] + [
        ("rope_theta", C.c_float), ("rms_norm_eps", C.c_float)]


class EngineOptions(C.Structure):
    """qraf_engine_options (include/qraf_hip.h)."""
    _fields_ = [(n, C.c_uint32) for n in ("kv_dtype", "page_size", "max_batch", "num_pages")]


class EngineStats(C.Structure):
    """qraf_engine_stats (include/qraf_hip.h)."""
    _fields_ = [("steps", C.c_uint64), ("rows", C.c_uint64), ("host_us", C.c_double), ("wait_us", C.c_double),
                ("eager_steps", C.c_uint64), ("graph_captures", C.c_uint64), ("graph_launches", C.c_uint64),
                ("pad_rows", C.c_uint64)]


class SamplingParams(C.Structure):
    """qraf_sampling_params (include/qraf_hip.h)."""
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int32), ("top_p", C.c_float),
                ("repetition_penalty", C.c_float)]


SIGNATURES.update({
    "qraf_hip_sample_dev": (C.c_int, [vp, C.c_int32, C.c_int32, C.POINTER(SamplingParams), vp, vp, C.c_int32, vp, vp,
                                      vp]),
    "qraf_engine_sample": (C.c_int, [vp, C.c_int32, C.c_int32, C.POINTER(SamplingParams), u32p, i32p, C.c_int32, fp,
                                     u32p]),
    "qraf_engine_create": (C.c_int, [C.POINTER(ModelConfig), C.POINTER(EngineOptions), C.POINTER(vp)]),
    "qraf_engine_destroy": (C.c_int, [vp]),
    "qraf_engine_set_tensor": (C.c_int, [vp, C.c_char_p, C.c_uint32, C.c_uint32, u32p, C.c_uint32, vp, C.c_uint64]),
    "qraf_engine_generate_weights": (C.c_int, [vp, C.c_uint32, C.c_uint32, C.c_uint32, C.c_int32, C.c_int32,
                                               C.c_uint64]),
    "qraf_engine_finalize": (C.c_int, [vp]),
    "qraf_engine_seq_create": (C.c_int, [vp, i32p]),
    "qraf_engine_seq_release": (C.c_int, [vp, C.c_int32]),
    "qraf_engine_seq_length": (C.c_int, [vp, C.c_int32, i32p]),
    "qraf_engine_free_pages": (C.c_int, [vp, i32p]),
    "qraf_engine_step": (C.c_int, [vp, C.c_int32, i32p, u32p, i32p, C.POINTER(C.c_uint8), fp, u32p]),
    "qraf_engine_step_async": (C.c_int, [vp, C.c_int32, i32p, u32p, i32p, i32p, C.POINTER(C.c_uint8)]),
    "qraf_engine_step_collect": (C.c_int, [vp, u32p, i32p]),
    "qraf_engine_set_graphs": (C.c_int, [vp, C.c_int32]),
    "qraf_engine_set_keep_logits": (C.c_int, [vp, C.c_int32]),
    "qraf_engine_set_row_padding": (C.c_int, [vp, C.c_int32]),
    "qraf_engine_set_fusion": (C.c_int, [vp, C.c_int32]),
    "qraf_engine_set_repetition_penalty": (C.c_int, [vp, C.c_int32, C.c_float]),
    "qraf_engine_forward": (C.c_int, [vp, C.c_uint32, C.c_int32, fp]),
    "qraf_engine_read_logits": (C.c_int, [vp, C.c_int32, C.c_int32, fp]),
    "qraf_engine_get_stats": (C.c_int, [vp, vp, C.c_int32]),
    "qraf_engine_reset": (C.c_int, [vp]),
    "qraf_file_read_config": (C.c_int, [C.c_char_p, C.POINTER(ModelConfig), u32p]),
    "qraf_engine_create_from_file": (C.c_int, [C.c_char_p, C.POINTER(EngineOptions), C.POINTER(vp)]),
})


class HipError(RuntimeError):
    def __init__(self, fn, code, msg):
        super().__init__(f"{fn} -> {code}: {msg}")
        self.code = code


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built; run `python qraf_amd/build.py` (no CPU fallback exists)")
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib


lib = _load()


def check(fn_name, rc):
    if rc != OK:
        msg = lib.qraf_hip_last_error()
        raise HipError(fn_name, rc, msg.decode() if msg else "")
    return rc


def call(name, *args):
    """Call `name` and raise HipError on a nonzero status."""
    return check(name, getattr(lib, name)(*args))
