"""QRAF file parsing on the host (qraf_file_read_config), against files
written by the reference's QrafWriter (writer.cpp), and the format checks of
validate_header (header.cpp:8-45) and get_string (loader.cpp:273-277) on
corrupted copies.  No GPU use: this runs in the CPU suite.
"""
import os
import struct

import pytest

from oracle import pyoracle as po

need_ref = pytest.mark.skipif(po.ref() is None, reason="oracle/_ref (the compiled reference) is not built")

KW = dict(vocab=640, hidden=128, layers=2, heads=4, kv_heads=1, inter=160, max_seq=128, rope_theta=1e6, eps=1e-6,
          wdtype=po.Q4_0, tied=True, qkv_bias=True)

# QrafHeader field offsets (format.h:26-49)
H_MAGIC, H_VERSION, H_FILE_SIZE = 0, 4, 8
H_TENSOR_DIR, H_STRINGS, H_STRINGS_SIZE, H_NUM_TENSORS = 48, 80, 88, 104


def lib():
    from qraf_amd._lib import lib as L
    return L


def read_config(path):
    import ctypes as C
    from qraf_amd._lib import ModelConfig
    cfg, n = ModelConfig(), C.c_uint32()
    rc = lib().qraf_file_read_config(os.fsencode(path), C.byref(cfg), C.byref(n))
    return rc, cfg, n.value


@pytest.fixture(scope="module")
def written(tmp_path_factory):
    m = po.Model(po.make_config(**KW), 21)
    path = str(tmp_path_factory.mktemp("qraf") / "m.qraf")
    m.write_qraf(path)
    yield m, path
    m.close()


@need_ref
def test_config_as_written(written):
    m, path = written
    rc, cfg, n = read_config(path)
    assert rc == 0, lib().qraf_hip_last_error()
    c = m.cfg
    assert (cfg.vocab_size, cfg.hidden_size, cfg.num_layers, cfg.num_heads, cfg.num_kv_heads,
            cfg.intermediate_size, cfg.max_seq_len) == (c.vocab, c.hidden, c.layers, c.heads, c.kv_heads, c.inter,
                                                        c.max_seq)
    assert cfg.rope_theta == pytest.approx(c.rope_theta, rel=0) and cfg.rms_norm_eps == pytest.approx(c.eps, rel=0)
    assert n == len(m.tensors())


def corrupt(path, tmp_path, patch, name):
    b = bytearray(open(path, "rb").read())
    b = patch(b)
    out = str(tmp_path / name)
    open(out, "wb").write(bytes(b))
    return out


def u32(b, off, v):
    struct.pack_into("<I", b, off, v)
    return b


def u64(b, off, v):
    struct.pack_into("<Q", b, off, v)
    return b


def first_tensor(b):
    return struct.unpack_from("<Q", b, H_TENSOR_DIR)[0]


@need_ref
@pytest.mark.parametrize("case", ["magic", "version", "size_field", "appended", "truncated", "tiny", "name_offset",
                                  "data_past_end", "string_table_cut", "tensor_count"])
def test_malformed_files_are_refused(written, tmp_path, case):
    from qraf_amd._lib import ERR_FORMAT
    _, path = written
    patches = {
        "magic": lambda b: u32(b, H_MAGIC, 0x12345678),
        "version": lambda b: u32(b, H_VERSION, 2),
        "size_field": lambda b: u64(b, H_FILE_SIZE, len(b) + 64),
        "appended": lambda b: b + b"\0",
        "truncated": lambda b: b[: len(b) // 2],
        "tiny": lambda b: b[:100],
        # first tensor's name offset (TensorMeta + 8) past the string table
        "name_offset": lambda b: u32(b, first_tensor(b) + 8, 0x7FFFFFF0),
        # first tensor's data offset (TensorMeta + 56) at the end of the file
        "data_past_end": lambda b: u64(b, first_tensor(b) + 56, len(b)),
        # a string table of 3 bytes: names no longer end inside it
        "string_table_cut": lambda b: u64(b, H_STRINGS_SIZE, 3),
        "tensor_count": lambda b: u32(b, H_NUM_TENSORS, 1 << 30),
    }
    bad = corrupt(path, tmp_path, patches[case], case + ".qraf")
    rc, _, _ = read_config(bad)
    assert rc == ERR_FORMAT, (case, rc, lib().qraf_hip_last_error())


@need_ref
@pytest.mark.parametrize("case", ["magic", "version", "size_field", "appended", "truncated", "data_past_end"])
def test_reference_refuses_the_same_files(written, tmp_path, case):
    """The cases validate_header and parse_tensor_directory check: the
    reference's own QrafModel::load refuses them too."""
    _, path = written
    patches = {
        "magic": lambda b: u32(b, H_MAGIC, 0x12345678),
        "version": lambda b: u32(b, H_VERSION, 2),
        "size_field": lambda b: u64(b, H_FILE_SIZE, len(b) + 64),
        "appended": lambda b: b + b"\0",
        "truncated": lambda b: b[: len(b) // 2],
        "data_past_end": lambda b: u64(b, first_tensor(b) + 56, len(b)),
    }
    bad = corrupt(path, tmp_path, patches[case], case + ".qraf")
    with pytest.raises(RuntimeError):
        po.RefModel(bad, KW["vocab"])


def test_missing_file():
    from qraf_amd._lib import ERR_INVALID
    rc, _, _ = read_config("/nonexistent/model.qraf")
    assert rc == ERR_INVALID and b"cannot open" in lib().qraf_hip_last_error()


def test_defaults_for_absent_keys(tmp_path):
    """A file with an empty config block and no tensors: ModelConfig's
    defaults (types.h:97-110) and num_kv_heads = num_heads (types.h:123)."""
    strings = b"\0"
    hdr_size, cfg_off = 128, 128
    cfg = struct.pack("<I", 0)
    str_off = cfg_off + len(cfg)
    data_off = (str_off + len(strings) + 63) // 64 * 64
    size = data_off
    hdr = struct.pack("<IIQ" + "Q" * 11 + "IIII8s", 0x46415251, 1, size, cfg_off, len(cfg), 0, 0, str_off, 0,
                      str_off, 0, str_off, len(strings), data_off, 0, 0, 0, 0, b"\0" * 8)
    assert len(hdr) == hdr_size
    body = hdr + cfg + strings
    body += b"\0" * (size - len(body))
    path = str(tmp_path / "empty.qraf")
    open(path, "wb").write(body)
    rc, c, n = read_config(path)
    assert rc == 0, lib().qraf_hip_last_error()
    assert (c.vocab_size, c.hidden_size, c.num_layers, c.num_heads, c.num_kv_heads, c.max_seq_len, n) == \
        (0, 0, 0, 0, 0, 2048, 0)
    assert c.rope_theta == 10000.0 and c.rms_norm_eps == pytest.approx(1e-5, rel=1e-7)
