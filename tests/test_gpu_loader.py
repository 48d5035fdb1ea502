"""A .qraf file written by the reference's QrafWriter, loaded by
qraf_engine_create_from_file (QrafModel::load + Transformer::init in one
call), must give bit-identical logits to the same tensors bound through
qraf_engine_set_tensor, and the oracle's logits within the engine bar
(1e-3 relative + 1e-4 absolute); the reference's own loader on the same file
gives the oracle's logits, which pins the file round trip on both sides.
"""
import numpy as np
import pytest

from oracle import pyoracle as po
from tests.test_gpu_engine import SMALL, check_logits, upload

pytestmark = [pytest.mark.gpu,
              pytest.mark.usefixtures("reference")]


@pytest.mark.parametrize("name", ["q8_llama", "q4_qwen2_tied_bias", "f32_llama", "q8_hd64_gqa3"])
def test_file_load_equals_tensor_binding(hip, tmp_path, name):
    from qraf_amd.engine import Transformer
    kw, seed = SMALL[name]
    print(f"file load {name}", flush=True)
    m = po.Model(po.make_config(**kw), seed)
    path = str(tmp_path / (name + ".qraf"))
    m.write_qraf(path)
    tf_file = Transformer.from_file(path)
    tf_bind = upload(m, kw)
    ref = po.RefModel(path, kw["vocab"])
    prompt = [po.lib().or_gen_token(seed, i, kw["vocab"]) for i in range(10)]
    m.reset()
    for pos, t in enumerate(prompt):
        a, b = tf_file.forward(t, pos), tf_bind.forward(t, pos)
        want = m.forward(t, pos)
        assert np.array_equal(a, b), f"{name} pos {pos}: file load differs from tensor binding"
        check_logits(a, want, f"{name} pos {pos}")
        assert np.array_equal(ref.forward(t, pos), want), f"{name} pos {pos}: reference loader vs oracle"
    ref.close()
    tf_file.engine.close()
    tf_bind.engine.close()
    m.close()


def test_unsupported_architecture_is_refused(hip, tmp_path):
    from qraf_amd._lib import ERR_INVALID, HipError
    from qraf_amd.engine import Engine
    kw, seed = SMALL["q8_llama"]
    m = po.Model(po.make_config(**kw), seed)
    path = str(tmp_path / "gpt2.qraf")
    m.write_qraf(path, arch="gpt2")
    with pytest.raises(HipError) as e:
        Engine.from_file(path)
    assert e.value.code == ERR_INVALID and "gpt2" in str(e.value)
    m.close()


def test_malformed_file_is_refused_before_any_allocation(hip, tmp_path):
    from qraf_amd._lib import ERR_FORMAT, HipError
    from qraf_amd.engine import Engine
    kw, seed = SMALL["q8_llama"]
    m = po.Model(po.make_config(**kw), seed)
    path = str(tmp_path / "m.qraf")
    m.write_qraf(path)
    b = bytearray(open(path, "rb").read())
    open(path, "wb").write(bytes(b[: len(b) - 1]))
    with pytest.raises(HipError) as e:
        Engine.from_file(path)
    assert e.value.code == ERR_FORMAT
    m.close()


@pytest.mark.parametrize("bs,dt", [(8, po.Q8_0), (16, po.Q4_0)])
def test_file_load_block_sizes(hip, tmp_path, bs, dt):
    """A file whose quant scheme carries block size 8 or 16 (QrafWriter writes
    the model's block size into the scheme record): qraf_engine_create_from_file
    binds every tensor at that size, and its logits are within the engine bar of
    the oracle's model of the same block size, which the reference's own loader
    reproduces bit for bit."""
    from qraf_amd.engine import Transformer
    kw = dict(vocab=300, hidden=128, layers=2, heads=4, kv_heads=2, inter=192, max_seq=64, rope_theta=1e5, eps=1e-5,
              wdtype=dt, tied=(dt == po.Q4_0), qkv_bias=(dt == po.Q4_0))
    m = po.Model(po.make_config(**kw, block_size=bs), 60 + bs)
    path = str(tmp_path / f"bs{bs}.qraf")
    m.write_qraf(path)
    tf = Transformer.from_file(path)
    ref = po.RefModel(path, kw["vocab"])
    m.reset()
    for pos, t in enumerate([5, 299, 0, 42, 42, 7, 100, 3]):
        got, want = tf.forward(t, pos), m.forward(t, pos)
        check_logits(got, want, f"block size {bs} pos {pos}")
        assert np.array_equal(ref.forward(t, pos), want), f"block size {bs} pos {pos}: reference loader vs oracle"
    ref.close()
    tf.engine.close()
    m.close()
