"""Model creation from esm.cpp GGUF files (esm_gfx950_model_create_from_gguf,
reference Model::LoadFromGguf, src/model.cpp:229-298), on the GPU.

* Round trip (tests/python/test_gguf_quantized.py:26-48, atol = rtol = 0): a
  file written by the reference's own GgufFile::Write in SaveToGguf's order,
  and one written by esm_gfx950.gguf.write_model, load into models whose
  logits are identical to the model created from the same weights directly;
  Q8_ESM (W8A8) and F32 files.
* Malformed or foreign files fail with the reference reader's messages.
"""
import struct

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

import esm_gfx950 as eg
from esm_gfx950 import gguf
from esm_gfx950 import synthetic as syn


def _weights(int8):
    if int8:
        return syn.make_weights(syn.ESM2_650M.with_layers(2), seed=20261201 + 4, int8=True, keep_f32_linears=True)
    return syn.make_weights(syn.ESM2_8M, seed=20261201 + 1, int8=False)


@pytest.fixture(scope="module")
def batch():
    return syn.batch_from_lengths([130, 61, 250, 2, 97], seed=7)


@pytest.mark.parametrize("writer", ["reference", "esm_gfx950"])
@pytest.mark.parametrize("int8", [True, False])
def test_gguf_round_trip_preserves_forward(dev, ref, tmp_path, batch, int8, writer):
    w = _weights(int8)
    p = str(tmp_path / f"{writer}_{int(int8)}.gguf")
    if writer == "reference":
        from pyoracle import RefModel
        rm = RefModel(ref, w, int8=int8)
        rm.save_gguf(p)
        rm.free()
    else:
        gguf.write_model(p, w, int8=int8)
    direct = eg.Model(dev, w, int8=int8)
    want = direct.forward_packed(batch.ids, batch.cu)
    direct.free()
    loaded = eg.Model.from_gguf(dev, p)
    got = loaded.forward_packed(batch.ids, batch.cu)
    loaded.free()
    np.testing.assert_array_equal(got, want)


def _write_bytes(path, data: bytes):
    with open(path, "wb") as f:
        f.write(data)


def test_gguf_errors(dev, tmp_path):
    p = str(tmp_path / "e.gguf")
    _write_bytes(p, b"NOTGGUFCONTENTSHERE\0" + bytes(16))
    with pytest.raises(eg.Gfx950Error, match="bad magic"):
        eg.Model.from_gguf(dev, p)
    _write_bytes(p, b"GGUF" + struct.pack("<IQQ", 2, 0, 0))
    with pytest.raises(eg.Gfx950Error, match="version 2 not supported"):
        eg.Model.from_gguf(dev, p)
    _write_bytes(p, b"GGUF" + struct.pack("<I", 3))
    with pytest.raises(eg.Gfx950Error, match="file too small"):
        eg.Model.from_gguf(dev, p)
    with pytest.raises(eg.Gfx950Error, match="open failed"):
        eg.Model.from_gguf(dev, str(tmp_path / "absent.gguf"))
    gguf.write(p, {"general.architecture": "llama"}, [])
    with pytest.raises(eg.Gfx950Error, match="not an esm-arch file"):
        eg.Model.from_gguf(dev, p)
    # Truncated data section.
    w = syn.make_weights(syn.ESM2_8M.with_layers(1), seed=3, int8=False)
    gguf.write_model(p, w, int8=False)
    data = open(p, "rb").read()
    _write_bytes(p, data[: len(data) - 4096])
    with pytest.raises(eg.Gfx950Error, match="overruns file"):
        eg.Model.from_gguf(dev, p)


def test_gguf_missing_and_mistyped_tensors(dev, tmp_path):
    w = syn.make_weights(syn.ESM2_8M.with_layers(1), seed=3, int8=True, keep_f32_linears=True)
    p = str(tmp_path / "m.gguf")
    gguf.write_model(p, w, int8=False)
    meta, ts = gguf.read(p)
    tensors = [(n, t, d, (a.tobytes())) for n, (t, d, a) in ts.items() if n != "blk.0.ffn_up.bias"]
    gguf.write(p, meta, tensors)
    with pytest.raises(eg.Gfx950Error, match="missing tensor blk.0.ffn_up.bias"):
        eg.Model.from_gguf(dev, p)
    # F32 linears in a file that says Q8_ESM.
    meta["esm.weights_quantized"] = True
    gguf.write(p, meta, [(n, t, d, a.tobytes()) for n, (t, d, a) in ts.items()])
    with pytest.raises(eg.Gfx950Error, match="expected Q8_ESM for blk.0.attn_q.weight"):
        eg.Model.from_gguf(dev, p)
    meta["esm.weights_quantized"] = False
    meta["esm.embedding_length"] = 640
    gguf.write(p, meta, [(n, t, d, a.tobytes()) for n, (t, d, a) in ts.items()])
    with pytest.raises(eg.Gfx950Error, match="expected"):
        eg.Model.from_gguf(dev, p)


def test_gguf_first_block_fc1_fp16_flag(dev, ref, tmp_path, batch):
    """esm.first_block_fc1_fp16 = true (as the reference's writer stores it)
    turns the escape on: same logits as the directly created model with
    set_first_block_fc1_fp16(True)."""
    from pyoracle import RefModel
    w = _weights(True)
    p = str(tmp_path / "fp16.gguf")
    rm = RefModel(ref, w, int8=True, fc1_fp16=True)
    rm.save_gguf(p)
    rm.free()
    assert gguf.read_metadata(p)["esm.first_block_fc1_fp16"] is True
    direct = eg.Model(dev, w, int8=True)
    direct.set_first_block_fc1_fp16(True)
    want = direct.forward_packed(batch.ids, batch.cu)
    direct.free()
    loaded = eg.Model.from_gguf(dev, p)
    got = loaded.forward_packed(batch.ids, batch.cu)
    loaded.free()
    np.testing.assert_array_equal(got, want)
