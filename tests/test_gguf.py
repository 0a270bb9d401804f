"""esm.cpp GGUF files (reference src/io/gguf.cpp; names and metadata of
Model::SaveToGguf, src/model.cpp:562-700) on the CPU.

* The writer / reader round trips of the reference's own tests
  (tests/cpp/test_gguf.cpp:19-160): one FP32 tensor, metadata of every kind,
  several tensors, bad magic and wrong version rejected, an empty file.
* A model file from esm_gfx950.gguf.write_model read back by the
  reference's GgufFile::Open (compiled from source under oracle/_ref): the
  same tensors, types, dims and bytes, and the same metadata.
* A model file from the reference's GgufFile::Write (driven in SaveToGguf's
  order) read by esm_gfx950.gguf.read: every tensor equals the weights.
"""
import os

import numpy as np
import pytest

from esm_gfx950 import gguf
from esm_gfx950 import synthetic as syn


def test_fp32_single_tensor_round_trip(tmp_path):
    p = str(tmp_path / "one.gguf")
    t = np.arange(1, 7, dtype=np.float32)
    gguf.write(p, {"general.architecture": "test", "general.alignment": 32}, [("my_tensor", gguf.F32, (3, 2), t.tobytes())])
    meta, ts = gguf.read(p)
    ttype, dims, arr = ts["my_tensor"]
    assert ttype == gguf.F32 and dims == (3, 2)
    np.testing.assert_array_equal(arr, t)


def test_metadata_round_trips_across_types(tmp_path):
    p = str(tmp_path / "meta.gguf")
    meta = {"general.architecture": "esm", "general.alignment": 32, "esm.block_count": 6,
            "esm.attention.layer_norm_epsilon": 1.0e-5, "esm.token_dropout": True, "esm.dims": [320, 6, 20, 1280]}
    gguf.write(p, meta, [("dummy", gguf.F32, (1,), np.zeros(1, np.float32).tobytes())])
    got, _ = gguf.read(p)
    assert got == meta


def test_multiple_tensors_round_trip(tmp_path):
    p = str(tmp_path / "multi.gguf")
    a = np.arange(64, dtype=np.float32)
    b = -np.arange(128, dtype=np.float32)
    gguf.write(p, {"general.architecture": "test"},
               [("alpha", gguf.F32, (8, 8), a.tobytes()), ("beta", gguf.F32, (16, 8), b.tobytes())])
    _, ts = gguf.read(p)
    np.testing.assert_array_equal(ts["alpha"][2], a)
    np.testing.assert_array_equal(ts["beta"][2], b)


def test_rejects_bad_magic_and_wrong_version(tmp_path):
    p = str(tmp_path / "bad.gguf")
    with open(p, "wb") as f:
        f.write(b"NOTGGUFCONTENTSHERE\0")
    with pytest.raises(ValueError, match="bad magic"):
        gguf.read(p)
    with open(p, "wb") as f:
        f.write(b"GGUF" + np.array([2], np.uint32).tobytes() + np.zeros(2, np.uint64).tobytes())
    with pytest.raises(ValueError, match="version 2 not supported"):
        gguf.read(p)


def test_empty_tensors_and_metadata(tmp_path):
    p = str(tmp_path / "empty.gguf")
    gguf.write(p, {}, [])
    meta, ts = gguf.read(p)
    assert meta == {} and ts == {}


def _small_weights(int8):
    if int8:
        return syn.make_weights(syn.ESM2_8M.with_layers(2), seed=20261201 + 9, int8=True, keep_f32_linears=True)
    return syn.make_weights(syn.ESM2_8M.with_layers(2), seed=20261201 + 9, int8=False)


@pytest.mark.parametrize("int8", [False, True])
def test_writer_read_by_reference_reader(ref, tmp_path, int8):
    w = _small_weights(int8)
    p = str(tmp_path / "model.gguf")
    gguf.write_model(p, w, int8=int8)
    meta, ts = gguf.read(p)
    for name, (ttype, dims, arr) in ts.items():
        got = ref.gguf_tensor(p, name)
        raw = arr.tobytes() if ttype != gguf.Q8_ESM else arr[0].tobytes() + arr[1].tobytes()
        assert got == (ttype, dims, raw), name
    for key, value in meta.items():
        rv = ref.gguf_meta(p, key)
        if isinstance(value, str):
            assert rv == ("str", len(value)), key
        else:
            assert rv == value, key


@pytest.mark.parametrize("int8", [False, True])
def test_reference_writer_read_back(ref, tmp_path, int8):
    from pyoracle import RefModel
    w = _small_weights(int8)
    p = str(tmp_path / "ref.gguf")
    rm = RefModel(ref, w, int8=int8)
    rm.save_gguf(p)
    rm.free()
    meta, ts = gguf.read(p)
    assert meta["esm.weights_quantized"] is bool(int8)
    assert meta["esm.block_count"] == 2 and meta["esm.embedding_length"] == 320
    np.testing.assert_array_equal(ts["token_embd.weight"][2], w.f32["embed"].ravel())
    for i in range(2):
        for gname, wname in (("attn_q", "q"), ("attn_output", "out"), ("ffn_up", "fc1"), ("ffn_down", "fc2")):
            ttype, dims, arr = ts[f"blk.{i}.{gname}.weight"]
            if int8:
                q, s = w.i8[f"layers.{i}.{wname}"]
                assert ttype == gguf.Q8_ESM and dims == (q.shape[1], q.shape[0])
                np.testing.assert_array_equal(arr[0], q)
                np.testing.assert_array_equal(arr[1], s)
            else:
                W = w.f32[f"layers.{i}.{wname}.weight"]
                assert ttype == gguf.F32 and dims == (W.shape[1], W.shape[0])
                np.testing.assert_array_equal(arr, W.ravel())
    np.testing.assert_array_equal(ts["output.bias"][2], w.f32["lm_head.decoder.bias"])
