"""Reading compressed-tensors checkpoints (src/checkpoint.rs:129-180, :196-453): the quantization_config scheme and
quantized matrices from safetensors files on disk."""

import json

import numpy as np
import pytest

import oracle
from qwenny_amd import synth
from qwenny_amd.checkpoint import Checkpoint, packed_scheme, quant_from_packed, save_safetensors


def _qc(bits=4, strategy="group", group=128, act=None, actorder=None, fmt="pack-quantized", typ="int"):
    w = {"num_bits": bits, "type": typ, "strategy": strategy, "group_size": group if strategy == "group" else None,
         "symmetric": True, "actorder": actorder}
    return {"format": fmt, "config_groups": {"group_0": {"weights": w, "input_activations": act}}}


def test_scheme():
    assert packed_scheme(_qc()) == (4, 128)
    assert packed_scheme(_qc(bits=8, strategy="channel")) == (8, 0)
    assert packed_scheme(_qc(actorder="static")) == (4, 128)
    for bad in (_qc(fmt="naive-quantized"), _qc(bits=3), _qc(typ="float"), _qc(strategy="tensor"),
                _qc(act={"num_bits": 8}), _qc(actorder="group")):
        with pytest.raises(ValueError):
            packed_scheme(bad)
    two = _qc()
    two["config_groups"]["group_1"] = _qc(bits=8, group=64)["config_groups"]["group_0"]
    with pytest.raises(ValueError):  # different group sizes
        packed_scheme(two)


def _write_ckpt(tmp_path, prefix="", scale_dtype="BF16"):
    a = synth.int4_quant(1, "a", 64, 256, zp=True)
    b = synth.int4_quant(2, "b", 32, 256)
    tensors = {}
    for name, t in (("model.layers.0.mlp.gate_proj", a), ("model.layers.0.mlp.up_proj", b)):
        tensors[f"{prefix}{name}.weight_packed"] = ("I32", t["weight_packed"].view(np.int32))
        sc = t["weight_scale"]
        if scale_dtype == "F16":
            tensors[f"{prefix}{name}.weight_scale"] = ("F16", synth.bf16_to_f32(sc).astype(np.float16).view(np.uint16))
        else:
            tensors[f"{prefix}{name}.weight_scale"] = ("BF16", sc)
        tensors[f"{prefix}{name}.weight_shape"] = ("I64", t["weight_shape"])
        if "weight_zero_point" in t:
            tensors[f"{prefix}{name}.weight_zero_point"] = ("I32", t["weight_zero_point"].view(np.int32))
    save_safetensors(str(tmp_path / "model.safetensors"), tensors)
    (tmp_path / "config.json").write_text(json.dumps({"quantization_config": _qc()}))
    return a, b


@pytest.mark.parametrize("prefix", ["", "language_model."])
def test_checkpoint_quant_matrix(tmp_path, prefix):
    a, _ = _write_ckpt(tmp_path, prefix)
    ck = Checkpoint(str(tmp_path))
    base = "model.layers.0.mlp.gate_proj"
    assert ck.is_quant(base) and ck.prequantized()
    q = ck.quant_matrix(base)
    assert (q.bits, q.group, q.rows, q.cols) == (4, 128, 64, 256)
    sc = synth.bf16_to_f32(a["weight_scale"])
    _, _, _, osc, ooff = oracle.packed_matrix(a["weight_packed"], sc, 4, 128, zero_point=a["weight_zero_point"])
    assert np.array_equal(q.scales, osc) and np.array_equal(q.offsets, ooff)
    assert np.array_equal(q.q, a["weight_packed"])


def test_checkpoint_f16_scales(tmp_path):
    _, b = _write_ckpt(tmp_path, scale_dtype="F16")
    q = Checkpoint(str(tmp_path)).quant_matrix("model.layers.0.mlp.up_proj")
    want = synth.bf16_to_f32(b["weight_scale"]).astype(np.float16).astype(np.float32).reshape(-1)
    assert np.array_equal(q.scales, want)
    assert (q.zero_points() == 8).all()


def test_quant_from_packed_errors():
    w = np.zeros((4, 2), np.uint32)
    with pytest.raises(Exception):
        quant_from_packed(w, np.ones(8, np.float32), 4, 128, weight_shape=np.array([5, 16]))
    with pytest.raises(Exception):  # 16 columns in groups of 128
        quant_from_packed(w, np.ones(8, np.float32), 4, 128)
