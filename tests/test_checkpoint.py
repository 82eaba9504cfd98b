"""The checkpoint reader (CPU): safetensors files written by the safetensors
package (an independent writer) read back exactly; quantization configs of
both families; a layer read from a file repacks to the oracle's result; and
the reader's refusals."""
import json
import os
import struct

import numpy as np
import pytest
from safetensors.numpy import save_file

import accel_amd
import oracle
from accel_amd import checkpoint
from oracle import foreign_np

AWQ, GPTQ, GPTQ2 = accel_amd.QFMT_AWQ, accel_amd.QFMT_GPTQ, accel_amd.QFMT_GPTQ_V2


def test_read_safetensors_matches_the_writer(tmp_path):
    rng = np.random.default_rng(1)
    tensors = {
        "a.qweight": rng.integers(-2**31, 2**31 - 1, (16, 4), dtype=np.int32),
        "a.scales": rng.standard_normal((2, 32)).astype(np.float16),
        "b": rng.standard_normal(7).astype(np.float32),
        "c": np.arange(5, dtype=np.int64),
        "scalar": np.array(3.0, np.float32),
    }
    path = str(tmp_path / "m.safetensors")
    save_file(tensors, path, metadata={"format": "pt"})
    got = checkpoint.read_safetensors(path)
    assert set(got) == set(tensors)
    for k, v in tensors.items():
        assert got[k].dtype == v.dtype and got[k].shape == v.shape and np.array_equal(got[k], v)


def test_read_safetensors_refuses_a_broken_file(tmp_path):
    p = tmp_path / "bad.safetensors"
    p.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    with pytest.raises(checkpoint.CheckpointError, match="header of"):
        checkpoint.read_safetensors(str(p))
    header = json.dumps({"x": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}).encode()
    p.write_bytes(struct.pack("<Q", len(header)) + header + b"\0" * 8)
    with pytest.raises(checkpoint.CheckpointError, match="spans"):
        checkpoint.read_safetensors(str(p))
    header = json.dumps({"x": {"dtype": "F8_E4M3", "shape": [1], "data_offsets": [0, 1]}}).encode()
    p.write_bytes(struct.pack("<Q", len(header)) + header + b"\0")
    with pytest.raises(checkpoint.CheckpointError, match="dtype"):
        checkpoint.read_safetensors(str(p))
    for bad, text in ((b"[1, 2]", "not a JSON object"),
                      (json.dumps({"x": 3}).encode(), "malformed header entry"),
                      (json.dumps({"x": {"dtype": "F32", "shape": [1]}}).encode(),
                       "malformed shape"),
                      (json.dumps({"x": {"dtype": "F32", "shape": [-1],
                                         "data_offsets": [0, 0]}}).encode(), "shape")):
        p.write_bytes(struct.pack("<Q", len(bad)) + bad + b"\0" * 4)
        with pytest.raises(checkpoint.CheckpointError, match=text):
            checkpoint.read_safetensors(str(p))


@pytest.mark.parametrize("cfg,fmt,group", [
    ({"quantization_config": {"quant_method": "awq", "bits": 4, "group_size": 128,
                              "version": "gemm", "zero_point": True}}, AWQ, 128),
    ({"w_bit": 4, "q_group_size": 64, "version": "GEMM", "zero_point": True}, AWQ, 64),
    ({"quant_method": "gptq", "bits": 4, "group_size": 128, "desc_act": True}, GPTQ, 128),
    ({"quantization_config": {"quant_method": "gptq", "bits": 4, "group_size": -1,
                              "checkpoint_format": "gptq_v2"}}, GPTQ2, -1),
])
def test_quant_config(cfg, fmt, group):
    q = checkpoint.quant_config(cfg)
    assert q.format == fmt and q.group_size == group


@pytest.mark.parametrize("cfg,text", [
    ({"quant_method": "gptq", "bits": 8}, "8-bit"),
    ({"quant_method": "awq", "version": "gemv"}, "gemm"),
    ({"quant_method": "awq", "zero_point": False}, "zero points"),
    ({"quant_method": "gptq", "checkpoint_format": "marlin"}, "marlin"),
    ({"quant_method": "bitsandbytes"}, "neither awq nor gptq"),
])
def test_quant_config_refusals(cfg, text):
    with pytest.raises(checkpoint.CheckpointError, match=text):
        checkpoint.quant_config(cfg)


def _write_layer(tmp_path, fmt, K, N, G, act=False, sharded=False):
    rng = np.random.default_rng(fmt + K + N)
    groups = -(-K // G)
    q = rng.integers(0, 16, (K, N))
    z = rng.integers(1, 16, (groups, N))
    s = (rng.random((groups, N)) * 0.01 + 1e-3).astype(np.float16)
    if fmt == AWQ:
        qw, qz = foreign_np.pack_awq(q, z)
    else:
        qw, qz = foreign_np.pack_gptq(q, z, v2=fmt == GPTQ2)
    t = {"model.layers.0.mlp.up_proj.qweight": qw.view(np.int32),
         "model.layers.0.mlp.up_proj.qzeros": qz.view(np.int32),
         "model.layers.0.mlp.up_proj.scales": s}
    g_idx = None
    if fmt != AWQ:
        g_idx = (np.arange(K) // G).astype(np.int32)
        if act:
            rng.shuffle(g_idx)
        t["model.layers.0.mlp.up_proj.g_idx"] = g_idx
    d = tmp_path / f"ckpt{fmt}{int(act)}{int(sharded)}"
    d.mkdir()
    if sharded:
        names = sorted(t)
        a, b = names[:2], names[2:]
        save_file({k: t[k] for k in a}, str(d / "model-00001-of-00002.safetensors"))
        save_file({k: t[k] for k in b}, str(d / "model-00002-of-00002.safetensors"))
        wm = {k: "model-00001-of-00002.safetensors" for k in a}
        wm.update({k: "model-00002-of-00002.safetensors" for k in b})
        (d / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wm}))
    else:
        save_file(t, str(d / "model.safetensors"))
    qc = {"quant_method": "awq" if fmt == AWQ else "gptq", "bits": 4, "group_size": G}
    if fmt == GPTQ2:
        qc["checkpoint_format"] = "gptq_v2"
    (d / "config.json").write_text(json.dumps({"quantization_config": qc}))
    return str(d), qw, qz, s.view(np.uint16), g_idx if act else None


@pytest.mark.parametrize("fmt,act,sharded", [(AWQ, False, False), (GPTQ, False, True),
                                             (GPTQ, True, False), (GPTQ2, True, True)])
def test_a_layer_read_from_a_file_repacks_to_the_oracle(tmp_path, fmt, act, sharded):
    K, N, G = 256, 128, 64
    path, qw, qz, s, g_idx = _write_layer(tmp_path, fmt, K, N, G, act, sharded)
    cfg = checkpoint.quant_config(path)
    lay = checkpoint.layer(checkpoint.open_checkpoint(path), "model.layers.0.mlp.up_proj", cfg)
    assert (lay.K, lay.N, lay.group_size) == (K, N, G)
    # an in-order g_idx is dropped; an act-order one is kept
    assert (lay.g_idx is not None) == act
    want = oracle.int4_repack(fmt, K, N, G, qw, qz, s, g_idx)
    for a, b in zip(accel_amd.int4_repack_host(lay), want):
        assert np.array_equal(a, b)


def test_layer_refusals(tmp_path):
    path, *_ = _write_layer(tmp_path, GPTQ, 64, 16, 32)
    t = checkpoint.open_checkpoint(path)
    cfg = checkpoint.quant_config(path)
    with pytest.raises(checkpoint.CheckpointError, match="no qweight"):
        checkpoint.layer(t, "model.layers.1.mlp.up_proj", cfg)
    bad = dict(t)
    bad["model.layers.0.mlp.up_proj.scales"] = np.zeros((2, 16), np.float32)
    with pytest.raises(checkpoint.CheckpointError, match="store f16"):
        checkpoint.layer(bad, "model.layers.0.mlp.up_proj", cfg)
    bad = dict(t)
    bad["model.layers.0.mlp.up_proj.qzeros"] = np.zeros((2, 3), np.int32)
    with pytest.raises(checkpoint.CheckpointError, match="do not describe one"):
        checkpoint.layer(bad, "model.layers.0.mlp.up_proj", cfg)
