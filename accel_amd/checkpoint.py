"""Reading published 4-bit checkpoints (AWQ, GPTQ) into the reference int4
format.

The reference names this as the unbuilt next step of its int4 format
(specs/048-int4.md:126-131,167: "the representation is theirs; the file
format, its permutation of columns, and its packing order are not").  This
module is the file side: a safetensors reader (memory-mapped, no code executed
from the file), the quantization config of a checkpoint (``config.json``'s
``quantization_config``, or ``quantize_config.json`` / ``quant_config.json``),
and the per-layer planes.  The repack itself is the library's
(``accel_int4_repack`` on the device, ``accel_int4_repack_host`` on the host).
"""
from __future__ import annotations

import json
import os
import struct
from dataclasses import dataclass

import numpy as np

from . import QFMT_AWQ, QFMT_GPTQ, QFMT_GPTQ_V2, ForeignInt4

_DTYPES = {
    "BOOL": np.bool_, "U8": np.uint8, "I8": np.int8, "U16": np.uint16, "I16": np.int16,
    "F16": np.float16, "BF16": np.uint16, "U32": np.uint32, "I32": np.int32,
    "F32": np.float32, "U64": np.uint64, "I64": np.int64, "F64": np.float64,
}
_MAX_HEADER = 100 << 20


class CheckpointError(ValueError):
    """A checkpoint this reader cannot use, with the reason."""


def read_safetensors(path: str) -> dict:
    """The tensors of a safetensors file as read-only memory-mapped arrays
    (BF16 as its u16 bits).  The format: an 8-byte little-endian header
    length, a JSON header mapping names to dtype, shape and data offsets, then
    the data."""
    size = os.path.getsize(path)
    with open(path, "rb") as f:
        raw = f.read(8)
        if len(raw) != 8:
            raise CheckpointError(f"{path}: shorter than a safetensors header")
        n = struct.unpack("<Q", raw)[0]
        if n > _MAX_HEADER or 8 + n > size:
            raise CheckpointError(f"{path}: header of {n} bytes in a {size}-byte file")
        try:
            header = json.loads(f.read(n))
        except ValueError as e:
            raise CheckpointError(f"{path}: header is not JSON ({e})") from None
    data_bytes = size - 8 - n
    mm = np.memmap(path, np.uint8, mode="r", offset=8 + n, shape=(data_bytes,)) \
        if data_bytes else np.zeros(0, np.uint8)
    if not isinstance(header, dict):
        raise CheckpointError(f"{path}: header is not a JSON object")
    out = {}
    for name, info in header.items():
        if name == "__metadata__":
            continue
        if not isinstance(info, dict):
            raise CheckpointError(f"{path}: tensor {name} has a malformed header entry")
        dt = _DTYPES.get(info.get("dtype"))
        if dt is None:
            raise CheckpointError(f"{path}: tensor {name} has dtype {info.get('dtype')!r}")
        try:
            shape = tuple(int(d) for d in info["shape"])
            b, e = (int(v) for v in info["data_offsets"])
        except (KeyError, TypeError, ValueError):
            raise CheckpointError(f"{path}: tensor {name} has a malformed shape or "
                                  "data_offsets") from None
        if any(d < 0 for d in shape):
            raise CheckpointError(f"{path}: tensor {name} has shape {shape}")
        count = int(np.prod(shape, dtype=np.int64)) if shape else 1
        if not 0 <= b <= e <= data_bytes or e - b != count * np.dtype(dt).itemsize:
            raise CheckpointError(f"{path}: tensor {name} spans [{b}, {e}) for {count} "
                                  f"{info['dtype']} values in {data_bytes} data bytes")
        out[name] = mm[b:e].view(dt).reshape(shape)
    return out


@dataclass
class QuantConfig:
    """What a checkpoint says about its 4-bit layers."""
    format: int          # QFMT_AWQ, QFMT_GPTQ or QFMT_GPTQ_V2
    group_size: int      # input rows a group spans; -1 for the whole of K
    desc_act: bool = False


def quant_config(src) -> QuantConfig:
    """The quantization config of a checkpoint directory, a JSON file, or a
    dict already read.  AWQ: ``quant_method`` "awq" (or AutoAWQ's
    ``w_bit``/``q_group_size``/``version`` keys), version "gemm".  GPTQ:
    ``quant_method`` "gptq", ``checkpoint_format`` "gptq" (zeros stored z - 1)
    or "gptq_v2".  Only 4-bit layers with zero points are read."""
    if isinstance(src, dict):
        cfg = src
    else:
        path = src
        if os.path.isdir(src):
            for name in ("quantize_config.json", "quant_config.json", "config.json"):
                if os.path.exists(os.path.join(src, name)):
                    path = os.path.join(src, name)
                    break
            else:
                raise CheckpointError(f"{src}: no quantize_config.json, quant_config.json or "
                                      "config.json")
        with open(path) as f:
            cfg = json.load(f)
    cfg = cfg.get("quantization_config", cfg)
    method = str(cfg.get("quant_method", "awq" if "w_bit" in cfg else "")).lower()
    bits = int(cfg.get("bits", cfg.get("w_bit", 4)))
    group = int(cfg.get("group_size", cfg.get("q_group_size", 128)))
    if bits != 4:
        raise CheckpointError(f"the checkpoint has {bits}-bit layers; the reference format is "
                              "4-bit")
    if method == "awq":
        version = str(cfg.get("version", "gemm")).lower()
        if version != "gemm":
            raise CheckpointError(f"AWQ version {version!r}: only the \"gemm\" packing is read")
        if cfg.get("zero_point", True) is False:
            raise CheckpointError("AWQ without zero points is not read")
        return QuantConfig(QFMT_AWQ, group)
    if method == "gptq":
        fmt = str(cfg.get("checkpoint_format", "gptq")).lower()
        if fmt not in ("gptq", "gptq_v2"):
            raise CheckpointError(f"GPTQ checkpoint_format {fmt!r}: only \"gptq\" and "
                                  "\"gptq_v2\" are read")
        return QuantConfig(QFMT_GPTQ if fmt == "gptq" else QFMT_GPTQ_V2, group,
                           bool(cfg.get("desc_act", False)))
    raise CheckpointError(f"quant_method {method!r} is neither awq nor gptq")


def layer(tensors: dict, prefix: str, cfg: QuantConfig) -> ForeignInt4:
    """The planes of one linear layer (``<prefix>.qweight``, ``.qzeros``,
    ``.scales`` and, for GPTQ, ``.g_idx``).  Shapes: AWQ qweight [K, N/8],
    GPTQ qweight [K/8, N]; qzeros [groups, N/8]; scales f16 [groups, N]."""
    def get(key):
        t = tensors.get(f"{prefix}.{key}")
        if t is None:
            raise CheckpointError(f"{prefix}: no {key} tensor")
        return t

    qweight, qzeros, scales = get("qweight"), get("qzeros"), get("scales")
    for name, t in (("qweight", qweight), ("qzeros", qzeros), ("scales", scales)):
        if t.ndim != 2:
            raise CheckpointError(f"{prefix}.{name} has shape {t.shape}; it is a matrix")
    if qweight.dtype.itemsize != 4 or qzeros.dtype.itemsize != 4:
        raise CheckpointError(f"{prefix}: qweight and qzeros are {qweight.dtype} and "
                              f"{qzeros.dtype}; both formats pack into 32-bit words")
    if scales.dtype != np.float16:
        raise CheckpointError(f"{prefix}.scales is {scales.dtype}; the formats read store f16")
    if cfg.format == QFMT_AWQ:
        K, N = qweight.shape[0], qweight.shape[1] * 8
    else:
        K, N = qweight.shape[0] * 8, qweight.shape[1]
    if scales.shape[1] != N or qzeros.shape[1] * 8 != N or qzeros.shape[0] != scales.shape[0]:
        raise CheckpointError(f"{prefix}: qweight {qweight.shape}, qzeros {qzeros.shape} and "
                              f"scales {scales.shape} do not describe one [{K}, {N}] layer")
    g_idx = None
    if cfg.format != QFMT_AWQ and f"{prefix}.g_idx" in tensors:
        g_idx = np.asarray(tensors[f"{prefix}.g_idx"]).astype(np.int32)
        if g_idx.shape != (K,):
            raise CheckpointError(f"{prefix}.g_idx has shape {g_idx.shape}; it is [{K}]")
    group = cfg.group_size if cfg.group_size > 0 else K
    if g_idx is not None and np.array_equal(g_idx, np.arange(K, dtype=np.int32) // group):
        g_idx = None   # rows in order: the plain k / group_size grouping
    return ForeignInt4(cfg.format, group, K, N, np.asarray(qweight), np.asarray(qzeros),
                       np.asarray(scales).view(np.uint16), g_idx)


def open_checkpoint(path: str) -> dict:
    """All tensors of a checkpoint: one safetensors file, or a directory with
    ``model.safetensors`` or a sharded ``model.safetensors.index.json``."""
    if os.path.isfile(path):
        return read_safetensors(path)
    index = os.path.join(path, "model.safetensors.index.json")
    if os.path.exists(index):
        with open(index) as f:
            weight_map = json.load(f)["weight_map"]
        out = {}
        for shard in sorted(set(weight_map.values())):
            out.update(read_safetensors(os.path.join(path, shard)))
        return out
    single = os.path.join(path, "model.safetensors")
    if os.path.exists(single):
        return read_safetensors(single)
    raise CheckpointError(f"{path}: no model.safetensors or model.safetensors.index.json")


def load_linear(dev, path: str, prefix: str, cfg: QuantConfig = None):
    """One published layer of a checkpoint, repacked on `dev` into the
    reference int4 format: (Int4Weights, K, N)."""
    cfg = cfg or quant_config(path if os.path.isdir(path) else os.path.dirname(path))
    lay = layer(open_checkpoint(path), prefix, cfg)
    return dev.Int4Repack(lay), lay.K, lay.N
