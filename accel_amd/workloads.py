"""Synthetic inputs of the benchmark configurations.

Each generator draws from numpy ``Generator(PCG64(seed))``: activations
first, then the weight as [out, in] ~ N(0, 0.02) cast to f32, then (for the
mixture of experts) the routing logits.  The weight is transposed to the
reference layout [K=in, N=out] before packing, so element (k, n) is
``k*N + n`` as tensor/int4.go:82 indexes it, and packed with this library's
host quantizer (quant.Int4Quantize's format: 128-weight groups, f16 scale and
zero, eight nibbles per u32, low nibble first).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass
class Linear:
    """One int4 linear product's host inputs."""
    x: np.ndarray          # f32 [M, K] (bf16 configs: already rounded to bf16)
    w: np.ndarray          # f32 [K, N], unquantized
    packed: np.ndarray     # u32 [K*N/8]
    scales: np.ndarray     # f16 bits [K*N/128]
    zeros: np.ndarray      # f16 bits [K*N/128]
    M: int
    K: int
    N: int
    bf16: bool


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bits, round to nearest even (NaN to 0x7fc0)."""
    b = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(np.isnan(x), np.uint16(0x7FC0), r).astype(np.uint16)


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def linear(M: int, K: int, N: int, seed: int, bf16: bool = False,
           wscale: float = 0.02) -> Linear:
    import accel_amd
    rng = np.random.Generator(np.random.PCG64(seed))
    x = rng.standard_normal((M, K)).astype(np.float32)
    w_out_in = (rng.standard_normal((N, K)) * wscale).astype(np.float32)
    w = np.ascontiguousarray(w_out_in.T)
    if bf16:
        x = bf16_to_f32(bf16_bits(x))
    packed, scales, zeros = accel_amd.int4_quantize(w)
    return Linear(x, w, packed, scales, zeros, M, K, N, bf16)


# BASELINE.json configs, in the reference format (G=128, f16 scale + zero).
CONFIGS = {
    "gemv_m1": dict(M=1, K=4096, N=4096, seed=0, bf16=False),
    "decode_m16": dict(M=16, K=4096, N=14336, seed=1, bf16=False),
    "prefill_m2048": dict(M=2048, K=4096, N=4096, seed=2, bf16=True),
    # config 3's shape in the reference API's own dtype (f32 activations)
    "prefill_m2048_f32": dict(M=2048, K=4096, N=4096, seed=2, bf16=False),
    # a short prefill (M >= 64 is the batched-GEMM range): too few tiles to
    # fill the chip, so the products split K
    "prefill_m64": dict(M=64, K=4096, N=4096, seed=2, bf16=True),
    "prefill_m64_f32": dict(M=64, K=4096, N=4096, seed=2, bf16=False),
}


@dataclass
class MoE:
    x: np.ndarray          # f32 values of the bf16 routed rows [R, K], sorted by expert
    counts: np.ndarray     # u32 [E]
    packed: np.ndarray     # stacked [E, K, N] int4 planes
    scales: np.ndarray
    zeros: np.ndarray
    E: int
    K: int
    N: int
    tokens: int
    order: np.ndarray      # routed row -> source token


def moe(tokens: int = 512, E: int = 8, top: int = 2, K: int = 4096, N: int = 14336,
        seed: int = 3) -> MoE:
    """Config 4: top-2 of a seeded softmax over N(0,1) logits (lower expert
    index wins ties), rows sorted by expert, stable by token."""
    import accel_amd
    rng = np.random.Generator(np.random.PCG64(seed))
    x = rng.standard_normal((tokens, K)).astype(np.float32)
    x = bf16_to_f32(bf16_bits(x))
    ws = []
    for _ in range(E):
        w_out_in = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        ws.append(np.ascontiguousarray(w_out_in.T))
    logits = rng.standard_normal((tokens, E))
    p = np.exp(logits - logits.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    chosen = np.argsort(-p, axis=1, kind="stable")[:, :top]
    pairs = sorted(((int(e), t) for t in range(tokens) for e in chosen[t]))
    order = np.array([t for _, t in pairs], np.int64)
    experts = np.array([e for e, _ in pairs], np.int64)
    counts = np.bincount(experts, minlength=E).astype(np.uint32)
    stacked = np.concatenate([w.ravel() for w in ws])
    packed, scales, zeros = accel_amd.int4_quantize(stacked)
    return MoE(x[order], counts, packed, scales, zeros, E, K, N, tokens, order)


def algorithmic_bytes(M: int, K: int, N: int, act_bytes: int = 4, out_bytes: int = 4) -> int:
    """Bytes one product must move: codes + f16 scale/zero + activations + output."""
    return K * N // 2 + 4 * (K * N // 128) + act_bytes * M * K + out_bytes * M * N


# Config 5: one Llama-3-8B-shaped decoder layer's seven projections, (K, N)
# in the reference layout [K=in, N=out].
LAYER_SHAPES = {
    "q": (4096, 4096), "k": (4096, 1024), "v": (4096, 1024), "o": (4096, 4096),
    "gate": (4096, 14336), "up": (4096, 14336), "down": (14336, 4096),
}


def fast_int4(K: int, N: int, rng) -> tuple:
    """Packed int4 planes of a [K, N] ~ N(0, 0.02) weight drawn in float32
    (benchmark inputs: fast to make, not the parity fixtures' f64 draw)."""
    import accel_amd
    w = rng.standard_normal((K, N), dtype=np.float32) * np.float32(0.02)
    return accel_amd.int4_quantize(w)


def moe_fast(tokens: int = 512, E: int = 8, top: int = 2, K: int = 4096, N: int = 14336,
             seed: int = 3) -> MoE:
    """Config 4's shape with float32 draws (benchmark inputs): top-2 routing of
    a seeded softmax, rows sorted by expert, stable by token."""
    import accel_amd
    rng = np.random.Generator(np.random.PCG64(seed))
    x = rng.standard_normal((tokens, K), dtype=np.float32)
    x = bf16_to_f32(bf16_bits(x))
    planes = [fast_int4(K, N, rng) for _ in range(E)]
    logits = rng.standard_normal((tokens, E))
    p = np.exp(logits - logits.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    chosen = np.argsort(-p, axis=1, kind="stable")[:, :top]
    pairs = sorted(((int(e), t) for t in range(tokens) for e in chosen[t]))
    order = np.array([t for _, t in pairs], np.int64)
    experts = np.array([e for e, _ in pairs], np.int64)
    counts = np.bincount(experts, minlength=E).astype(np.uint32)
    packed = np.concatenate([pl[0] for pl in planes])
    scales = np.concatenate([pl[1] for pl in planes])
    zeros = np.concatenate([pl[2] for pl in planes])
    return MoE(x[order], counts, packed, scales, zeros, E, K, N, tokens, order)
