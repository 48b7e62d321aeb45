"""Synthetic workloads of the bench configs, generated through the C ABI
(cpb_synth_*) so the host here, the GPU box and every test produce identical
bytes from (seed, layer).

Distributions:
  MXFP4 codes uniform over 16 values, e8m0 = 127 + U{-6..-3};
  expert biases N(0, 0.01); router N(0, 0.02), bias 0 (config 0) or
  Zipf(1.1) over a seeded expert permutation (stacks); input x N(0, 1);
  Q4_K / Q6_K bytes uniform, fp16 d/dmin ~ |N(0, 0.01)|.
The reference reads real GGUF weights instead; there is no network for
model files here.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import f32p, lib, u8p

# stream ids per tensor (stream = layer * 16 + id)
_GATE, _UP, _DOWN, _GB, _UB, _DB, _RW, _RB, _X = range(9)


def _stream(layer: int, tid: int) -> int:
    return layer * 16 + tid


def mxfp4(n_rows: int, nb: int, seed: int, stream: int, e_lo: int = 121, e_span: int = 4) -> np.ndarray:
    out = np.empty((n_rows, nb * 17), np.uint8)
    lib().cpb_synth_mxfp4(out.ctypes.data_as(u8p), n_rows * nb, e_lo, e_span, seed, stream)
    return out


def normal(shape, sigma: float, seed: int, stream: int, mean: float = 0.0) -> np.ndarray:
    out = np.empty(shape, np.float32)
    lib().cpb_synth_normal(out.ctypes.data_as(f32p), out.size, mean, sigma, seed, stream)
    return out


def q4k(n_rows: int, cols: int, seed: int, stream: int, dsig: float = 0.01) -> np.ndarray:
    out = np.empty((n_rows, cols // 256 * 144), np.uint8)
    lib().cpb_synth_q4k(out.ctypes.data_as(u8p), n_rows * (cols // 256), dsig, seed, stream)
    return out


def q6k(n_rows: int, cols: int, seed: int, stream: int, dsig: float = 0.01) -> np.ndarray:
    out = np.empty((n_rows, cols // 256 * 210), np.uint8)
    lib().cpb_synth_q6k(out.ctypes.data_as(u8p), n_rows * (cols // 256), dsig, seed, stream)
    return out


def zipf_bias(ne: int, s: float, seed: int, stream: int) -> np.ndarray:
    out = np.empty(ne, np.float32)
    lib().cpb_synth_zipf_bias(out.ctypes.data_as(f32p), ne, s, seed, stream)
    return out


def gptoss_layer(d: int, dff: int, ne: int, k: int, seed: int = 0, layer: int = 0, zipf: float | None = None,
                 e_lo: int = 121, e_span: int = 4) -> dict:
    """One gpt-oss-shaped MoE layer in native GGUF layouts (dict of numpy arrays)."""
    nb, nbf = d // 32, dff // 32
    L = {
        "d": d, "dff": dff, "ne": ne, "k": k, "alpha": 1.702, "limit": 7.0, "eps": 1e-5,
        "gate": mxfp4(ne * dff, nb, seed, _stream(layer, _GATE), e_lo, e_span),
        "up": mxfp4(ne * dff, nb, seed, _stream(layer, _UP), e_lo, e_span),
        "down": mxfp4(ne * d, nbf, seed, _stream(layer, _DOWN), e_lo, e_span),
        "gate_b": normal((ne, dff), 0.01, seed, _stream(layer, _GB)),
        "up_b": normal((ne, dff), 0.01, seed, _stream(layer, _UB)),
        "down_b": normal((ne, d), 0.01, seed, _stream(layer, _DB)),
        "router_w": normal((ne, d), 0.02, seed, _stream(layer, _RW)),
        "router_b": (zipf_bias(ne, zipf, seed, _stream(layer, _RB)) if zipf else np.zeros(ne, np.float32)),
        "norm_w": np.ones(d, np.float32),
    }
    return L


def qwen_layer(d: int, dff: int, ne: int, k: int, seed: int = 0, layer: int = 0, down_type: int = 14) -> dict:
    """One Qwen3-30B-A3B-shaped MoE layer: Q4_K gate/up, Q6_K (or Q4_K) down,
    no biases (the reference's Qwen router has none, engine_qwen2.rs:400)."""
    L = {
        "d": d, "dff": dff, "ne": ne, "k": k, "nt": 12, "eps": 1e-6,
        "gate_type": 12, "up_type": 12, "down_type": down_type,
        "gate": q4k(ne * dff, d, seed, _stream(layer, _GATE)),
        "up": q4k(ne * dff, d, seed, _stream(layer, _UP)),
        "down": (q6k if down_type == 14 else q4k)(ne * d, dff, seed, _stream(layer, _DOWN)),
        "router_w": normal((ne, d), 0.02, seed, _stream(layer, _RW)),
        "norm_w": np.ones(d, np.float32),
    }
    return L


def token(d: int, seed: int = 0, index: int = 0) -> np.ndarray:
    """fp32 N(0,1) activation (config 0 feeds it as the input after RMSNorm)."""
    return normal(d, 1.0, seed, 1_000_000 + index)


def bf16(a: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest even (the GGUF BF16 tensor type)."""
    b = np.asarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return (((b + 0x7FFF + ((b >> 16) & 1)) >> 16) & 0xFFFF).astype(np.uint16)


def attn_layer(d: int, nh: int, nkv: int, hd: int, seed: int = 0, layer: int = 0, swa: int = 128) -> dict:
    """One gpt-oss attention block: bf16 q/k/v/o weights N(0, 0.02), fp32
    biases N(0, 0.01), sinks N(0, 1), attn_norm near 1 (the reference loads
    these from the GGUF: attn_q/k/v/out.weight BF16, .bias, attn_sinks,
    attn_norm, engine_gpt2.rs:1293-1305)."""
    base = 1_000 + layer * 16
    return {
        "d": d, "nh": nh, "nkv": nkv, "hd": hd, "swa": swa, "eps": 1e-5,
        "attn_norm": 1.0 + normal(d, 0.05, seed, base + 0),
        "wq": bf16(normal((nh * hd, d), 0.02, seed, base + 1)),
        "wk": bf16(normal((nkv * hd, d), 0.02, seed, base + 2)),
        "wv": bf16(normal((nkv * hd, d), 0.02, seed, base + 3)),
        "wo": bf16(normal((d, nh * hd), 0.02, seed, base + 4)),
        "bq": normal(nh * hd, 0.01, seed, base + 5),
        "bk": normal(nkv * hd, 0.01, seed, base + 6),
        "bv": normal(nkv * hd, 0.01, seed, base + 7),
        "bo": normal(d, 0.01, seed, base + 8),
        "sinks": normal(nh, 1.0, seed, base + 9),
    }
