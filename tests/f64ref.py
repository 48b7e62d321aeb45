"""Independent float64 references used to pin the oracle (numpy only).

These follow published format definitions, not the oracle's code:
  - MXFP4 (OCP Microscaling Formats v1.0): element = E2M1(code) * 2^(e-127),
    E2M1 = {0, .5, 1, 1.5, 2, 3, 4, 6} with a sign bit; GGUF block layout
    [e8m0][16 bytes], element j<16 = low nibble of byte j, 16+j = high nibble.
    (The reference's scripts/ffn_reference.py:23-33 computes the same with a
    doubled table and a 2^(e-127) scale, i.e. 2x too large; this uses the
    corrected form, equivalent to doubled table * 2^(e-128).)
  - Q4_K / Q6_K: ggml's dequantize_row_q4_K / q6_K definitions (superblock
    formats as documented in the reference's qk_verify.rs:47-100).
  - The gpt-oss MoE layer math of scripts/ffn_reference.py:2-9, 52-62.
"""
from __future__ import annotations

import numpy as np

E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], np.float64)
E2M1_SIGNED = np.concatenate([E2M1, -E2M1])


def e2m1_codes(blocks: np.ndarray) -> np.ndarray:
    """[..., 17] GGUF blocks -> [..., 32] 4-bit codes in element order."""
    qs = blocks[..., 1:17]
    return np.concatenate([qs & 0xF, qs >> 4], axis=-1)


def deq_mxfp4(rows: np.ndarray, cols: int) -> np.ndarray:
    """[n, cols/32*17] uint8 -> [n, cols] float64."""
    nb = cols // 32
    blk = rows.reshape(rows.shape[0], nb, 17)
    vals = E2M1_SIGNED[e2m1_codes(blk)]                                   # [n, nb, 32]
    scale = np.exp2(blk[..., 0].astype(np.float64) - 127.0)               # OCP e8m0
    return (vals * scale[..., None]).reshape(rows.shape[0], cols)


def mx_block_sums(row: np.ndarray, xq: np.ndarray) -> np.ndarray:
    """Exact int block sums sum(2*E2M1(c) * xq) per 32-block (int64)."""
    nb = xq.size // 32
    blk = row.reshape(nb, 17)
    w2 = (2 * E2M1_SIGNED[e2m1_codes(blk)]).astype(np.int64)              # doubled values, exact ints
    return (w2 * xq.reshape(nb, 32).astype(np.int64)).sum(axis=1)


def half(h: np.ndarray) -> np.ndarray:
    return np.asarray(h, np.uint16).view(np.float16).astype(np.float64)


def deq_q4k(rows: np.ndarray, cols: int) -> np.ndarray:
    """ggml dequantize_row_q4_K: y = d*sc*q - dmin*m per 32-sub-block."""
    n = rows.shape[0]
    sb = rows.reshape(n, cols // 256, 144)
    d = half(sb[..., 0].astype(np.uint16) | (sb[..., 1].astype(np.uint16) << 8))
    dmin = half(sb[..., 2].astype(np.uint16) | (sb[..., 3].astype(np.uint16) << 8))
    s = sb[..., 4:16].astype(np.int64)
    sc = np.empty(s.shape[:-1] + (8,), np.int64); mn = np.empty_like(sc)
    for j in range(8):
        if j < 4:
            sc[..., j] = s[..., j] & 63; mn[..., j] = s[..., j + 4] & 63
        else:
            sc[..., j] = (s[..., j + 4] & 0xF) | ((s[..., j - 4] >> 6) << 4)
            mn[..., j] = (s[..., j + 4] >> 4) | ((s[..., j] >> 6) << 4)
    qs = sb[..., 16:144].astype(np.int64)
    out = np.empty((n, cols // 256, 256), np.float64)
    for c in range(4):
        q = qs[..., c * 32:(c + 1) * 32]
        for nib in range(2):
            j = 2 * c + nib
            v = (q & 0xF) if nib == 0 else (q >> 4)
            out[..., j * 32:(j + 1) * 32] = (d * sc[..., j])[..., None] * v - (dmin * mn[..., j])[..., None]
    return out.reshape(n, cols)


def deq_q6k(rows: np.ndarray, cols: int) -> np.ndarray:
    """ggml dequantize_row_q6_K."""
    n = rows.shape[0]
    sb = rows.reshape(n, cols // 256, 210).astype(np.int64)
    ql, qh, sc = sb[..., 0:128], sb[..., 128:192], sb[..., 192:208]
    sc = np.where(sc > 127, sc - 256, sc)
    d = half((sb[..., 208] | (sb[..., 209] << 8)).astype(np.uint16))
    out = np.empty((n, cols // 256, 256), np.float64)
    for h in range(2):
        for l in range(32):
            q1 = ((ql[..., h * 64 + l] & 0xF) | (((qh[..., h * 32 + l] >> 0) & 3) << 4)) - 32
            q2 = ((ql[..., h * 64 + l + 32] & 0xF) | (((qh[..., h * 32 + l] >> 2) & 3) << 4)) - 32
            q3 = ((ql[..., h * 64 + l] >> 4) | (((qh[..., h * 32 + l] >> 4) & 3) << 4)) - 32
            q4 = ((ql[..., h * 64 + l + 32] >> 4) | (((qh[..., h * 32 + l] >> 6) & 3) << 4)) - 32
            is_ = l // 16
            base = h * 128
            out[..., base + l] = d * sc[..., h * 8 + is_ + 0] * q1
            out[..., base + l + 32] = d * sc[..., h * 8 + is_ + 2] * q2
            out[..., base + l + 64] = d * sc[..., h * 8 + is_ + 4] * q3
            out[..., base + l + 96] = d * sc[..., h * 8 + is_ + 6] * q4
    return out.reshape(n, cols)


def q8_f64(x: np.ndarray, block: int = 32):
    """Per-block symmetric int8 (amax seeded 1e-12, ties away from zero), in f64."""
    xb = x.reshape(-1, block).astype(np.float64)
    amax = np.maximum(1e-12, np.abs(xb).max(axis=1))
    sc = amax / 127.0
    r = xb / sc[:, None]
    q = np.clip(np.sign(r) * np.floor(np.abs(r) + 0.5), -127, 127)
    return q.reshape(x.shape), sc


def gptoss_ffn_f64(L: dict, xn: np.ndarray, ids=None, quantize: bool = True):
    """scripts/ffn_reference.py's layer (corrected scale) in float64.
    quantize=True simulates the engine's Q8 of the input and of h so that the
    only difference from the fp32 path is rounding; ids forces the routing.
    Returns (ffn_out, ids, wts)."""
    d, dff, ne, k = L["d"], L["dff"], L["ne"], L["k"]
    xn = xn.astype(np.float64)
    logits = L["router_w"].astype(np.float64) @ xn + L["router_b"].astype(np.float64)
    if ids is None:
        ids = np.argsort(-logits, kind="stable")[:k]
    w = logits[ids]; w = np.exp(w - w.max()); w /= w.sum()
    if quantize:
        q, sc = q8_f64(xn)
        xin = (q.reshape(-1, 32) * sc[:, None]).reshape(-1)
    else:
        xin = xn
    out = np.zeros(d)
    for e, we in zip(ids, w):
        g = deq_mxfp4(L["gate"][e * dff:(e + 1) * dff], d) @ xin + L["gate_b"][e]
        u = deq_mxfp4(L["up"][e * dff:(e + 1) * dff], d) @ xin + L["up_b"][e]
        xg = np.minimum(g, L["limit"]); yu = np.clip(u, -L["limit"], L["limit"])
        h = (xg / (1 + np.exp(-L["alpha"] * xg))) * (yu + 1)
        if quantize:
            q, sc = q8_f64(h)
            h = (q.reshape(-1, 32) * sc[:, None]).reshape(-1)
        out += we * (deq_mxfp4(L["down"][e * d:(e + 1) * d], dff) @ h + L["down_b"][e])
    return out, np.asarray(ids), w
