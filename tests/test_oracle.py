"""Pins the oracle (oracle/oracle.c) against independent checks: published
format definitions, exact integer arithmetic, closed forms and float64
references.  CPU only.

The reference ships no golden vectors (its verifiers need a GGUF blob or
/tmp JSON that is not in the repository), so every oracle function is pinned
by the checks below instead; tests/golden/ holds fixtures written from them.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O
from tests import f64ref as R

rng = np.random.default_rng(1234)


def f32(x):
    return np.float32(x)


# ---------------------------------------------------------------- scalars
def test_e8m0_table():
    # engine_gpt2.rs:436-438: 2f32.powi(e-128); powi(2,-128) = 1/inf = 0
    assert O.e8m0_half(0) == 0.0
    for e in range(1, 256):
        assert O.e8m0_half(e) == math.ldexp(1.0, e - 128), e
    # OCP MX: element scale 2^(e-127) applied to E2M1 = doubled table * 2^(e-128)
    assert O.e8m0_half(127) * 2 == 1.0


def test_half_to_f32_all_codes():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([O.half_to_f32(int(v)) for v in h], np.float32)
    same = (got == ref) | (np.isnan(got) & np.isnan(ref))
    assert same.all()


# ---------------------------------------------------------------- Q8 / Q8_K
def _check_q8(x, xq, sc, block):
    xb = x.reshape(-1, block).astype(np.float64)
    amax = np.maximum(1e-12, np.abs(xb).max(1)).astype(np.float32)
    assert np.array_equal(sc, amax / np.float32(127.0))
    r = xb / sc.astype(np.float64)[:, None]
    q = xq.reshape(-1, block).astype(np.float64)
    # |q - v/sc| <= 1/2 (+ the fp32 rounding of v/sc), clamp never exceeded
    assert np.all(np.abs(q - np.clip(r, -127, 127)) <= 0.5 + 1e-5)
    assert np.all(np.abs(q) <= 127)


def test_qblock32_properties():
    x = rng.standard_normal(2880).astype(np.float32) * 3
    xq, xsb = O.qblock32(x)
    _check_q8(x, xq, xsb, 32)
    # the block maximum maps to +-127
    xb = x.reshape(-1, 32)
    i = np.abs(xb).argmax(1)
    assert np.all(np.abs(xq.reshape(-1, 32)[np.arange(90), i]) == 127)


def test_qblock32_ties_round_away_from_zero():
    # sc = 127/127 = 1: v/sc is exact, ties at .5 go away from zero
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1:9] = [0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 126.5, -126.5]
    xq, xsb = O.qblock32(x)
    assert xsb[0] == 1.0
    assert list(xq[:9]) == [127, 1, -1, 2, -2, 3, -3, 127, -127]


def test_qblock32_zero_block():
    xq, xsb = O.qblock32(np.zeros(64, np.float32))
    assert np.all(xq == 0) and np.all(xsb == np.float32(1e-12) / np.float32(127.0))


def test_qblock_k_properties():
    x = rng.standard_normal(2048).astype(np.float32)
    xq, ys, xsum = O.qblock_k(x)
    _check_q8(x, xq, ys, 256)
    assert np.array_equal(xsum, xq.reshape(-1, 32).astype(np.int32).sum(1))


# ---------------------------------------------------------------- norms
def test_rmsnorm_gptoss_vs_f64():
    x = rng.standard_normal(2880).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(2880)).astype(np.float32)
    out = O.rmsnorm_gptoss(x, w, 1e-5)
    ref = x.astype(np.float64) / np.sqrt((x.astype(np.float64) ** 2).mean() + 1e-5) * w
    assert np.max(np.abs(out - ref)) <= 4e-7 * np.max(np.abs(ref))
    s = O.ssq_gptoss(x)
    assert abs(float(s) - float((x.astype(np.float64) ** 2).sum())) <= 1e-5 * float(s)


def test_ssq_order_is_16_lanes():
    # one large value in lane 0 and many tiny ones elsewhere: a serial sum and
    # the 16-lane sum differ in the last bits; the oracle follows the lanes.
    x = np.full(2880, 1e-4, np.float32)
    x[0] = 3.0
    lanes = np.zeros(16, np.float32)
    for i in range(0, 2880, 16):
        for l in range(16):
            lanes[l] = np.float32(np.float64(x[i + l]) * x[i + l] + np.float64(lanes[l]))  # fma = one rounding
    L = [(lanes[l] + lanes[4 + l]) + (lanes[8 + l] + lanes[12 + l]) for l in range(4)]
    expect = (L[0] + L[1]) + (L[2] + L[3])
    assert O.ssq_gptoss(x) == expect


def test_rmsnorm_qwen_vs_f64():
    x = rng.standard_normal(2048).astype(np.float32)
    w = np.ones(2048, np.float32)
    out = O.rmsnorm_qwen(x, w, 1e-6, 12)
    ref = x.astype(np.float64) / np.sqrt((x.astype(np.float64) ** 2).mean() + 1e-6)
    assert np.max(np.abs(out - ref)) <= 4e-7 * np.max(np.abs(ref))


def test_rmsnorm_qwen_slice_order_known_answer():
    # engine_qwen2.rs:243-250, 457-467: NT static slices, each summed serially,
    # then the NT partials summed serially.  x = [2^12, 1, 1, ...] (d = 24):
    # in fp32, 2^24 + 1 rounds back to 2^24 (tie to even), so a serial sum
    # stays at 2^24 while 12 slices of 2 keep 11 partials of 2:
    # tot = 2^24 + 22 exactly.  A serial sum (nt = 1) gives 2^24.
    d = 24
    x = np.ones(d, np.float32)
    x[0] = 4096.0
    w = np.ones(d, np.float32)
    for nt, tot in ((12, 2.0 ** 24 + 22), (1, 2.0 ** 24), (24, 2.0 ** 24)):
        inv = f32(1.0) / np.sqrt(f32(f32(tot) / f32(d)) + f32(1e-6), dtype=np.float32)
        out = O.rmsnorm_qwen(x, w, 1e-6, nt)
        assert out[1] == f32(f32(1.0) * inv), (nt, out[1], inv)
        assert out[0] == f32(f32(4096.0) * inv), nt
    # (nt = 24: one element per slice, the partials summed serially as above)
    # the slice order and the serial order give different scales
    outs = {nt: O.rmsnorm_qwen(x, w, 1e-6, nt)[1] for nt in (1, 12)}
    assert outs[1] != outs[12]
    # uneven slices (d % nt != 0): the first d % nt slices take one more element
    d = 26
    x = np.ones(d, np.float32)
    x[0] = 4096.0
    w = np.ones(d, np.float32)
    # slices: 2 of 3 elements, 10 of 2 -> slice 0 = 2^24 (both ones lost), slice 1 = 3,
    # slices 2..11 = 2: tot = 2^24 + 3 + 20 -> rounds: 2^24 + 3 -> 2^24 + 4 (tie to even), + 20
    tot = f32(2.0 ** 24)
    for part in [3.0] + [2.0] * 10:
        tot = f32(tot + f32(part))
    assert tot == f32(2.0 ** 24 + 24)
    inv = f32(1.0) / np.sqrt(f32(tot / f32(d)) + f32(1e-6), dtype=np.float32)
    assert O.rmsnorm_qwen(x, w, 1e-6, 12)[1] == inv


def _pack_q4k_scales(sc, mn):
    """Pack 8 six-bit scales and mins into the 12 Q4_K scale bytes, written
    from the format's description (ggml's quantize_row_q4_K packing): bytes
    0-3 hold sc[0..3] plus the top 2 bits of sc[4..7]; bytes 4-7 hold
    mn[0..3] plus the top 2 bits of mn[4..7]; bytes 8-11 hold the low nibbles
    of sc[4..7] (low) and mn[4..7] (high)."""
    q = [0] * 12
    for j in range(4):
        q[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        q[j + 4] = mn[j] | ((mn[j + 4] >> 4) << 6)
        q[j + 8] = (sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4)
    return q


def test_q4k_scale_unpack_hand_built():
    # engine_qwen2.rs:57-74 (get_scale_min_k4): a superblock with hand-packed
    # scales/mins, d = dmin = 1.0, every quant nibble = 1, x = 1 on one
    # sub-block only: sumi = 32 * sc_j and mint = mn_j * xsum_j recover each
    # sub-block's 6-bit scale and min.
    r = np.random.default_rng(7)
    for trial in range(20):
        sc = [int(v) for v in r.integers(0, 64, 8)]
        mn = [int(v) for v in r.integers(0, 64, 8)]
        if trial == 0:
            sc, mn = [63] * 8, [63] * 8
        if trial == 1:
            sc, mn = [1, 2, 4, 8, 16, 32, 48, 63], [63, 32, 16, 8, 4, 2, 1, 0]
        blk = np.zeros(144, np.uint8)
        blk[0:2] = [0x00, 0x3C]          # fp16 1.0
        blk[2:4] = [0x00, 0x3C]
        blk[4:16] = _pack_q4k_scales(sc, mn)
        blk[16:] = 0x11
        for j in range(8):
            xq = np.zeros(256, np.int8)
            xq[32 * j:32 * j + 32] = 1
            xsum = np.zeros(8, np.int32)
            xsum[j] = 32
            v, s = O.q4k_dot(blk, xq, np.ones(1, np.float32), xsum)
            assert s[0] == 32 * sc[j] and s[1] == 32 * mn[j], (trial, j, s, sc[j], mn[j])
            assert v == f32(32 * sc[j]) - f32(32 * mn[j])


# ---------------------------------------------------------------- router / top-k
def test_router_serial_order_and_bound():
    ne, d = 8, 2880
    W = (0.02 * rng.standard_normal((ne, d))).astype(np.float32)
    b = (0.1 * rng.standard_normal(ne)).astype(np.float32)
    x = rng.standard_normal(d).astype(np.float32)
    lg = O.router(W, b, x)
    exact = (W.astype(np.float64) * x).sum(1) + b
    # Higham's recursive-summation bound
    u = 2.0 ** -24
    bound = d * u * (np.abs(W.astype(np.float64) * x).sum(1) + np.abs(b)) * 1.01
    assert np.all(np.abs(lg - exact) <= bound)
    # a short chain restated with numpy fp32 scalars agrees bit for bit
    acc = b[3]
    for j in range(d):
        acc = f32(acc + f32(W[3, j] * x[j]))
    assert lg[3] == acc
    assert np.array_equal(O.router(W, None, x)[:1], O.router(W[:1], None, x))


def test_topk_gptoss_bruteforce():
    for trial in range(200):
        ne = 32
        lg = rng.standard_normal(ne).astype(np.float32)
        if trial % 3 == 0:
            lg = np.round(lg * 2) / 2            # many exact ties
        ids, w = O.topk_gptoss(lg, 4)
        order = sorted(range(ne), key=lambda e: (-float(lg[e]), e))[:4]   # lowest index wins ties
        assert list(ids) == order
        v = lg[order].astype(np.float64)
        ref = np.exp(v - v.max()); ref /= ref.sum()
        assert np.allclose(w, ref, rtol=2e-6, atol=1e-7)


def test_topk_qwen_equivalences():
    for trial in range(100):
        ne, k = 128, 8
        lg = rng.standard_normal(ne).astype(np.float32)
        if trial % 4 == 0:
            lg = np.round(lg * 4) / 4
        ids, w = O.topk_qwen(lg, k)
        ids_g, w_g = O.topk_gptoss(lg, k)
        assert np.array_equal(ids, ids_g)                   # both: lowest index wins ties
        # definition (engine_qwen.rs:374-381): softmax over all, top-k, renormalise
        p = np.exp(lg.astype(np.float64) - lg.max()); p /= p.sum()
        sel = p[ids] / p[ids].sum()
        assert np.allclose(w, sel, rtol=3e-6, atol=1e-7)


# ---------------------------------------------------------------- MXFP4 dot
def test_mx_block_sums_exact_and_dot():
    d = 2880
    from cpubrrr_amd import synth
    rows = synth.mxfp4(16, d // 32, 7, 99)
    x = rng.standard_normal(d).astype(np.float32)
    xq, xsb = O.qblock32(x)
    for r in range(16):
        v, sums = O.mx_row_dot(rows[r], xq, xsb)
        exact = R.mx_block_sums(rows[r], xq)
        assert np.array_equal(sums.astype(np.int64), exact)
        assert np.all(np.abs(exact) <= 48768)
        # float: sum_b S_b * 2^(e-128) * xsb_b in f64
        e = rows[r].reshape(-1, 17)[:, 0].astype(np.float64)
        ref = (exact * np.exp2(e - 128) * xsb.astype(np.float64)).sum()
        assert abs(v - ref) <= 1e-6 * np.abs(exact * np.exp2(e - 128) * xsb).sum()
        # against OCP dequant of the weights
        ref2 = R.deq_mxfp4(rows[r:r + 1], d)[0] @ (xq.astype(np.float64).reshape(-1, 32) * xsb[:, None]).reshape(-1)
        assert abs(v - ref2) <= 1e-5 * (abs(ref2) + 1)


def test_mx_known_answers():
    d = 64
    # every code = 2 (E2M1 1.0), e = 127 -> weight 1.0 -> row dot = sum(xq*xsb)
    row = np.zeros((2, 17), np.uint8)
    row[:, 0] = 127
    row[:, 1:] = 0x22
    x = np.arange(d, dtype=np.float32) - 20
    xq, xsb = O.qblock32(x)
    v, sums = O.mx_row_dot(row.reshape(-1), xq, xsb)
    assert list(sums) == [2 * int(xq[:32].sum()), 2 * int(xq[32:].sum())]
    assert abs(v - float((xq.reshape(2, 32).sum(1) * xsb).sum())) < 1e-4
    # one-hot activation picks out one weight: code 15 = -6.0 (doubled -12)
    row[:, 1:] = 0
    row[0, 1 + 5] = 0xF0            # element 16+5 = code 15
    xo = np.zeros(d, np.float32); xo[21] = 1.0
    xq, xsb = O.qblock32(xo)
    v, sums = O.mx_row_dot(row.reshape(-1), xq, xsb)
    assert sums[0] == -12 * 127 and sums[1] == 0
    assert v == np.float32(-12 * 127) * (np.float32(0.5) * xsb[0])


# ---------------------------------------------------------------- k-quants
def test_q4k_q6k_vs_ggml_dequant():
    from cpubrrr_amd import synth
    d = 2048
    g = synth.q4k(8, d, 3, 5)
    dn = synth.q6k(8, d, 3, 6)
    x = rng.standard_normal(d).astype(np.float32)
    xq, ys, xsum = O.qblock_k(x)
    xdeq = (xq.astype(np.float64).reshape(-1, 256) * ys[:, None]).reshape(-1)
    W4 = R.deq_q4k(g, d)
    W6 = R.deq_q6k(dn, d)
    for r in range(8):
        v, s = O.q4k_dot(g[r], xq, ys, xsum)
        ref = W4[r] @ xdeq
        mag = np.abs(W4[r] * xdeq).sum()
        assert abs(v - ref) <= 2e-6 * mag + 1e-9
        v6, s6 = O.q6k_dot(dn[r], xq, ys)
        ref6 = W6[r] @ xdeq
        assert abs(v6 - ref6) <= 2e-6 * np.abs(W6[r] * xdeq).sum() + 1e-9
        # integer identity: sumi*d - mint*dmin per superblock equals the dequant sum / ys
        sb = g[r].reshape(-1, 144)
        dd = R.half(sb[:, 0].astype(np.uint16) | (sb[:, 1].astype(np.uint16) << 8))
        dm = R.half(sb[:, 2].astype(np.uint16) | (sb[:, 3].astype(np.uint16) << 8))
        per = (W4[r] * xq.astype(np.float64)).reshape(-1, 256).sum(1)
        assert np.allclose(per, dd * s[0::2] - dm * s[1::2], rtol=1e-12, atol=1e-9)
        sb6 = dn[r].reshape(-1, 210)
        d6 = R.half(sb6[:, 208].astype(np.uint16) | (sb6[:, 209].astype(np.uint16) << 8))
        per6 = (W6[r] * xq.astype(np.float64)).reshape(-1, 256).sum(1)
        assert np.allclose(per6, d6 * s6, rtol=1e-12, atol=1e-9)


# ---------------------------------------------------------------- whole layers
def _small_gptoss(seed=0, d=480, dff=480, ne=8, k=4, zipf=None):
    from cpubrrr_amd import synth
    return synth.gptoss_layer(d, dff, ne, k, seed=seed, zipf=zipf)


@pytest.mark.parametrize("apply_norm", [False, True])
def test_gptoss_layer_vs_f64(apply_norm):
    L = _small_gptoss()
    from cpubrrr_amd import synth
    x = synth.token(L["d"], 0)
    xo, t = O.gptoss_moe(L, x, apply_norm, want_sums=True)
    ffn = (xo - x).astype(np.float64)
    xn = t["xn"]
    ref, ids, w = R.gptoss_ffn_f64(L, xn, ids=t["ids"], quantize=True)
    rms = np.sqrt((ref ** 2).mean())
    assert np.max(np.abs(ffn - ref)) <= 1e-3 * rms
    # routing agrees with an f64 argsort (gaps here are far above rounding)
    _, ids64, _ = R.gptoss_ffn_f64(L, xn, quantize=False)
    assert np.array_equal(t["ids"], ids64)
    # unquantised f64 layer (ffn_reference.py semantics): int8 activations cost ~0.4%
    ref_fp, _, _ = R.gptoss_ffn_f64(L, xn, quantize=False)
    cos = ffn @ ref_fp / np.linalg.norm(ffn) / np.linalg.norm(ref_fp)
    assert cos > 0.9995
    # block sums are exact integer dots of the trace's own int8 operands
    for ei in range(L["k"]):
        e = t["ids"][ei]
        r = 7
        assert np.array_equal(t["gu_sums"][ei, 0, r], R.mx_block_sums(L["gate"][e * L["dff"] + r], t["xq"]))
        assert np.array_equal(t["dn_sums"][ei, r], R.mx_block_sums(L["down"][e * L["d"] + r], t["hq"][ei]))


@pytest.mark.parametrize("apply_norm", [False, True])
def test_gptoss_f64_dequant_mode_vs_numpy(apply_norm):
    # the CPU baseline's second mode (orc_gptoss_moe_f64, C) against the
    # numpy float64 layer of tests/f64ref.py (OCP MX decode, 2^(e-127) with
    # the plain E2M1 table), unquantised: the same mathematics summed in
    # another order
    L = _small_gptoss(seed=3, zipf=1.1)
    from cpubrrr_amd import synth
    x = synth.token(L["d"], 3) * np.float32(2.0)
    got = O.gptoss_moe_f64(L, x, apply_norm)
    x64 = x.astype(np.float64)
    if apply_norm:
        xn = x64 / np.sqrt((x64 ** 2).mean() + 1e-5) * L["norm_w"].astype(np.float64)
    else:
        xn = x64
    ref, _, _ = R.gptoss_ffn_f64(L, xn, quantize=False)
    want = (x64 + ref).astype(np.float32)
    assert np.max(np.abs(got.astype(np.float64) - want)) <= 1e-6 * np.abs(want).max()


def test_qwen_layer_vs_f64():
    from cpubrrr_amd import synth
    d, dff, ne, k = 512, 256, 16, 8
    L = synth.qwen_layer(d, dff, ne, k, seed=1)
    x = synth.token(d, 1)
    xo, t = O.qwen_moe(L, x, True, want_sums=True)
    ffn = (xo - x).astype(np.float64)
    xq, ys = t["xq"], t["xsb"]
    xin = (xq.astype(np.float64).reshape(-1, 256) * ys[:, None]).reshape(-1)
    ids = t["ids"]
    lg = L["router_w"].astype(np.float64) @ t["xn"].astype(np.float64)
    assert np.array_equal(ids, np.argsort(-lg, kind="stable")[:k])
    w = lg[ids]; w = np.exp(w - w.max()); w /= w.sum()
    out = np.zeros(d)
    for ei, e in enumerate(ids):
        g = R.deq_q4k(L["gate"][e * dff:(e + 1) * dff], d) @ xin
        u = R.deq_q4k(L["up"][e * dff:(e + 1) * dff], d) @ xin
        h = g / (1 + np.exp(-g)) * u
        hq, hs = R.q8_f64(h, 256)
        hdq = (hq.reshape(-1, 256) * hs[:, None]).reshape(-1)
        out += w[ei] * (R.deq_q6k(L["down"][e * d:(e + 1) * d], dff) @ hdq)
    rms = np.sqrt((out ** 2).mean())
    assert np.max(np.abs(ffn - out)) <= 1e-3 * rms
