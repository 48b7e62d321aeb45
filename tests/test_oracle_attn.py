"""Pins the attention restatement (oracle/attn.c) with independent float64
computations: the YaRN RoPE table (engine_gpt2.rs:556-576), and one decode
step of the block (:772-843) -- Q8 projections, RoPE, the cache, the
sink-augmented softmax over the (sliding) window and the o-projection.
CPU only."""
import math

import numpy as np

from cpubrrr_amd import synth
from oracle import oracle as O


def rope_f64(hd, pos, base):
    """rope_yarn_slow's formula in float64 (freq_base, factor 32, original
    context 4096, beta_fast 32, beta_slow 1, mscale 1 + 0.1 ln 32)"""
    fd = lambda beta: hd * math.log(4096.0 / (beta * 2 * math.pi)) / (2 * math.log(base))
    low, high = max(math.floor(fd(32.0)), 0.0), min(math.ceil(fd(1.0)), hd - 1.0)
    ms = 1 + 0.1 * math.log(32.0)
    out = []
    for i in range(hd // 2):
        ex = pos * base ** (-(2.0 * i) / hd)
        y = (i - low) / max(high - low, 0.001)
        mix = 1 - min(max(y, 0.0), 1.0)
        th = ex / 32 * (1 - mix) + ex * mix
        out.append((math.cos(th) * ms, math.sin(th) * ms))
    return np.array(out)


def test_rope_table():
    hd, base = 64, 150000.0
    tab = O.rope_table(hd, 300, base).reshape(300, hd // 2, 2)
    ms = np.float32(1 + np.float32(0.1) * np.float32(math.log(32.0)))
    assert np.all(tab[0, :, 0] == ms) and np.all(tab[0, :, 1] == 0)        # pos 0: no rotation
    for pos in (1, 7, 129, 299):
        ref = rope_f64(hd, pos, base)
        # fp32 theta (pos * base^-x) carries a relative error ~pos * 1e-7 into the angle
        assert np.max(np.abs(tab[pos] - ref)) <= 2e-6 * (1 + pos), pos


def f64_step(L, il, pos, x, kc, vc, tab):
    """float64 restatement of one decode step on the same Q8 weights"""
    d, nh, nkv, hd, swa = L["d"], L["nh"], L["nkv"], L["hd"], L["swa"]
    xn = O.rmsnorm_gptoss(x, L["attn_norm"], L["eps"])
    xq, xsb = O.qblock32(xn)
    xd = xq.astype(np.float64) * np.repeat(xsb, 32)
    deq = lambda q, s: q.astype(np.float64) * np.repeat(s, 32, axis=1)
    q = deq(L["wq"], L["sq"]) @ xd + L["bq"]
    k = deq(L["wk"], L["sk"]) @ xd + L["bk"]
    v = deq(L["wv"], L["sv"]) @ xd + L["bv"]
    t = tab.reshape(-1, hd // 2, 2)[pos].astype(np.float64)

    def rot(a):
        a = a.reshape(-1, hd).copy()
        lo, hi = a[:, :hd // 2].copy(), a[:, hd // 2:].copy()
        a[:, :hd // 2] = lo * t[:, 0] - hi * t[:, 1]
        a[:, hd // 2:] = hi * t[:, 0] + lo * t[:, 1]
        return a
    q, k = rot(q), rot(k)
    kc = kc.astype(np.float64).copy()
    vc = vc.astype(np.float64).copy()
    kc[pos], vc[pos] = k, v.reshape(nkv, hd)
    start = max(pos - (swa - 1), 0) if (il + 1) % 2 else 0
    ao = np.zeros((nh, hd))
    for h in range(nh):
        kvh = h // (nh // nkv)
        sc = kc[start:pos + 1, kvh] @ q[h] / math.sqrt(hd)
        mx = max(L["sinks"][h], sc.max())
        e = np.exp(sc - mx)
        den = math.exp(L["sinks"][h] - mx) + e.sum()
        ao[h] = (e[:, None] * vc[start:pos + 1, kvh]).sum(0) / den
    aq, asb = O.qblock32(ao.reshape(-1).astype(np.float32))
    o = deq(L["wo"], L["so"]) @ (aq.astype(np.float64) * np.repeat(asb, 32)) + L["bo"]
    return x + o, q.reshape(-1), k.reshape(-1), ao.reshape(-1)


def _layer(seed, swa):
    L = synth.attn_layer(256, 8, 2, 64, seed=seed, swa=swa)
    for n in ("q", "k", "v", "o"):
        L["w" + n], L["s" + n] = O.q8_rows(L["w" + n])
    return L


def test_attention_step_vs_f64():
    L = _layer(5, 4)
    hd, nkv, S = 64, 2, 16
    tab = O.rope_table(hd, S, 150000.0)
    r = np.random.default_rng(5)
    for il in (0, 1):                    # layer 0 uses the sliding window, layer 1 full causal
        kc = np.zeros((S, nkv, hd), np.float32)
        vc = np.zeros((S, nkv, hd), np.float32)
        for pos in range(10):
            x = (r.standard_normal(256) * 2).astype(np.float32)
            kc0, vc0 = kc.copy(), vc.copy()
            xo, t = O.attn_layer(L, il, pos, x, kc, vc, tab)
            xr, qr, kr, aor = f64_step(L, il, pos, x, kc0, vc0, tab)
            assert np.allclose(t["q"], qr, rtol=1e-5, atol=1e-5)
            assert np.allclose(kc[pos].reshape(-1), kr, rtol=1e-5, atol=1e-5)
            assert np.allclose(t["ao"], aor, rtol=1e-4, atol=1e-5)
            rms = np.sqrt(((xr - x) ** 2).mean())
            assert np.max(np.abs(xo - xr)) <= 2e-3 * rms, (il, pos)


def test_sliding_window_ignores_old_positions():
    L = _layer(6, 4)
    hd, nkv, S, pos = 64, 2, 16, 9
    tab = O.rope_table(hd, S, 150000.0)
    r = np.random.default_rng(6)
    kc = r.standard_normal((S, nkv, hd)).astype(np.float32)
    vc = r.standard_normal((S, nkv, hd)).astype(np.float32)
    x = r.standard_normal(256).astype(np.float32)
    y0, _ = O.attn_layer(L, 0, pos, x, kc.copy(), vc.copy(), tab)
    kc2, vc2 = kc.copy(), vc.copy()
    kc2[:pos - 3] += 5.0                 # outside the window of 4 positions
    vc2[:pos - 3] -= 5.0
    y1, _ = O.attn_layer(L, 0, pos, x, kc2, vc2, tab)
    assert np.array_equal(y0, y1)
    y2, _ = O.attn_layer(L, 1, pos, x, kc2, vc2, tab)     # full-causal layer sees them
    assert not np.array_equal(y0, y2)
