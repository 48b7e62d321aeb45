"""Pins the head restatement (oracle/head.c) against independent numpy
float32 restatements and closed forms: bf16 rounding, the Q4 scale search
(engine_gpt2.rs:274-300), Q4 / Q8 row quantisation and dots (:240-272,
:314-342, :466-494, :169-191) and the two-stage head's candidate and greedy
logic (:937-1002).  CPU only."""
import numpy as np

from oracle import oracle as O

rng = np.random.default_rng(99)
f32 = np.float32


def fma32(a, b, c):
    """a * b + c with one rounding to fp32 (round to nearest even), exactly"""
    from fractions import Fraction
    exact = Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))
    cand = np.float32(float(exact))
    best = None
    for v in (np.nextafter(cand, np.float32(-np.inf)), cand, np.nextafter(cand, np.float32(np.inf))):
        err = abs(Fraction(float(v)) - exact)
        key = (err, int(np.float32(v).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, v)
    return np.float32(best[1])


def bf16_np(v):
    """round-to-nearest-even of fp32 into its top 16 bits (numpy, vectorised)"""
    b = np.asarray(v, np.float32).view(np.uint32).astype(np.uint64)
    return (((b + 0x7FFF + ((b >> 16) & 1)) >> 16) & 0xFFFF).astype(np.uint16)


def from_bf16(h):
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def test_bf16_rounding():
    vals = np.concatenate([rng.standard_normal(2000).astype(np.float32),
                           np.array([1.0, -1.0, 0.0, 1.00390625, 1.01171875, 3.0e38, 1e-40], np.float32)])
    # exact ties: low 16 bits = 0x8000 round to even
    ties = (rng.integers(0, 1 << 15, 200).astype(np.uint32) << 16 | 0x8000).view(np.float32) + np.float32(0)
    vals = np.concatenate([vals, ties[np.isfinite(ties)]])
    got = np.array([O.f32_to_bf16(v) for v in vals], np.uint16)
    assert np.array_equal(got, bf16_np(vals))
    # bf16 of exactly representable values is exact
    r = from_bf16(rng.integers(0, 0x7F80, 500).astype(np.uint16))
    assert np.array_equal(from_bf16(np.array([O.f32_to_bf16(v) for v in r], np.uint16)), r)


def scale_search_np(vals):
    vals = np.asarray(vals, np.float32)
    amax, vmax = f32(0), f32(0)
    for v in vals:
        if abs(v) > amax:
            amax, vmax = abs(v), v
    if amax == 0:
        return 0, f32(0)
    best_err, best_db = np.float32(np.finfo(np.float32).max), 0
    for t in range(17):
        nmax = f32(7.0) + f32(t) * f32(0.0625)
        db = int(bf16_np(vmax / -nmax))
        d = from_bf16(np.uint16(db))
        if d == 0:
            continue
        idq = f32(1.0) / d
        err = f32(0)
        for v in vals:
            c = int(np.clip(np.floor(v * idq + f32(8.5)), 0, 15))
            e = v - f32(c - 8) * d
            err = f32(err + f32(e * e))
        if err < best_err:
            best_err, best_db = err, db
    d = from_bf16(np.uint16(best_db))
    return best_db, (f32(1.0) / d if d != 0 else f32(0))


def test_q4_scale_search_and_codes():
    for trial in range(60):
        vals = from_bf16(bf16_np(rng.standard_normal(32).astype(np.float32) * f32(10 ** rng.uniform(-3, 1))))
        if trial == 0:
            vals[:] = 0
        if trial == 1:
            vals = from_bf16(bf16_np(np.linspace(-1, 2, 32)))
        db, idq = O.q4_scale_search(vals)
        db2, idq2 = scale_search_np(vals)
        assert db == db2 and idq == idq2, trial
    # the row quantiser: codes from the chosen scale; block of zeros -> code 8
    w = bf16_np(rng.standard_normal(256).astype(np.float32) * 0.02)
    w[32:64] = 0
    nib, sc = O.q4_quant_row(w)
    for b in range(8):
        vals = from_bf16(w[b * 32:(b + 1) * 32])
        db, idq = scale_search_np(vals)
        assert sc[b] == db
        c = np.clip(np.floor(vals * idq + f32(8.5)), 0, 15).astype(np.uint8)
        assert np.array_equal(nib[b * 16:(b + 1) * 16], c[:16] | (c[16:] << 4)), b
    assert np.all(nib[16:32] == 0x88) and sc[1] == 0


def test_q4_scale_search_known_answers():
    # Pins of engine_gpt2.rs:279-300 that do not restate its loop: blocks
    # whose optimum the arithmetic fixes.
    # (a) values k * d0 with k in [-8, 7] and one k = -8: the Q4_0 end
    #     (nmax = 8, t = 16) reproduces every value exactly (error 0); no
    #     earlier candidate rounds to d0 in bf16, so it is the unique best
    k = rng.integers(-7, 8, 32)
    k[5] = -8
    vals = (k * np.float32(-0.25)).astype(np.float32)           # vmax = +2.0
    db, idq = O.q4_scale_search(vals)
    assert db == 0xBE80 and idq == np.float32(-4.0)             # bf16(-0.25)
    nib, sc = O.q4_quant_row(bf16_np(vals))
    codes = np.concatenate([nib[:16] & 15, nib[:16] >> 4])
    assert sc[0] == 0xBE80 and np.array_equal(codes.astype(int) - 8, k)
    # (b) symmetric end: |k| <= 7 and vmax = 7 * d0 < 0: nmax = 7 (t = 0)
    #     gives d = +0.25 and error 0; the first exact candidate wins
    k = rng.integers(-7, 8, 32)
    k[9] = 7
    vals = (k * np.float32(-0.25)).astype(np.float32)           # vmax = -1.75
    db, idq = O.q4_scale_search(vals)
    assert db == 0x3E80 and idq == np.float32(4.0)              # bf16(+0.25)
    # (c) all-equal block 3.0: only nmax = 8 reconstructs it exactly
    #     (code 0, (0 - 8) * -0.375 = 3); every other candidate's bf16 scale
    #     leaves an error
    db, idq = O.q4_scale_search(np.full(32, 3.0, np.float32))
    assert db == 0xBEC0                                          # bf16(-0.375)
    # (d) the zero block: scale 0, every code 8
    db, idq = O.q4_scale_search(np.zeros(32, np.float32))
    assert db == 0 and idq == 0
    nib, sc = O.q4_quant_row(np.zeros(32, np.uint16))
    assert sc[0] == 0 and np.all(nib == 0x88)


def test_q4_scale_search_error_minimal_f64():
    # The chosen scale's reconstruction error, recomputed in float64, is the
    # least among the 17 candidates vmax / -(7 + t/16) rounded to bf16
    # (up to the float32 rounding of the reference's own error sums).
    for trial in range(200):
        vals = from_bf16(bf16_np(rng.standard_normal(32).astype(np.float32) * f32(10 ** rng.uniform(-3, 1))))
        vmax = vals[np.argmax(np.abs(vals))]
        errs = {}
        for t in range(17):
            d = float(from_bf16(bf16_np(np.float32(vmax) / -np.float32(7 + t / 16))))
            if d == 0.0:
                continue
            idq = float(np.float32(1.0) / np.float32(d))
            c = np.clip(np.floor(vals.astype(np.float64) * idq + 8.5), 0, 15)
            errs[t] = float(((vals.astype(np.float64) - (c - 8) * d) ** 2).sum())
        db, _ = O.q4_scale_search(vals)
        d_chosen = float(from_bf16(np.uint16(db)))
        e_chosen = min(e for t, e in errs.items()
                       if float(from_bf16(bf16_np(np.float32(vmax) / -np.float32(7 + t / 16)))) == d_chosen)
        assert e_chosen <= min(errs.values()) * (1 + 1e-5) + 1e-30, trial


def _q2_codes(nib):
    """[nb * 8] Q2 bytes -> [nb][32] codes in element order (element e: bits
    2 (e // 8) of byte e % 8, engine_gpt2.rs:356-399)"""
    b = np.asarray(nib, np.uint8).reshape(-1, 8)
    return np.concatenate([(b >> (2 * k)) & 3 for k in range(4)], axis=1)


def test_q2_quant_known_answers():
    # values k * d0 with k in {-2, -1, 0, 1} and vmax = -2 * d0: scale
    # bf16(vmax / -2) = d0 exactly, every value reproduced (code k + 2)
    k = rng.integers(-2, 2, 32)
    k[3] = -2
    vals = (k * np.float32(-0.5)).astype(np.float32)            # vmax = +1.0
    nib, sc = O.q2_quant_row(bf16_np(vals))
    assert sc[0] == 0xBF00                                        # bf16(-0.5)
    assert np.array_equal(_q2_codes(nib)[0].astype(int) - 2, k)
    # byte j packs elements j, j + 8, j + 16, j + 24, two bits each, low first
    c = k + 2
    for j in range(8):
        assert nib[j] == c[j] | (c[j + 8] << 2) | (c[j + 16] << 4) | (c[j + 24] << 6)
    # clamping: a value beyond the scale's range takes code 0 or 3
    v2 = np.zeros(32, np.float32)
    v2[0], v2[1], v2[2] = 4.0, -4.0, -9.0                         # vmax = -9 -> scale bf16(4.5) = 4.5
    nib, sc = O.q2_quant_row(bf16_np(v2))
    cc = _q2_codes(nib)[0]
    # floor(4/4.5 + 2.5) = 3, floor(-4/4.5 + 2.5) = 1, floor(-2 + 2.5) = 0, zeros -> 2
    assert sc[0] == bf16_np(np.float32(4.5)) and list(cc[:4]) == [3, 1, 0, 2]
    # the zero block: vmax / -2 = -0.0 (bf16 0x8000), codes 2 (value 0)
    nib, sc = O.q2_quant_row(np.zeros(32, np.uint16))
    assert sc[0] == 0x8000 and np.all(nib == 0xAA)


def test_q2_row_dot_lane_order():
    d = 2880
    xq, xsb = _xq(d)
    w = bf16_np(rng.standard_normal(d).astype(np.float32) * 0.02)
    nib, sc = O.q2_quant_row(w)
    codes = _q2_codes(nib)
    a = [f32(0)] * 4
    for b in range(d // 32):
        sv = from_bf16(sc[b]) * xsb[b]
        for j in range(4):
            e = np.concatenate([np.arange(4 * j, 4 * j + 4), np.arange(16 + 4 * j, 20 + 4 * j)])
            t = int(((codes[b, e].astype(int) - 2) * xq[b * 32 + e]).sum())
            a[j] = fma32(f32(t), sv, a[j])
    want = f32(f32(a[0] + a[1]) + f32(a[2] + a[3]))
    assert O.q2_row_dot(nib, sc, xq, xsb) == want
    deq = ((codes.astype(np.float64) - 2) * from_bf16(sc)[:, None].astype(np.float64)).reshape(-1)
    ref = float((deq * xq.astype(np.float64) * np.repeat(xsb, 32)).sum())
    assert abs(float(want) - ref) <= 1e-5 * float(np.abs(deq * xq * np.repeat(xsb, 32)).sum())


def test_head_q2_screen_candidates():
    V, d, nt, cand = 1024, 256, 12, 8
    w = bf16_np(rng.standard_normal((V, d)).astype(np.float32) * 0.02)
    x = rng.standard_normal(d).astype(np.float32)
    out = O.head(w, x, np.ones(d, np.float32), 1e-5, nt, cand, q2=True)
    xq, xsb = out["xq"], out["xsb"]
    screen = np.array([O.q2_row_dot(*O.q2_quant_row(w[r]), xq, xsb) for r in range(V)], np.float32)
    ids = []
    for wid in range(nt):
        r0, r1 = 4 * O.head_slice_start(V // 4, nt, wid), 4 * O.head_slice_start(V // 4, nt, wid + 1)
        order = np.argsort(-screen[r0:r1].astype(np.float64), kind="stable")[:cand]
        ids += list(r0 + order)
    assert np.array_equal(out["cand_ids"], np.array(ids, np.int32))
    assert np.array_equal(out["cand_screen"], screen[ids])
    logits = np.array([O.q8_row_dot(*O.q8_quant_row(w[r]), xq, xsb) for r in ids], np.float32)
    assert np.array_equal(out["cand_logits"], logits)
    assert out["chosen"] == ids[int(np.argmax(logits))]


def test_q8_quant_row_closed_form():
    w = bf16_np(rng.standard_normal(512).astype(np.float32) * 0.05)
    q, s = O.q8_quant_row(w)
    v = from_bf16(w).reshape(-1, 32)
    amax = np.maximum(np.abs(v).max(1), f32(1e-12))
    assert np.array_equal(s, (amax / f32(127.0)).astype(np.float32))
    ratio = v / s[:, None]
    want = np.clip(np.sign(ratio) * np.floor(np.abs(ratio) + 0.5), -127, 127).astype(np.int8)
    assert np.array_equal(q, want.reshape(-1))


def _xq(d):
    x = rng.standard_normal(d).astype(np.float32)
    return O.qblock32(x)


def test_q4_and_q8_row_dots():
    d = 2880
    xq, xsb = _xq(d)
    w = bf16_np(rng.standard_normal(d).astype(np.float32) * 0.02)
    nib, sc = O.q4_quant_row(w)
    # numpy float32 restatement of the lane order (lane j: elements 4j..4j+3, 16+4j..)
    a = [f32(0)] * 4
    nb16 = nib.reshape(-1, 16)
    codes = np.stack([nb16 & 15, nb16 >> 4], 1)                          # [block][half][16]
    for b in range(d // 32):
        sv = from_bf16(sc[b]) * xsb[b]
        for j in range(4):
            e = np.arange(4 * j, 4 * j + 4)
            t = int(((codes[b, 0, e].astype(int) - 8) * xq[b * 32 + e]).sum() +
                    ((codes[b, 1, e].astype(int) - 8) * xq[b * 32 + 16 + e]).sum())
            a[j] = fma32(f32(t), sv, a[j])
    want = f32(f32(a[0] + a[1]) + f32(a[2] + a[3]))
    assert O.q4_row_dot(nib, sc, xq, xsb) == want
    # and against float64 of the dequantised row
    deq = ((codes.reshape(-1, 32).astype(np.float64) - 8)
           * from_bf16(sc)[:, None].astype(np.float64)).reshape(-1)
    ref = float((deq * xq.astype(np.float64) * np.repeat(xsb, 32)).sum())
    assert abs(float(want) - ref) <= 1e-5 * float(np.abs(deq * xq * np.repeat(xsb, 32)).sum())
    q, s = O.q8_quant_row(w)
    ref8 = float((q.astype(np.float64) * np.repeat(s, 32) * xq * np.repeat(xsb, 32)).sum())
    got8 = float(O.q8_row_dot(q, s, xq, xsb))
    assert abs(got8 - ref8) <= 1e-5 * float(np.abs(q * np.repeat(s, 32) * xq * np.repeat(xsb, 32)).sum())
    # the exact lane / accumulator order of dot_q8_i8 (even blocks -> acc0, odd -> acc1)
    a0, a1 = [f32(0)] * 4, [f32(0)] * 4
    for b in range(d // 32):
        sv = f32(s[b] * xsb[b])
        for j in range(4):
            e = np.r_[np.arange(4 * j, 4 * j + 4), np.arange(16 + 4 * j, 16 + 4 * j + 4)]
            t = int((q[b * 32 + e].astype(int) * xq[b * 32 + e]).sum())
            if b % 2 == 0:
                a0[j] = fma32(f32(t), sv, a0[j])
            else:
                a1[j] = fma32(f32(t), sv, a1[j])
    v = [f32(a0[j] + a1[j]) for j in range(4)]
    assert O.q8_row_dot(q, s, xq, xsb) == f32(f32(v[0] + v[1]) + f32(v[2] + v[3]))
    # odd block count: the last block goes into the first accumulator
    assert np.isfinite(O.q8_row_dot(q[:96], s[:3], xq[:96], xsb[:3]))


def test_head_candidates_and_greedy():
    V, d, nt, cand = 1024, 512, 12, 8
    w = bf16_np(rng.standard_normal((V, d)).astype(np.float32) * 0.02)
    x = rng.standard_normal(d).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    out = O.head(w, x, nw, 1e-5, nt, cand)
    xq, xsb = out["xq"], out["xsb"]
    xn = O.rmsnorm_gptoss(x, nw, 1e-5)
    xq2, xsb2 = O.qblock32(xn)
    assert np.array_equal(xq, xq2) and np.array_equal(xsb, xsb2)
    screen = np.array([O.q4_row_dot(*O.q4_quant_row(w[r]), xq, xsb) for r in range(V)], np.float32)
    nq = V // 4
    ids = []
    for wid in range(nt):
        r0, r1 = 4 * O.head_slice_start(nq, nt, wid), 4 * O.head_slice_start(nq, nt, wid + 1)
        order = np.argsort(-screen[r0:r1].astype(np.float64), kind="stable")[:cand]
        ids += list(r0 + order)
    assert np.array_equal(out["cand_ids"], np.array(ids, np.int32))
    assert np.array_equal(out["cand_screen"], screen[ids])
    logits = np.array([O.q8_row_dot(*O.q8_quant_row(w[r]), xq, xsb) for r in ids], np.float32)
    assert np.array_equal(out["cand_logits"], logits)
    assert out["chosen"] == ids[int(np.argmax(logits))]       # first maximum


def test_head_worker_slices_known_answers():
    # sl() weights workers 0-11 at 5 units and workers 12+ at 2
    # (engine_gpt2.rs:21-38, 636-642): with n equal to the total units the
    # slice starts are the unit offsets themselves
    assert [O.head_slice_start(68, 16, w) for w in range(17)] == \
        [0, 5, 10, 15, 20, 25, 30, 35, 40, 45, 50, 55, 60, 62, 64, 66, 68]
    assert [O.head_slice_start(100, 32, w) for w in range(33)] == \
        list(range(0, 60, 5)) + list(range(60, 101, 2))
    # gpt-oss vocabulary quads (201088 / 4 = 50272) over 16 workers (68
    # units): 50272 * 60 / 68 = 44357.6, * 62 / 68 = 45836.2, * 66 / 68 = 48793.4
    assert [O.head_slice_start(50272, 16, w) for w in (12, 13, 15, 16)] == [44357, 45836, 48793, 50272]
    # up to 12 workers every slice has the same weight: n * w / nt
    assert [O.head_slice_start(50272, 12, w) for w in (1, 5, 11)] == [50272 // 12, 50272 * 5 // 12, 50272 * 11 // 12]


def test_head_candidates_more_than_12_workers():
    # E-core workers (12+) get the narrower slices
    V, d, nt, cand = 1600, 128, 20, 4
    r = np.random.default_rng(5)
    w = bf16_np(r.standard_normal((V, d)).astype(np.float32) * 0.02)
    x = r.standard_normal(d).astype(np.float32)
    out = O.head(w, x, np.ones(d, np.float32), 1e-5, nt, cand)
    xq, xsb = out["xq"], out["xsb"]
    screen = np.array([O.q4_row_dot(*O.q4_quant_row(w[i]), xq, xsb) for i in range(V)], np.float32)
    units = [5 * k if k < 12 else 60 + 2 * (k - 12) for k in range(nt + 1)]
    ids = []
    for wid in range(nt):
        r0, r1 = 4 * (400 * units[wid] // units[nt]), 4 * (400 * units[wid + 1] // units[nt])
        order = np.argsort(-screen[r0:r1].astype(np.float64), kind="stable")[:cand]
        ids += list(r0 + order)
    assert np.array_equal(out["cand_ids"], np.array(ids, np.int32))


def test_head_prequantised_rows_agree():
    # the load-time Q4 quantisation split off (orc_head_pre) gives the same head
    r = np.random.default_rng(11)
    V, d = 512, 96
    w = r.integers(0, 0x7F00, (V, d), dtype=np.uint16) ^ (r.integers(0, 2, (V, d), dtype=np.uint16) << 15)
    x = r.standard_normal(d).astype(np.float32)
    nw = np.ones(d, np.float32)
    a = O.head(w, x, nw, 1e-5)
    pre = O.q4_quant_rows(w)
    for row in (0, 17, V - 1):
        nib, sc = O.q4_quant_row(w[row])
        assert np.array_equal(pre[0][row], nib) and np.array_equal(pre[1][row], sc)
    b = O.head(w, x, nw, 1e-5, pre=pre)
    for k in a:
        assert np.array_equal(np.asarray(a[k]), np.asarray(b[k])), k
