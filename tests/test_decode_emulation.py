"""CPU emulation of the GPU's exact MXFP4 block sums on the matrix cores
(mx_dev.h: load_win_act / load_act_frag / window_sums, moe_common.h: the fp8
activation image tables) and of the stream layout (moe_mx.hip), checked
against exact integer block sums.  Pins the lane mappings, the permlane
transposes and the image encoding before they run on a GPU.

MFMA operand layouts emulated (v_mfma_scale_f32_16x16x128_f8f6f4, A fp8,
B fp4, scales 1): A lane (m = l%16, g = l/16) holds K 16g..16g+15 in bytes
0-15 and K 64+16g.. in bytes 16-31; B lane (n = l%16, g) holds K 32g..32g+31
as nibbles, low nibble first; D lane l holds column l%16, rows 4(l/16)..+3.
"""
import numpy as np

from tests import f64ref as R

rng = np.random.default_rng(7)

E2M1 = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]


def e2m1(c: int) -> float:
    return (-1.0 if c & 8 else 1.0) * E2M1[c & 7]


def e4m3_int(v: int) -> int:
    """moe_common.h e4m3_int: exact encoding of 0 or a small integer."""
    if v == 0:
        return 0
    s, a = (0x80 if v < 0 else 0), abs(v)
    E = a.bit_length() - 1
    m = ((a >> (E - 3)) & 7) if E >= 3 else ((a << (3 - E)) & 7)
    return s | ((E + 7) << 3) | m


def e4m3_val(b: int) -> float:
    s = -1.0 if b & 0x80 else 1.0
    E, m = (b >> 3) & 15, b & 7
    return s * (m / 8 * 2.0 ** -6 if E == 0 else (1 + m / 8) * 2.0 ** (E - 7))


def perm(hi: int, lo: int, sel: int) -> int:
    """V_PERM_B32 restricted to selector bytes 0..7 (the only ones used)."""
    src = lo.to_bytes(4, "little") + hi.to_bytes(4, "little")
    return sum(src[(sel >> (8 * i)) & 0xFF] << (8 * i) for i in range(4))


def table4(f, c):
    return sum(f(4 * c + i) << (8 * i) for i in range(4))


H_T = [table4(lambda i: e4m3_int(32 * (i if i < 8 else i - 16)), c) for c in range(4)]
L_T = [table4(lambda i: e4m3_int(2 * i), c) for c in range(4)]


def nib_lookup(v: int, sh: int, t) -> int:
    i7 = (v >> sh) & 0x07070707
    lo, hi = perm(t[1], t[0], i7), perm(t[3], t[2], i7)
    return perm(hi, lo, ((v >> (sh + 1)) & 0x04040404) | 0x03020100)


def img_hi(v):
    return nib_lookup(v, 4, H_T)


def img_lo(v):
    return nib_lookup(v, 0, L_T)


def k_of_elem(j: int) -> int:
    return 2 * j if j < 16 else 2 * (j - 16) + 1


def image(xq: np.ndarray) -> np.ndarray:
    """The route kernel's image of a Q8 vector: per block [32h | 2l] in K order."""
    nb = len(xq) // 32
    img = np.zeros((nb, 64), np.uint8)
    for b in range(nb):
        for j in range(32):
            qb = int(np.uint8(xq[b * 32 + j]))
            img[b, k_of_elem(j)] = img_hi(qb) & 0xFF
            img[b, 32 + k_of_elem(j)] = img_lo(qb) & 0xFF
    return img


def test_image_tables_exact():
    for x in range(-127, 128):
        qb = x & 0xFF
        h, l = x >> 4, x - 16 * (x >> 4)
        assert e4m3_val(img_hi(qb) & 0xFF) == 32 * h
        assert e4m3_val(img_lo(qb) & 0xFF) == 2 * l
        assert 32 * h + 2 * l == 2 * x


# ---- registers: 64 lanes x 4 dwords ----
def swap32(a, b):
    a, b = a.copy(), b.copy()
    a[32:], b[:32] = b[:32].copy(), a[32:].copy()
    return a, b


def swap16(a, b):
    a, b = a.copy(), b.copy()
    for r in (1, 3):
        a[16 * r:16 * r + 16], b[16 * (r - 1):16 * r] = b[16 * (r - 1):16 * r].copy(), a[16 * r:16 * r + 16].copy()
    return a, b


def transpose_window(r):
    r = [x.copy() for x in r]
    r[0], r[2] = swap32(r[0], r[2])
    r[1], r[3] = swap32(r[1], r[3])
    r[0], r[1] = swap16(r[0], r[1])
    r[2], r[3] = swap16(r[2], r[3])
    return r


def mfma(A, B):
    """A: [64 lanes][32 bytes] fp8, B: [64 lanes][16 bytes] fp4 -> D [64 lanes][4]."""
    Am = np.zeros((16, 128))
    Bm = np.zeros((128, 16))
    for l in range(64):
        m, g = l % 16, l // 16
        for j in range(16):
            Am[m, 16 * g + j] = e4m3_val(int(A[l][j]))
            Am[m, 64 + 16 * g + j] = e4m3_val(int(A[l][16 + j]))
        for i in range(16):
            byte = int(B[l][i])
            Bm[32 * g + 2 * i, m] = e2m1(byte & 15)
            Bm[32 * g + 2 * i + 1, m] = e2m1(byte >> 4)
    D = Am @ Bm                                    # exact: small integers
    return np.array([[D[4 * (l // 16) + i, l % 16] for i in range(4)] for l in range(64)])


def act_fragment(img, wb, u0, nb, lane):
    """load_act_frag: the 16 bytes lane `lane` holds for window block wb."""
    m, g = lane % 16, lane // 16
    bi = (0 if m < 4 else 2) + (g >> 1)
    if m < 8 and (m >> 1) == bi and u0 + bi < 15 and wb + bi < nb:
        o = (m & 1) * 32 + (g & 1) * 16
        return img[wb + bi, o:o + 16]
    return np.zeros(16, np.uint8)


def act_operand(frag, lane):
    z = np.zeros(16, np.uint8)
    return np.concatenate([frag, z]) if lane % 16 < 4 else np.concatenate([z, frag])


def window_sums(regs, afn):
    """regs[0..3]: [64 lanes][16 bytes] = each lane's row, window blocks 0..3."""
    t = transpose_window([np.array(r) for r in regs])
    sa, sb = [], []
    for k in range(4):
        A = np.array([afn(k, l) for l in range(64)])
        D = mfma(A, t[k])
        sa.append(D[:, 0] + D[:, 1])
        sb.append(D[:, 2] + D[:, 3])
    sa[0], sa[2] = swap32(sa[0], sa[2])
    sa[1], sa[3] = swap32(sa[1], sa[3])
    sa[0], sa[1] = swap16(sa[0], sa[1])
    sb[0], sb[2] = swap32(sb[0], sb[2])
    sb[1], sb[3] = swap32(sb[1], sb[3])
    sb[0], sb[1] = swap16(sb[0], sb[1])
    return [sa[0], sb[0], sa[1], sb[1]]           # per lane: blocks 0, 1, 2, 3


def test_window_sums_one_vector():
    """Gate/up: 64 rows x 4 blocks against one activation vector."""
    nb = 8
    for trial in range(3):
        rows = [rng.integers(0, 256, nb * 17, dtype=np.uint8) for _ in range(64)]
        xq = rng.integers(-127, 128, nb * 32).astype(np.int8)
        if trial == 2:
            xq[:] = rng.choice([-127, 127], nb * 32)
        img = image(xq)
        for wb in (0, 4):
            regs = [np.array([rows[l].reshape(nb, 17)[wb + k, 1:] for l in range(64)]) for k in range(4)]

            def afn(k, l):
                m, g = l % 16, l // 16
                lo = hi = np.zeros(16, np.uint8)
                if m < 8 and (m >> 1) == (g >> 1):
                    o = (m & 1) * 32 + (g & 1) * 16
                    lo = img[wb + (g >> 1), o:o + 16]
                if m < 8 and (m >> 1) == 2 + (g >> 1):
                    o = (m & 1) * 32 + (g & 1) * 16
                    hi = img[wb + 2 + (g >> 1), o:o + 16]
                return np.concatenate([lo, hi])

            S = window_sums(regs, afn)
            for l in range(64):
                want = R.mx_block_sums(rows[l], xq)
                for k in range(4):
                    assert S[k][l] == want[wb + k], (trial, wb, l, k)


def test_window_sums_vector_per_group():
    """Down: 16-lane group g uses expert slot g's activation vector."""
    nb = 4
    rows = [rng.integers(0, 256, nb * 17, dtype=np.uint8) for _ in range(64)]
    xqs = [rng.integers(-127, 128, nb * 32).astype(np.int8) for _ in range(4)]
    imgs = [image(x) for x in xqs]
    regs = [np.array([rows[l].reshape(nb, 17)[k, 1:] for l in range(64)]) for k in range(4)]
    S = window_sums(regs, lambda k, l: act_operand(act_fragment(imgs[k], 0, 0, nb, l), l))
    for l in range(64):
        want = R.mx_block_sums(rows[l], xqs[l // 16])
        for k in range(4):
            assert S[k][l] == want[k]


def test_fragment_zero_past_kpart_and_row():
    """Blocks beyond the k-part (u0 + bi >= 15) or the row (>= nb) read zero;
    every other live (m < 8, m/2 == bi) fragment is the image's."""
    img = np.full((32, 64), 0x38, np.uint8)
    for wb, u0, nb in ((12, 12, 32), (28, 0, 30)):
        for l in range(64):
            m, g = l % 16, l // 16
            bi = (0 if m < 4 else 2) + (g >> 1)
            live = m < 8 and (m >> 1) == bi
            exists = u0 + bi < 15 and wb + bi < nb
            assert act_fragment(img, wb, u0, nb, l).any() == (live and exists), (wb, l)


def stream_gateup(gate, up, ne, dff, nb):
    """Python restatement of k_repack_gateup's output, unit (e,t,q,u,lane)."""
    P = (nb + 14) // 15
    out = np.zeros((ne, dff // 32, P, 16, 64, 16), np.uint8)
    for e in range(ne):
        for t in range(dff // 32):
            for lane in range(64):
                row = t * 32 + (lane & 31)
                src = (gate if lane < 32 else up)[e * dff + row].reshape(nb, 17)
                for q in range(P):
                    for u in range(16):
                        if u == 0:
                            for i in range(15):
                                if q * 15 + i < nb:
                                    out[e, t, q, 0, lane, i] = src[q * 15 + i, 0]
                        elif q * 15 + u - 1 < nb:
                            out[e, t, q, u, lane] = src[q * 15 + u - 1, 1:]
    return out


def test_stream_layout_roundtrip_sums():
    # block sums through the stream layout exactly as k_gateup_mx indexes it:
    # sub-part hh of k-part q = units 1 + 8hh .. (two windows), unit 16 absent
    from cpubrrr_amd import synth
    ne, dff, d = 1, 64, 480
    nb = d // 32
    gate = synth.mxfp4(ne * dff, nb, 3, 1)
    up = synth.mxfp4(ne * dff, nb, 3, 2)
    st = stream_gateup(gate, up, ne, dff, nb)
    xq = rng.integers(-127, 128, d).astype(np.int8)
    img = image(xq)
    zero = np.zeros((64, 16), np.uint8)
    for t in range(dff // 32):
        want = [R.mx_block_sums((gate if l < 32 else up)[t * 32 + (l & 31)], xq) for l in range(64)]
        for q in range((nb + 14) // 15):
            for hh in range(2):
                ub = 8 * hh
                units = [st[0, t, q, 1 + ub + i] if ub + i < 15 else zero for i in range(8)]
                for w in range(2):
                    wb = q * 15 + ub + 4 * w

                    def afn(k, l, wb=wb, u0=ub + 4 * w):
                        m, g = l % 16, l // 16
                        lo = hi = np.zeros(16, np.uint8)
                        for half in (0, 1):
                            bi = (g >> 1) + 2 * half
                            if m < 8 and (m >> 1) == bi and u0 + bi < 15 and wb + bi < nb:
                                o = (m & 1) * 32 + (g & 1) * 16
                                if half == 0:
                                    lo = img[wb + bi, o:o + 16]
                                else:
                                    hi = img[wb + bi, o:o + 16]
                        return np.concatenate([lo, hi])

                    S = window_sums(units[4 * w:4 * w + 4], afn)
                    for l in (0, 7, 31, 32, 50, 63):
                        for k in range(4):
                            blk = wb + k
                            if ub + 4 * w + k < 15 and blk < nb:
                                assert S[k][l] == want[l][blk]
                            else:
                                assert S[k][l] == 0
        for lane in (0, 33):
            src = (gate if lane < 32 else up)[t * 32 + (lane & 31)].reshape(nb, 17)
            for q in range((nb + 14) // 15):
                for u in range(15):
                    if q * 15 + u < nb:
                        assert st[0, t, q, 0, lane, u] == src[q * 15 + u, 0]
