"""CPU emulation of the GPU's MXFP4 block-sum decode (moe_common.h:
mx_block_sum) and of the stream layout (moe_mx.hip), checked against exact
integer block sums.  Pins the bit manipulation before it runs on a GPU.
"""
import numpy as np

from tests import f64ref as R

rng = np.random.default_rng(7)
M7, M4, SEL, TLO, THI = 0x07070707, 0x04040404, 0x03020100, 0x03020100, 0x0C080604


def perm(hi: int, lo: int, sel: int) -> int:
    """V_PERM_B32 restricted to selector bytes 0..7 (the only ones used)."""
    src = lo.to_bytes(4, "little") + hi.to_bytes(4, "little")
    out = 0
    for i in range(4):
        s = (sel >> (8 * i)) & 0xFF
        assert s < 8
        out |= src[s] << (8 * i)
    return out


def sdot4(a: int, b: int, c: int) -> int:
    av = np.frombuffer(a.to_bytes(4, "little"), np.int8).astype(np.int64)
    bv = np.frombuffer(b.to_bytes(4, "little"), np.int8).astype(np.int64)
    return c + int((av * bv).sum())


def neg4(v: int) -> int:
    b = np.frombuffer(v.to_bytes(4, "little"), np.int8).astype(np.int16)
    return int.from_bytes((-b).astype(np.int8).tobytes(), "little")


def mx_block_sum(q, xp, xn):
    S = 0
    for c in range(4):
        lo = q[c]
        ma = perm(THI, TLO, lo & M7)
        mb = perm(THI, TLO, (lo >> 4) & M7)
        sa = ((lo >> 1) & M4) | SEL
        sb = ((lo >> 5) & M4) | SEL
        xa = perm(xn[c], xp[c], sa)
        xb = perm(xn[4 + c], xp[4 + c], sb)
        S = sdot4(ma, xa, S)
        S = sdot4(mb, xb, S)
    return S


def test_block_sum_matches_exact():
    for _ in range(300):
        blk = rng.integers(0, 256, 17, dtype=np.uint8)
        xq = rng.integers(-127, 128, 32).astype(np.int8)
        if _ % 10 == 0:
            xq[:] = rng.choice([-127, 127], 32)
        q = [int.from_bytes(blk[1 + 4 * c:5 + 4 * c].tobytes(), "little") for c in range(4)]
        xd = [int.from_bytes(xq[4 * c:4 * c + 4].tobytes(), "little") for c in range(8)]
        xn = [neg4(v) for v in xd]
        got = mx_block_sum(q, xd, xn)
        assert got == int(R.mx_block_sums(blk, xq)[0])


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
    # decode through the stream layout exactly as k_gateup_mx indexes it
    from cpubrrr_amd import synth
    ne, dff, d = 2, 64, 480
    nb = d // 32
    gate = synth.mxfp4(ne * dff, nb, 3, 1)
    up = synth.mxfp4(ne * dff, nb, 3, 2)
    st = stream_gateup(gate, up, ne, dff, nb)
    xq = rng.integers(-127, 128, d).astype(np.int8)
    for e in range(ne):
        for t in range(dff // 32):
            for lane in (0, 5, 31, 32, 63):
                row = t * 32 + (lane & 31)
                src = (gate if lane < 32 else up)[e * dff + row]
                want = R.mx_block_sums(src, xq)
                for q in range((nb + 14) // 15):
                    ex = st[e, t, q, 0, lane]
                    for u in range(15):
                        blk = q * 15 + u
                        if blk >= nb:
                            continue
                        qb = st[e, t, q, u + 1, lane]
                        words = [int.from_bytes(qb[4 * c:4 * c + 4].tobytes(), "little") for c in range(4)]
                        xd = [int.from_bytes(xq[blk * 32 + 4 * c:blk * 32 + 4 * c + 4].tobytes(), "little")
                              for c in range(8)]
                        assert mx_block_sum(words, xd, [neg4(v) for v in xd]) == want[blk]
                        assert ex[u] == src.reshape(nb, 17)[blk, 0]
