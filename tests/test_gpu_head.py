"""GPU parity of the two-stage LM head (head.hip) against the oracle
(oracle/head.c, pinned in tests/test_oracle_head.py): Q8 activations,
every row's Q4 (or Q2) screen value, the candidate set (ids in worker / rank order),
the candidates' exact Q8 logits and the greedy token, all bit for bit;
including tied rows (lower index first) and an odd block count."""
import numpy as np
import pytest

from cpubrrr_amd import LmHead
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


def bf16(a):
    b = np.asarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return (((b + 0x7FFF + ((b >> 16) & 1)) >> 16) & 0xFFFF).astype(np.uint16)


def run(V, d, seed, nt=12, cand=8, dup=False, full_screen=True, q2=False):
    say(f"case head V={V} d={d} seed={seed} nt={nt} cand={cand} dup={dup} q2={q2}")
    r = np.random.default_rng(seed)
    w = bf16(r.standard_normal((V, d)).astype(np.float32) * 0.02)
    if dup:
        # rows with identical weights tie exactly in both stages
        src = r.integers(0, V, 64)
        w[(src + V // 3) % V] = w[src]
    nw = (1 + 0.1 * r.standard_normal(d)).astype(np.float32)
    x = (r.standard_normal(d) * 3).astype(np.float32)
    with LmHead(d, V, 1e-5, nt, cand) as hd:
        hd.load(w, nw)
        if q2:
            hd.set_screen(2)
        ch, t = hd.forward(x, trace=True)
        ch2, _ = hd.forward(x)
    o = O.head(w, x, nw, 1e-5, nt, cand, q2=q2)
    assert ch == ch2
    assert np.array_equal(t["xq"], o["xq"]) and np.array_equal(t["xsb"].view(np.uint32), o["xsb"].view(np.uint32))
    rows = range(V) if full_screen else list(range(0, V, max(1, V // 300))) + list(o["cand_ids"])
    for row in rows:
        want = (O.q2_row_dot(*O.q2_quant_row(w[row]), o["xq"], o["xsb"]) if q2
                else O.q4_row_dot(*O.q4_quant_row(w[row]), o["xq"], o["xsb"]))
        assert t["screen"][row].view(np.uint32) == np.float32(want).view(np.uint32), row
    assert np.array_equal(t["cand_ids"], o["cand_ids"]), (t["cand_ids"], o["cand_ids"])
    assert np.array_equal(t["cand_screen"].view(np.uint32), o["cand_screen"].view(np.uint32))
    assert np.array_equal(t["cand_logits"].view(np.uint32), o["cand_logits"].view(np.uint32))
    assert ch == o["chosen"], (ch, o["chosen"])
    say(f"  ok chosen={ch}")


def test_head_small(gpu):
    run(4096, 512, 1)
    run(2048, 480, 2, nt=5, cand=3)          # odd block count (15), other worker split


def test_head_ties(gpu):
    run(4096, 256, 3, dup=True)


def test_head_gptoss_shape(gpu):
    # gpt-oss output.weight: 201088 x 2880
    run(201088, 2880, 4, full_screen=False)


def test_head_edge_shapes(gpu):
    # fewer row quads than workers: empty slices keep the reference's initial
    # entries (-FLT_MAX, row 0); a vocabulary that ends mid-tile and mid
    # workgroup; the largest worker x candidate product; one worker
    run(16, 64, 5, nt=12, cand=8)
    run(4, 32, 6, nt=3, cand=2)
    run(1000, 96, 7, nt=8, cand=16)
    run(2052, 128, 8, nt=1, cand=16)
    run(300, 64, 9, nt=32, cand=4, dup=True)


def test_head_q2_screen(gpu):
    # the reference's Q2 screen option (CPBRR_HEAD2): every row's Q2 value,
    # the candidates and the token bit-exact, at a small shape, with ties,
    # with 20 workers, and at gpt-oss's 201088 x 2880
    run(4096, 512, 11, q2=True)
    run(4096, 256, 12, dup=True, q2=True)
    run(1000, 96, 13, nt=20, cand=4, q2=True)
    run(201088, 2880, 14, full_screen=False, q2=True)
