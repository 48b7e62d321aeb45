"""GPU parity of the grouped (n_tok > 1) MXFP4 path: tokens grouped by expert,
expert products on the matrix cores.  The reference's batched tile path
computes what its per-token decode computes (engine_gpt2.rs:1120-1239).
Here the batched router evaluates the reference's own serial fp32 logits, so
the selection and weights are the reference's (tests/grouped_ref.py), and
the expert products are per-token decode's: every int32 block sum is
compared bit for bit with the per-token kernels (whose block sums
tests/test_gpu_mx.py pins to the oracle), every layer output with the
reference's combine of those rows (within an expf ulp of the weights; most
tokens bit for bit), and the outputs with the oracle to tolerance.
"""
import numpy as np
import pytest

from cpubrrr_amd import MoeBlock, MoeConfig, synth
from oracle import oracle as O
from tests.grouped_ref import BatchCheck, grouped_expect

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


def tokens(d, n, seed):
    return np.stack([synth.token(d, seed, 100 + i) for i in range(n)])


def per_token(blk, X, apply_norm):
    return np.stack([blk.forward(0, X[i], apply_norm=apply_norm)[0] for i in range(X.shape[0])])


@pytest.mark.parametrize("d,dff,ne,k,n_tok,seed,norm,zipf", [
    (480, 480, 8, 4, 37, 0, True, None),
    (960, 480, 16, 2, 70, 1, False, None),
    (512, 1024, 4, 1, 33, 2, True, None),
    (2880, 2880, 32, 4, 64, 3, True, 1.1),
    (960, 960, 32, 8, 45, 4, True, 1.1),
    (480, 480, 8, 3, 29, 5, False, None),
    # 1100 tokens x 128 experts: past the token x expert table's LDS size,
    # so the pairs are grouped by the ranking kernel (k_group), not k_group_dense
    (384, 64, 128, 4, 1100, 6, True, None),
    # 1024 x 128: the table at its largest (128 KB), still k_group_dense
    (384, 64, 128, 4, 1024, 7, True, None),
])
def test_grouped_equals_per_token(gpu, d, dff, ne, k, n_tok, seed, norm, zipf):
    say(f"case grouped d={d} dff={dff} ne={ne} k={k} n_tok={n_tok} seed={seed} norm={norm} zipf={zipf}")
    L = synth.gptoss_layer(d, dff, ne, k, seed=seed, zipf=zipf)
    X = tokens(d, n_tok, seed)
    with MoeBlock(MoeConfig.gptoss(d=d, n_expert=ne, top_k=k, d_ff=dff, max_tokens=n_tok)) as blk:
        blk.load_layer(0, L)
        Y, _ = blk.forward(0, X, apply_norm=norm)          # n_tok > 1: grouped path
        bc = BatchCheck()
        for i in range(n_tok):
            _, tr = blk.forward(0, X[i], apply_norm=norm, trace=True)
            ye, _, _ = grouped_expect(L, X[i], tr, "gptoss")
            bc.add(Y[i], ye, X[i], i)
        bc.done()
    # and against the oracle, to max-abs <= 1e-3 * RMS of the output
    for i in range(0, n_tok, max(1, n_tok // 5)):
        yo, _ = O.gptoss_moe(L, X[i], norm)
        rms = np.sqrt(((yo - X[i]).astype(np.float64) ** 2).mean())
        assert np.max(np.abs(Y[i] - yo)) <= 1e-3 * rms


def test_grouped_block_sums_bit_exact(gpu):
    d, dff, ne, k, n_tok = 960, 960, 16, 4, 40
    say(f"case grouped block sums d={d} n_tok={n_tok}")
    L = synth.gptoss_layer(d, dff, ne, k, seed=7, zipf=1.1)
    X = tokens(d, n_tok, 7)
    with MoeBlock(MoeConfig.gptoss(d=d, n_expert=ne, top_k=k, d_ff=dff, max_tokens=n_tok)) as blk:
        blk.load_layer(0, L)
        Y, gs, ds = blk.grouped_sums(0, X, apply_norm=True)
        bc = BatchCheck()
        for t in range(n_tok):
            y, tr = blk.forward(0, X[t], apply_norm=True, trace=True)
            ye, _, order = grouped_expect(L, X[t], tr, "gptoss")
            bc.add(Y[t], ye, X[t], t)
            # grouped slot s is the reference's rank s: decode's slot order[s]
            for s in range(k):
                assert np.array_equal(gs[t * k + s], tr["gu_sums"][order[s]]), ("gate/up sums", t, s)
                assert np.array_equal(ds[t * k + s], tr["dn_sums"][order[s]]), ("down sums", t, s)
        bc.done()


def test_grouped_falls_back_on_special_scales(gpu):
    # an e8m0 byte of 0 (tbl[0] = 0 in the reference) cannot be a hardware
    # scale: such a layer runs the per-token kernels and stays exact
    d, dff, ne, k, n_tok = 480, 480, 8, 4, 9
    say("case grouped fallback (e8m0 = 0 present)")
    L = synth.gptoss_layer(d, dff, ne, k, seed=8)
    g = L["gate"].reshape(-1, 17)
    g[::97, 0] = 0
    X = tokens(d, n_tok, 8)
    with MoeBlock(MoeConfig.gptoss(d=d, n_expert=ne, top_k=k, d_ff=dff, max_tokens=n_tok)) as blk:
        blk.load_layer(0, L)
        Y, _ = blk.forward(0, X, apply_norm=True)
        Yt = per_token(blk, X, True)
    assert np.array_equal(Y.view(np.uint32), Yt.view(np.uint32))
    for i in range(n_tok):
        yo, _ = O.gptoss_moe(L, X[i], True)
        rms = np.sqrt(((yo - X[i]).astype(np.float64) ** 2).mean())
        assert np.max(np.abs(Y[i] - yo)) <= 1e-3 * rms
