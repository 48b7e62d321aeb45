"""GPU parity of the batched Qwen3 path (moe_grouped_kq.hip): tokens grouped
by expert, Q4_K / Q6_K products on the int8 matrix cores.  Like the
reference's k-wide dot q4k_dot_k (engine_qwen2.rs:115-163), it must give
per-token decode's results: every layer output and every integer superblock
sum is compared bit for bit with the per-token kernels (pinned to the oracle
by tests/test_gpu_kq.py), and the outputs also with the oracle."""
import numpy as np
import pytest

from cpubrrr_amd import MoeBlock, MoeConfig, synth
from oracle import oracle as O
from tests.grouped_ref import BatchCheck, grouped_expect

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("d,dff,ne,k,n_tok,seed,norm,down", [
    (512, 256, 8, 2, 19, 0, True, 14),
    (1024, 512, 32, 8, 40, 1, True, 14),
    (512, 512, 16, 4, 33, 2, False, 12),
    (2048, 768, 128, 8, 96, 3, True, 14),
    (2048, 768, 128, 8, 512, 4, True, 14),
])
def test_kq_grouped_equals_per_token(gpu, d, dff, ne, k, n_tok, seed, norm, down):
    say(f"case kq grouped d={d} dff={dff} ne={ne} k={k} n_tok={n_tok} down={down}")
    L = synth.qwen_layer(d, dff, ne, k, seed=seed, down_type=down)
    X = np.stack([synth.token(d, seed, 200 + i) for i in range(n_tok)])
    cfg = MoeConfig.qwen3(d=d, n_expert=ne, top_k=k, d_ff=dff, max_tokens=n_tok, down_type=down)
    with MoeBlock(cfg) as blk:
        blk.load_layer(0, L)
        Y, _ = blk.forward(0, X, apply_norm=norm)               # n_tok > 1: grouped path
        Y2, gs, ds = blk.grouped_sums(0, X, apply_norm=norm)
        assert np.array_equal(Y.view(np.uint32), Y2.view(np.uint32))
        bc = BatchCheck()
        for t in range(n_tok):
            y, tr = blk.forward(0, X[t], apply_norm=norm, trace=True)
            ye, _, order = grouped_expect(L, X[t], tr, "qwen")
            bc.add(Y[t], ye, X[t], t)
            if t % (7 if n_tok < 200 else 61) == 0:
                # grouped slot s is the reference's rank s: decode's slot order[s]
                for s in range(k):
                    assert np.array_equal(gs[t * k + s], tr["gu_sums"][order[s]]), ("gate/up sums", t, s)
                    assert np.array_equal(ds[t * k + s], tr["dn_sums"][order[s]]), ("down sums", t, s)
        bc.done()
    for t in range(0, n_tok, max(1, n_tok // 4)):
        yo, _ = O.qwen_moe(L, X[t], norm)
        rms = np.sqrt(((yo - X[t]).astype(np.float64) ** 2).mean())
        assert np.max(np.abs(Y[t] - yo)) <= 1e-3 * rms, t
