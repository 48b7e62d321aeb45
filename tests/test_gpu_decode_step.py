"""A gpt-oss decode step entirely on the GPU: per layer the attention block
(attn.hip) then the MoE block (MoE decode kernels) on one stream over the same
device x, then the LM head (head.hip) -- the reference's forward_worker layer
loop and head_worker (engine_gpt2.rs:772-923, 937-1002) with no host round
trip between them.

Each stage is checked against the oracle on the stage's own GPU input (the
stages are pinned one by one elsewhere; this checks the composition: shared
stream, shared device x, the cache positions): attention and the MoE block
within 1e-3 of their update's RMS (attention is bit-exact where no Q8 code of
the heads' outputs moved, checked with its trace in tests/test_gpu_attn.py),
the head's token exactly.
Then the whole step is captured into one graph on the caller's stream and
replayed, bit-identical to the eager step on every replay."""
import numpy as np
import pytest

from cpubrrr_amd import Attention, LmHead, MoeBlock, MoeConfig, synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu

D, NH, NKV, NE, K, NL, V, SWA = 2880, 64, 8, 32, 4, 2, 4096, 4


def say(msg):
    print(msg, flush=True)


def _q8(L):
    Lq = dict(L)
    for n in ("q", "k", "v", "o"):
        Lq["w" + n], Lq["s" + n] = O.q8_rows(L["w" + n])
    return Lq


def test_decode_step_stagewise_and_graph(gpu):
    import torch
    say(f"case decode step d={D} layers={NL} experts={NE} vocab={V}")
    attn_l = [synth.attn_layer(D, NH, NKV, 64, seed=8, layer=l, swa=SWA) for l in range(NL)]
    attn_q = [_q8(L) for L in attn_l]
    moe_l = [synth.gptoss_layer(D, D, NE, K, seed=8, layer=l, zipf=1.1) for l in range(NL)]
    r = np.random.default_rng(8)
    w_out = synth.bf16(r.standard_normal((V, D)).astype(np.float32) * 0.02)
    n_out = (1 + 0.1 * r.standard_normal(D)).astype(np.float32)
    max_seq = 16
    tab = O.rope_table(64, max_seq, 150000.0)
    kc = [np.zeros((max_seq, NKV, 64), np.float32) for _ in range(NL)]
    vc = [np.zeros((max_seq, NKV, 64), np.float32) for _ in range(NL)]
    at = Attention(D, NH, NKV, NL, max_seq, SWA, 150000.0, 1e-5)
    moe = MoeBlock(MoeConfig.gptoss(d=D, n_expert=NE, top_k=K, d_ff=D, n_layer=NL))
    hd = LmHead(D, V)
    try:
        for l in range(NL):
            at.load_layer(l, attn_l[l])
            moe.load_layer(l, moe_l[l])
        hd.load(w_out, n_out)
        s = torch.cuda.Stream()
        for h in (at, moe, hd):
            h.set_stream(s.cuda_stream)
        ch = torch.zeros(1, dtype=torch.int32, device="cuda:0")
        n_exact = 0
        for pos in range(6):
            x = torch.from_numpy(synth.token(D, 8, pos) * 4).to("cuda:0")
            torch.cuda.synchronize()
            for l in range(NL):
                x_in = x.cpu().numpy()
                at.forward_device(l, pos, x.data_ptr())
                s.synchronize()
                x_att = x.cpu().numpy()
                xo, _ = O.attn_layer(attn_q[l], l, pos, x_in, kc[l], vc[l], tab)
                rms = np.sqrt(((xo - x_in) ** 2).mean())
                assert np.max(np.abs(x_att - xo)) <= 1e-3 * rms, (pos, l)
                n_exact += int(np.array_equal(x_att.view(np.uint32), xo.view(np.uint32)))
                moe.forward_device(l, 1, x.data_ptr(), 1, True)
                s.synchronize()
                x_moe = x.cpu().numpy()
                xm, _ = O.gptoss_moe(moe_l[l], x_att, True)
                rms = np.sqrt(((xm - x_att) ** 2).mean())
                assert np.max(np.abs(x_moe - xm)) <= 1e-3 * rms, (pos, l)
            hd.forward_device(x.data_ptr(), ch.data_ptr())
            s.synchronize()
            want = O.head(w_out, x.cpu().numpy(), n_out, 1e-5)["chosen"]
            assert int(ch.item()) == want, pos
        # one ulp in a head's output moves its Q8 code now and then (expf and the
        # softmax sums), so x after attention is compared to tolerance here; the
        # teacher-forced bit-exact check is tests/test_gpu_attn.py's
        say(f"  attention steps bit-exact: {n_exact} of {6 * NL}")

        # the whole step at position 6 as one graph on the caller's stream
        pos = 6
        x0 = torch.from_numpy(synth.token(D, 8, 100)).to("cuda:0")

        def step(xt):
            for l in range(NL):
                at.forward_device(l, pos, xt.data_ptr())
                moe.forward_device(l, 1, xt.data_ptr(), 1, True)
            hd.forward_device(xt.data_ptr(), ch.data_ptr())

        ref = x0.clone()
        step(ref)
        s.synchronize()
        ref_tok = int(ch.item())
        xg = x0.clone()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            step(xg)
        for rep in range(3):
            xg.copy_(x0)
            ch.zero_()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(xg.view(torch.int32), ref.view(torch.int32)), rep
            assert int(ch.item()) == ref_tok, rep
        for h in (at, moe, hd):
            h.set_stream(None)
    finally:
        hd.close()
        moe.close()
        at.close()
