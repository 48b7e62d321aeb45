"""The no-allocation entry point (cpb_moe_forward_device_noalloc, static
per-GPU scratch) against cpb_moe_forward_device, bit for bit, on two calls in
a row (the second with a smaller input), for both weight families, and its
size limit.  It runs the per-token kernels for every token, so a batch is
compared with single-token cpb_moe_forward_device calls (a batched
forward_device takes the grouped path).  Runs last: it shares one device
array across handles."""
import numpy as np
import pytest

from cpubrrr_amd import MoeBlock, MoeConfig, synth
from cpubrrr_amd import _lib as L

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


def _pair(blk, X, n_tok, nl, norm):
    import torch
    a = torch.from_numpy(np.ascontiguousarray(X[:n_tok])).to("cuda:0")
    b = a.clone()
    torch.cuda.synchronize()
    for t in range(n_tok):                     # single-token calls
        blk.forward_device(0, nl, a[t].data_ptr(), 1, norm)
    blk.sync()
    blk.forward_device_noalloc(0, nl, b.data_ptr(), n_tok, norm)
    blk.sync()
    return a.cpu().numpy(), b.cpu().numpy()


def test_noalloc_matches_forward_device_mx(gpu):
    say("case noalloc gpt-oss: n_tok 4 then 2, 2 layers")
    d, ne, k, nl = 960, 16, 4, 2
    layers = [synth.gptoss_layer(d, d, ne, k, seed=31, layer=l, zipf=1.1) for l in range(nl)]
    X = np.stack([synth.token(d, 31, i) for i in range(4)])
    with MoeBlock(MoeConfig.gptoss(d=d, n_expert=ne, top_k=k, d_ff=d, n_layer=nl, max_tokens=4)) as blk:
        for l in range(nl):
            blk.load_layer(l, layers[l])
        for n_tok in (4, 2):
            want, got = _pair(blk, X, n_tok, nl, True)
            assert np.array_equal(want.view(np.uint32), got.view(np.uint32)), n_tok


def test_noalloc_matches_forward_device_qwen(gpu):
    say("case noalloc qwen: n_tok 3 then 1")
    d, dff, ne, k = 1024, 512, 32, 8
    L0 = synth.qwen_layer(d, dff, ne, k, seed=32)
    X = np.stack([synth.token(d, 32, i) for i in range(3)])
    with MoeBlock(MoeConfig.qwen3(d=d, n_expert=ne, top_k=k, d_ff=dff, max_tokens=3)) as blk:
        blk.load_layer(0, L0)
        for n_tok in (3, 1):
            want, got = _pair(blk, X, n_tok, 1, True)
            assert np.array_equal(want.view(np.uint32), got.view(np.uint32)), n_tok


def test_noalloc_under_graph_capture(gpu):
    # the entry point's purpose: a caller capturing its stream into a graph.
    # Captured into a torch CUDA graph on the handle's stream and replayed
    # three times, with eager work and synchronisations between the replays;
    # every replay equals the eager call bit for bit, and the calls change
    # the device's free memory by nothing
    import torch
    say("case noalloc captured in a graph, 3 replays")
    d, ne, k, nl = 960, 16, 4, 2
    layers = [synth.gptoss_layer(d, d, ne, k, seed=33, layer=l, zipf=1.1) for l in range(nl)]
    X = np.stack([synth.token(d, 33, i) for i in range(3)])
    with MoeBlock(MoeConfig.gptoss(d=d, n_expert=ne, top_k=k, d_ff=d, n_layer=nl)) as blk:
        for l in range(nl):
            blk.load_layer(l, layers[l])
        s = torch.cuda.Stream()
        blk.set_stream(s.cuda_stream)
        want = []
        for i in range(3):
            a = torch.from_numpy(X[i].copy()).to("cuda:0")
            torch.cuda.synchronize()
            blk.forward_device_noalloc(0, nl, a.data_ptr(), 1, True)
            blk.sync()
            want.append(a.cpu().numpy())
        free0 = torch.cuda.mem_get_info()[0]
        for i in range(3):
            a = torch.from_numpy(X[i].copy()).to("cuda:0")
            torch.cuda.synchronize()
            blk.forward_device_noalloc(0, nl, a.data_ptr(), 1, True)
            blk.sync()
        assert torch.cuda.mem_get_info()[0] == free0
        xs = torch.from_numpy(X[0].copy()).to("cuda:0")
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            blk.forward_device_noalloc(0, nl, xs.data_ptr(), 1, True)
        for i in (1, 0, 2):
            xs.copy_(torch.from_numpy(X[i]).to("cuda:0"))
            junk = torch.ones(4096, device="cuda:0") * float(i)      # eager work between replays
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(xs.cpu().numpy().view(np.uint32), want[i].view(np.uint32)), i
            del junk
        blk.set_stream(None)


def test_noalloc_rejects_shapes_beyond_scratch(gpu):
    say("case noalloc size limit")
    cfg = MoeConfig.qwen3(d=8192, n_expert=8, top_k=8, d_ff=4096)
    with MoeBlock(cfg) as blk:
        with pytest.raises(L.CpbError) as ei:
            blk.forward_device_noalloc(0, 1, 0x1000, 1, True)
        assert ei.value.code == L.CPB_EINVAL and "static scratch" in str(ei.value)
