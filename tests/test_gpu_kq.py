"""GPU parity of the Qwen3 (Q4_K gate/up, Q6_K or Q4_K down) decode path
against the oracle.

Bit-exact: xn, Q8_K activation bytes / scales / per-32 sums, expert ids,
int32 superblock sums (sumi, mint) of gate/up and (given the same hq) of
down, and the gate/up row outputs (each is a serial fp32 sum over
superblocks of the reference's own float terms).  To tolerance: router
logits (serial-sum bound), softmax weights, h = SiLU(g)*u (expf), hq (+-1 on
a few bytes) and the layer output (max-abs <= 1e-3 * RMS of the FFN output).
"""
import numpy as np
import pytest

from cpubrrr_amd import MoeBlock, MoeConfig, synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


def check_qwen(L, x, apply_norm, xo, t):
    xo_o, to = O.qwen_moe(L, x, apply_norm, want_sums=True)
    d, dff, k = L["d"], L["dff"], L["k"]
    assert np.array_equal(t["xn"].view(np.uint32), to["xn"].view(np.uint32)), "xn"
    assert np.array_equal(t["xq"], to["xq"]), "xq"
    assert np.array_equal(t["xsb"].view(np.uint32), to["xsb"].view(np.uint32)), "ys"
    assert np.array_equal(t["xsum"], to["xsum"]), "xsum"
    assert np.array_equal(t["ids"], to["ids"]), (t["ids"], to["ids"])
    assert np.allclose(t["logits"], to["logits"], rtol=0, atol=2e-4 + 1e-6 * np.abs(to["logits"]).max())
    assert np.allclose(t["wts"], to["wts"], rtol=2e-5, atol=1e-7)
    assert np.array_equal(t["gu_sums"], to["gu_sums"]), "gate/up superblock sums"
    assert np.array_equal(t["gu"].view(np.uint32), to["gu"].view(np.uint32)), "gate/up outputs (bit-exact)"
    assert np.allclose(t["h"], to["h"], rtol=2e-6, atol=1e-30), "h"
    dq = t["hq"].astype(np.int32) - to["hq"].astype(np.int32)
    assert np.abs(dq).max() <= 1 and np.count_nonzero(dq) <= max(2, dq.size // 1000), "hq"
    assert np.allclose(t["hsb"], to["hsb"], rtol=1e-5), "hs"
    # down superblock sums from the GPU's own hq / hs / hsum: exact
    nsbf = dff // 256
    dt = L.get("down_type", 14)
    rb = nsbf * (144 if dt == 12 else 210)
    for ei in range(k):
        e = t["ids"][ei]
        hq, hs, hm = t["hq"][ei], t["hsb"][ei], t["hsum"][ei]
        for r in range(0, d, max(1, d // 61)):
            row = L["down"].reshape(-1)[(e * d + r) * rb:(e * d + r + 1) * rb]
            if dt == 12:
                v, s = O.q4k_dot(row, hq, hs, hm)
                assert np.array_equal(t["dn_sums"][ei, r].reshape(-1), s), ("down sums", ei, r)
            else:
                v, s = O.q6k_dot(row, hq, hs)
                assert np.array_equal(t["dn_sums"][ei, r], s), ("down sums", ei, r)
            # the row output itself is bit-exact given the same activations
            assert np.float32(v).view(np.uint32) == np.float32(t["dn"][ei, r]).view(np.uint32), ("down out", ei, r)
    ffn_o = (xo_o - x).astype(np.float64)
    ffn_g = (xo - x).astype(np.float64)
    rms = np.sqrt((ffn_o ** 2).mean())
    if np.count_nonzero(dq):
        # an hq byte differs (expf upstream, unpinned): check the down rows and
        # the combine (engine_qwen2.rs:425-432) on the GPU's own hq / hs / hsum
        s = np.array(x, np.float32, copy=True)
        for ei in range(k):
            e = int(t["ids"][ei])
            v = np.empty(d, np.float32)
            for r in range(d):
                row = L["down"].reshape(-1)[(e * d + r) * rb:(e * d + r + 1) * rb]
                v[r] = (O.q4k_dot(row, t["hq"][ei], t["hsb"][ei], t["hsum"][ei]) if dt == 12
                        else O.q6k_dot(row, t["hq"][ei], t["hsb"][ei]))[0]
            s = (s + np.float32(to["wts"][ei]) * v).astype(np.float32)
        ffn_o = s.astype(np.float64) - x
    err = np.max(np.abs(ffn_g - ffn_o))
    assert err <= 1e-3 * rms, (err, rms, np.count_nonzero(dq))
    return err / rms


def run_qwen(d, dff, ne, k, seed=0, layer=0, apply_norm=True, down_type=14):
    say(f"case qwen d={d} dff={dff} ne={ne} k={k} seed={seed} layer={layer} norm={apply_norm} down={down_type}")
    L = synth.qwen_layer(d, dff, ne, k, seed=seed, layer=layer, down_type=down_type)
    cfg = MoeConfig.qwen3(d=d, n_expert=ne, top_k=k, d_ff=dff, down_type=down_type)
    with MoeBlock(cfg) as blk:
        blk.load_layer(0, L)
        x = synth.token(d, seed, layer)
        xo, t = blk.forward(0, x, apply_norm=apply_norm, trace=True)
        rel = check_qwen(L, x, apply_norm, xo, t)
        xo2, _ = blk.forward(0, x, apply_norm=apply_norm)
        assert np.array_equal(xo2.view(np.uint32), xo.view(np.uint32)), "traced and untraced kernels differ"
    say(f"  ok rel_err={rel:.3e} fallback={t['exact_router_fallbacks']}")


def test_qwen_small_shapes(gpu):
    run_qwen(512, 256, 8, 2)
    run_qwen(768, 512, 16, 4, seed=1, apply_norm=False)
    run_qwen(1024, 768, 32, 8, seed=2)
    run_qwen(256, 256, 4, 1, seed=3)


def test_qwen_q4k_down(gpu):
    run_qwen(512, 512, 16, 8, seed=4, down_type=12)


def test_qwen_config3_layer(gpu):
    # bench config 3 layer shape: d 2048, 128 experts, top-8, d_ff 768
    for layer in (0, 5):
        run_qwen(2048, 768, 128, 8, seed=0, layer=layer)


def test_qwen_stack_device(gpu):
    import torch
    say("case qwen 3-layer device stack")
    d, dff, ne, k, nl = 2048, 768, 128, 8, 3
    layers = [synth.qwen_layer(d, dff, ne, k, seed=0, layer=l) for l in range(nl)]
    cfg = MoeConfig.qwen3(d=d, n_expert=ne, top_k=k, d_ff=dff, n_layer=nl)
    x = synth.token(d, 0, 0)
    with MoeBlock(cfg) as blk:
        for l in range(nl):
            blk.load_layer(l, layers[l])
        xd = torch.from_numpy(x.copy()).to("cuda:0")
        torch.cuda.synchronize()
        blk.forward_device(0, nl, xd.data_ptr(), 1, True)
        blk.sync()
        y = xd.cpu().numpy()
    xr = x.copy()
    for l in range(nl):
        xr, _ = O.qwen_moe(layers[l], xr, True)
    rms = np.sqrt(((xr - x).astype(np.float64) ** 2).mean())
    assert np.max(np.abs(y - xr)) <= 1e-3 * rms


def test_qwen_router_tie_128_experts(gpu):
    # 128 experts: the workgroup-ranked selection.  The experts ranked 8th and
    # 9th get identical router rows, so their logits tie exactly at the top-8
    # boundary: the certification must fail, the exact serial logits decide,
    # and the lower index wins (engine_qwen2.rs:403-410)
    say("case qwen router tie, 128 experts")
    d, dff, ne, k = 1024, 256, 128, 8
    L = synth.qwen_layer(d, dff, ne, k, seed=7)
    x = synth.token(d, 7)
    _, to = O.qwen_moe(L, x, True, want_sums=True)
    order = np.argsort(-to["logits"].astype(np.float64), kind="stable")
    a, b = order[k - 1], order[k]
    L["router_w"][max(a, b)] = L["router_w"][min(a, b)]
    cfg = MoeConfig.qwen3(d=d, n_expert=ne, top_k=k, d_ff=dff)
    with MoeBlock(cfg) as blk:
        blk.load_layer(0, L)
        xo, t = blk.forward(0, x, apply_norm=True, trace=True)
        assert t["exact_router_fallbacks"] == 1
        assert min(a, b) in t["ids"] and max(a, b) not in t["ids"], (a, b, t["ids"])
        check_qwen(L, x, True, xo, t)
        xo2, _ = blk.forward(0, x, apply_norm=True)
        assert np.array_equal(xo2.view(np.uint32), xo.view(np.uint32))


def test_qwen_mixed_down_types_per_layer(gpu):
    # Q4_K_M files mix Q6_K and Q4_K ffn_down across layers; each layer's
    # tensors carry their own GGUF type (engine_qwen2.rs:202-233)
    import torch
    say("case qwen mixed down types: layer 0 Q6_K, layer 1 Q4_K")
    d, dff, ne, k = 1024, 512, 32, 8
    layers = [synth.qwen_layer(d, dff, ne, k, seed=13, layer=0, down_type=14),
              synth.qwen_layer(d, dff, ne, k, seed=13, layer=1, down_type=12)]
    cfg = MoeConfig.qwen3(d=d, n_expert=ne, top_k=k, d_ff=dff, n_layer=2, down_type=14)
    x0 = synth.token(d, 13, 0)
    with MoeBlock(cfg) as blk:
        # a type the k-quant kernels do not take is rejected, not misread
        bad = dict(layers[1], down_type=39)
        with pytest.raises(Exception) as ei:
            blk.load_layer(1, bad)
        assert getattr(ei.value, "code", None) == -22
        x = x0.copy()
        for l, L in enumerate(layers):
            blk.load_layer(l, L)
            xo, t = blk.forward(l, x, apply_norm=True, trace=True)
            check_qwen(L, x, True, xo, t)
            x = xo
        xd = torch.from_numpy(x0.copy()).to("cuda:0")
        torch.cuda.synchronize()
        blk.forward_device(0, 2, xd.data_ptr(), 1, True)
        blk.sync()
        y = xd.cpu().numpy()
    assert np.array_equal(y.view(np.uint32), x.view(np.uint32))
