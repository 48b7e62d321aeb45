"""MoE layers loaded straight from a mapped GGUF file (cpb_moe_load_gguf_layer)
run bit-identically to the same tensors passed as arrays, for gpt-oss (MXFP4,
biases) and Qwen3 (Q4_K gate/up, a Q6_K and a Q4_K down layer); tensors of
the wrong type or shape are rejected (engine_gpt2.rs:600-617 asserts)."""
import numpy as np
import pytest

from cpubrrr_amd import GgufFile, MoeBlock, synth
from cpubrrr_amd import _lib as L
from tests import gguf_writer as W

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


def _same_as_arrays(g, layers, apply_norm, x):
    cfg = g.moe_config()
    with MoeBlock(cfg) as a, MoeBlock(cfg) as b:
        for l, Lr in enumerate(layers):
            a.load_gguf_layer(g, l)
            b.load_layer(l, Lr)
        for l in range(len(layers)):
            ya, ta = a.forward(l, x, apply_norm=apply_norm, trace=True)
            yb, tb = b.forward(l, x, apply_norm=apply_norm, trace=True)
            assert np.array_equal(ya.view(np.uint32), yb.view(np.uint32)), l
            assert np.array_equal(ta["ids"], tb["ids"]) and np.array_equal(ta["dn_sums"], tb["dn_sums"])


def test_gptoss_from_gguf(gpu, tmp_path):
    say("case gguf gpt-oss 2 layers")
    d, dff, ne, k = 960, 480, 16, 4
    layers = [synth.gptoss_layer(d, dff, ne, k, seed=41, layer=l, zipf=1.1) for l in range(2)]
    path = tmp_path / "g.gguf"
    W.moe_model(path, "gptoss", layers, d, dff, ne, k, 1e-5)
    with GgufFile(path) as g:
        _same_as_arrays(g, layers, True, synth.token(d, 41, 0))


def test_qwen_from_gguf_mixed_down(gpu, tmp_path):
    say("case gguf qwen Q6_K + Q4_K down")
    d, dff, ne, k = 1024, 512, 32, 8
    layers = [synth.qwen_layer(d, dff, ne, k, seed=42, layer=0, down_type=14),
              synth.qwen_layer(d, dff, ne, k, seed=42, layer=1, down_type=12)]
    path = tmp_path / "q.gguf"
    W.moe_model(path, "qwen", layers, d, dff, ne, k, 1e-6)
    with GgufFile(path) as g:
        _same_as_arrays(g, layers, True, synth.token(d, 42, 0))


def test_gguf_type_and_shape_checks(gpu, tmp_path):
    say("case gguf type / shape checks")
    d, dff, ne, k = 480, 480, 8, 4
    L0 = synth.gptoss_layer(d, dff, ne, k, seed=43)
    good = tmp_path / "ok.gguf"
    W.moe_model(good, "gptoss", [L0], d, dff, ne, k, 1e-5)
    with GgufFile(good) as g:
        cfg = g.moe_config()
    # router stored as BF16 instead of F32
    bad = tmp_path / "bf16.gguf"
    meta = [("general.architecture", W.T_STR, "gpt-oss")]
    t = [("blk.0.ffn_gate_exps.weight", 39, [d, dff, ne], L0["gate"].tobytes()),
         ("blk.0.ffn_up_exps.weight", 39, [d, dff, ne], L0["up"].tobytes()),
         ("blk.0.ffn_down_exps.weight", 39, [dff, d, ne], L0["down"].tobytes()),
         ("blk.0.ffn_gate_inp.weight", 30, [d, ne], bytes(2 * d * ne)),
         ("blk.0.ffn_gate_exps.bias", 0, [dff, ne], L0["gate_b"].tobytes()),
         ("blk.0.ffn_up_exps.bias", 0, [dff, ne], L0["up_b"].tobytes()),
         ("blk.0.ffn_down_exps.bias", 0, [d, ne], L0["down_b"].tobytes()),
         ("blk.0.ffn_gate_inp.bias", 0, [ne], L0["router_b"].tobytes())]
    W.write_gguf(bad, meta, t)
    with GgufFile(bad) as g, MoeBlock(cfg) as blk:
        with pytest.raises(L.CpbError, match="F32"):
            blk.load_gguf_layer(g, 0)
    # a norm weight that is present in a type the reader does not handle
    # (Q4_0), or present as F16: rejected, not read as "no norm weight"
    t_ok = list(t)
    t_ok[3] = ("blk.0.ffn_gate_inp.weight", 0, [d, ne], L0["router_w"].tobytes())
    for typ, raw in ((2, bytes(d // 32 * 18)), (1, bytes(2 * d))):
        W.write_gguf(bad, meta, t_ok + [("blk.0.ffn_norm.weight", typ, [d], raw)])
        with GgufFile(bad) as g, MoeBlock(cfg) as blk:
            with pytest.raises(L.CpbError, match="F32"):
                blk.load_gguf_layer(g, 0)
    # down declared with swapped dims
    t2 = list(t)
    t2[3] = ("blk.0.ffn_gate_inp.weight", 0, [d, ne], L0["router_w"].tobytes())
    t2[2] = ("blk.0.ffn_down_exps.weight", 39, [d, dff * 2, ne // 2], L0["down"].tobytes())
    W.write_gguf(bad, meta, t2)
    with GgufFile(bad) as g, MoeBlock(cfg) as blk:
        with pytest.raises(L.CpbError, match="dims"):
            blk.load_gguf_layer(g, 0)
    # a k-quant down in an MXFP4 model: rejected by the per-matrix type check
    d2 = 512
    L1 = synth.gptoss_layer(d2, d2, ne, k, seed=44)
    t3 = [("blk.0.ffn_gate_exps.weight", 39, [d2, d2, ne], L1["gate"].tobytes()),
          ("blk.0.ffn_up_exps.weight", 39, [d2, d2, ne], L1["up"].tobytes()),
          ("blk.0.ffn_down_exps.weight", 12, [d2, d2, ne], synth.q4k(ne * d2, d2, 44, 1).tobytes()),
          ("blk.0.ffn_gate_inp.weight", 0, [d2, ne], L1["router_w"].tobytes()),
          ("blk.0.ffn_gate_exps.bias", 0, [d2, ne], L1["gate_b"].tobytes()),
          ("blk.0.ffn_up_exps.bias", 0, [d2, ne], L1["up_b"].tobytes()),
          ("blk.0.ffn_down_exps.bias", 0, [d2, ne], L1["down_b"].tobytes()),
          ("blk.0.ffn_gate_inp.bias", 0, [ne], L1["router_b"].tobytes())]
    W.write_gguf(bad, meta, t3)
    from cpubrrr_amd import MoeConfig
    with GgufFile(bad) as g, MoeBlock(MoeConfig.gptoss(d=d2, n_expert=ne, top_k=k, d_ff=d2)) as blk:
        with pytest.raises(L.CpbError, match="type 39"):
            blk.load_gguf_layer(g, 0)
