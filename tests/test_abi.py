"""C ABI checks that need no GPU: the library loads, exports every symbol the
public headers declare, and rejects bad configurations with error codes
(the reference panics on the same conditions, engine_gpt2.rs:73-74, 603-615)."""
import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

from cpubrrr_amd import MoeConfig, _lib as L

ROOT = Path(__file__).resolve().parent.parent


def header_symbols():
    syms = set()
    for h in (ROOT / "include").glob("*.h"):
        for m in re.finditer(r"^\s*(?:[A-Za-z_][\w\s\*]*?)\b(cpb_\w+)\s*\(", h.read_text(), re.M):
            syms.add(m.group(1))
    return syms


def test_exports_every_declared_symbol():
    lib = L.lib()
    syms = header_symbols()
    assert "cpb_moe_forward" in syms and "cpb_synth_mxfp4" in syms
    for s in sorted(syms):
        assert hasattr(lib, s), s
    assert syms <= set(L.SIGNATURES), syms - set(L.SIGNATURES)


def _create(cfg):
    h = C.c_void_p()
    c = cfg.c()
    return L.lib().cpb_moe_create(C.byref(c), 0, C.byref(h))


@pytest.mark.parametrize("mut", [
    dict(top_k=0), dict(top_k=9), dict(top_k=3, n_expert=2), dict(d=2880 + 16), dict(n_expert=1000),
    dict(act=L.ACT_SILU), dict(wtype_down=L.GGUF_Q6_K), dict(max_tokens=0), dict(router=7),
])
def test_bad_configs_rejected(mut):
    cfg = MoeConfig.gptoss()
    for k, v in mut.items():
        setattr(cfg, k, v)
    rc = _create(cfg)
    assert rc == L.CPB_EINVAL, (mut, rc)
    assert L.lib().cpb_moe_last_error()


@pytest.mark.parametrize("mut", [dict(norm_nt=0), dict(norm_nt=65), dict(d=256, norm_nt=17)])
def test_bad_qwen_norm_slices_rejected(mut):
    # the Qwen sum of squares runs one lane per slice, each at least 16 long
    cfg = MoeConfig.qwen3(d=256, d_ff=256, n_expert=8, top_k=2)
    for k, v in mut.items():
        setattr(cfg, k, v)
    assert _create(cfg) == L.CPB_EINVAL, mut
    assert L.lib().cpb_moe_last_error()


def test_null_args():
    lib = L.lib()
    assert lib.cpb_moe_create(None, 0, None) == L.CPB_EINVAL
    assert lib.cpb_moe_forward(None, 0, None, 1, 0, None) == L.CPB_EINVAL
    assert lib.cpb_moe_load_layer(None, 0, None, None, None, None, None, None, None, None, None) == L.CPB_EINVAL
    lib.cpb_moe_destroy(None)


def test_layer_bytes_20b():
    n = L.lib()
    cfg = MoeConfig.gptoss()
    got = C.c_size_t()
    assert n.cpb_moe_layer_bytes(C.byref(cfg.c()), C.byref(got)) == 0
    raw = 32 * 3 * 2880 * 90 * 17
    # stream layout pads 90 blocks to 6 k-parts of 15 + one 16-byte e8m0 unit each: 96/90 * 16/17
    assert got.value == 32 * 3 * 2880 * 6 * 16 * 16
    assert got.value / raw < 1.005


def test_synth_deterministic():
    from cpubrrr_amd import synth
    a = synth.mxfp4(100, 90, 0, 3)
    b = synth.mxfp4(100, 90, 0, 3)
    assert np.array_equal(a, b)
    e = a.reshape(-1, 17)[:, 0]
    assert e.min() == 121 and e.max() == 124
    codes = np.concatenate([a.reshape(-1, 17)[:, 1:] & 15, a.reshape(-1, 17)[:, 1:] >> 4]).ravel()
    assert np.bincount(codes, minlength=16).min() > 0.9 * codes.size / 16
    x = synth.normal(100000, 1.0, 0, 5)
    assert abs(x.mean()) < 0.02 and abs(x.std() - 1) < 0.02
    z = synth.zipf_bias(32, 1.1, 0, 1)
    p = np.exp(z)
    assert abs(p.sum() - 1) < 1e-5 and np.allclose(np.sort(p)[::-1], (np.arange(1, 33) ** -1.1) / (np.arange(1, 33) ** -1.1).sum(), rtol=1e-5)
    for v in (0.0, 1.0, -2.5, 65504.0, 1e-5, 3e-8, 0.1, 7e4):
        assert L.lib().cpb_f32_to_half(v) == np.float16(v).view(np.uint16)


@pytest.mark.parametrize("mut", [
    dict(head_dim=128), dict(d=2880 + 16), dict(d=8192), dict(n_head_kv=3), dict(n_head=0),
    dict(n_head=64, n_head_kv=4), dict(n_layer=0), dict(max_seq=0), dict(max_seq=1 << 14), dict(sliding_window=0),
])
def test_attention_bad_configs_rejected(mut):
    # checked before any device is touched (GPU or not)
    base = dict(d=2880, n_head=64, n_head_kv=8, head_dim=64, n_layer=2, max_seq=64, sliding_window=128,
                rope_base=150000.0, rms_eps=1e-5)
    base.update(mut)
    c = L.AttnCfg(**base)
    h = C.c_void_p()
    assert L.lib().cpb_attn_create(C.byref(c), 0, C.byref(h)) == L.CPB_EINVAL, mut
    assert not h.value


@pytest.mark.parametrize("mut", [
    dict(d=100), dict(d=8192), dict(n_vocab=1001), dict(n_vocab=0), dict(n_slices=0), dict(n_slices=33),
    dict(n_cand=0), dict(n_cand=17), dict(n_slices=32, n_cand=8),
])
def test_head_bad_configs_rejected(mut):
    base = dict(d=2880, n_vocab=4096, n_slices=12, n_cand=8, rms_eps=1e-5)
    base.update(mut)
    c = L.HeadCfg(**base)
    h = C.c_void_p()
    assert L.lib().cpb_head_create(C.byref(c), 0, C.byref(h)) == L.CPB_EINVAL, mut
    assert not h.value
    n = C.c_size_t()
    assert L.lib().cpb_head_bytes(C.byref(c), C.byref(n)) == L.CPB_EINVAL


def test_attention_and_head_null_args():
    lib = L.lib()
    assert lib.cpb_attn_create(None, 0, None) == L.CPB_EINVAL
    assert lib.cpb_attn_forward(None, 0, 0, None, None) == L.CPB_EINVAL
    assert lib.cpb_attn_forward_device(None, 0, 0, None) == L.CPB_EINVAL
    assert lib.cpb_attn_reset(None) == L.CPB_EINVAL
    assert lib.cpb_attn_sync(None) == L.CPB_EINVAL
    lib.cpb_attn_destroy(None)
    assert lib.cpb_head_create(None, 0, None) == L.CPB_EINVAL
    assert lib.cpb_head_forward(None, None, None, None) == L.CPB_EINVAL
    assert lib.cpb_head_forward_device(None, None, None) == L.CPB_EINVAL
    assert lib.cpb_head_sync(None) == L.CPB_EINVAL
    lib.cpb_head_destroy(None)
