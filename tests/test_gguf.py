"""GGUF v3 reader (include/cpb_gguf.h) against files written from the format
spec by tests/gguf_writer.py: tensor index, offsets, aligned data start,
metadata, the manifest of scripts/setup_model.sh, derived hparams, and clean
errors on corrupt or truncated files.  CPU only (parsing needs no GPU)."""
import numpy as np
import pytest

from cpubrrr_amd import GgufFile, synth
from cpubrrr_amd import _lib as L
from tests import gguf_writer as W


def _gptoss(tmp_path, alignment=None, name="m.gguf"):
    d, dff, ne, k = 64, 96, 4, 2
    layers = [synth.gptoss_layer(d, dff, ne, k, seed=3, layer=l, zipf=1.1) for l in range(2)]
    path = tmp_path / name
    rec, data_start = W.moe_model(path, "gptoss", layers, d, dff, ne, k, 1e-5, alignment)
    return path, rec, data_start, layers


@pytest.mark.parametrize("alignment", [None, 64, 256])
def test_index_matches_writer(tmp_path, alignment):
    path, rec, data_start, layers = _gptoss(tmp_path, alignment)
    raw = path.read_bytes()
    with GgufFile(path) as g:
        ver, ds, al = g.version()
        assert ver == 3 and ds == data_start and al == (alignment or 32)
        ts = g.tensors()
        assert [t["name"] for t in ts] == [r[0] for r in rec]
        for t, (name, typ, off, n, nbytes) in zip(ts, rec):
            assert (t["type"], t["offset"], t["n_elements"]) == (typ, off, n), name
            assert t["n_bytes"] == nbytes
            assert g.data(name).tobytes() == raw[ds + off: ds + off + nbytes], name
        assert g.tensor("blk.1.ffn_down_exps.weight")["dims"] == [96, 64, 4]
        assert np.array_equal(g.f32v("blk.1.ffn_gate_inp.bias"), layers[1]["router_b"])
        assert np.array_equal(g.data("blk.0.ffn_gate_exps.weight"), layers[0]["gate"].reshape(-1))
        with pytest.raises(ValueError):
            g.f32v("blk.0.ffn_gate_exps.weight")          # MXFP4, not F32 (engine_gpt2.rs:603)


def test_metadata_and_hparams(tmp_path):
    path, _, _, _ = _gptoss(tmp_path)
    with GgufFile(path) as g:
        assert g.meta_str("general.architecture") == "gpt-oss"
        assert g.meta_int("gpt-oss.block_count") == 2
        assert g.meta_int("general.flag") == 1 and g.meta_int("general.i8") == -5
        assert g.meta_float("general.f64") == 2.5
        assert g.meta_float("gpt-oss.attention.layer_norm_rms_epsilon") == np.float32(1e-5)
        with pytest.raises(L.CpbError):
            g.meta_int("tokenizer.ggml.tokens")                 # an array: skipped, not a scalar
        with pytest.raises(L.CpbError):
            g.meta_str("nope")
        hp = g.hparams()
        assert hp["arch"] == "gpt-oss"
        assert (hp["n_embd"], hp["n_layer"], hp["n_expert"], hp["n_expert_used"]) == (64, 2, 4, 2)
        assert hp["n_ff_exp"] == 96                              # derived from ffn_gate_exps dims[1]
        assert hp["context_length"] == 131072 and hp["rope_freq_base"] == 150000.0
        assert hp["n_head"] == -1 and hp["n_vocab"] == -1       # absent keys / tensors
        cfg = g.moe_config()
        assert (cfg.d, cfg.d_ff, cfg.n_expert, cfg.top_k, cfg.n_layer, cfg.has_bias) == (64, 96, 4, 2, 2, True)


def test_hparam_suffix_match_in_file_order(tmp_path):
    # setup_model.sh:54-58 g(): the first key in file order that equals
    # "<arch>.<suffix>" or ends in ".<suffix>" -- an earlier key of another
    # prefix wins over the exact key written after it
    meta = [("general.architecture", W.T_STR, "gpt-oss"),
            ("foo.block_count", W.T_U32, 7),
            ("gpt-oss.block_count", W.T_U32, 2),
            ("gpt-oss.expert_count", W.T_U32, 4),
            ("bar.expert_count", W.T_U32, 9)]
    p = tmp_path / "order.gguf"
    W.write_gguf(p, meta, [("a", 0, [4], bytes(16))])
    with GgufFile(p) as g:
        hp = g.hparams()
        assert hp["n_layer"] == 7 and hp["n_expert"] == 4


def test_qwen_hparams_and_types(tmp_path):
    d, dff, ne, k = 512, 256, 8, 2
    layers = [synth.qwen_layer(d, dff, ne, k, seed=4, layer=0, down_type=14),
              synth.qwen_layer(d, dff, ne, k, seed=4, layer=1, down_type=12)]
    path = tmp_path / "q.gguf"
    W.moe_model(path, "qwen", layers, d, dff, ne, k, 1e-6)
    with GgufFile(path) as g:
        hp = g.hparams()
        assert hp["arch"] == "qwen3moe" and hp["n_ff_exp"] == 256
        assert g.tensor("blk.0.ffn_down_exps.weight")["type"] == 14
        assert g.tensor("blk.1.ffn_down_exps.weight")["type"] == 12
        assert g.tensor("blk.0.ffn_gate_exps.weight")["n_bytes"] == ne * dff * (d // 256) * 144
        cfg = g.moe_config()
        assert cfg.wtype_gate_up == 12 and cfg.wtype_down == 14 and not cfg.has_bias


def test_manifest_matches_setup_model(tmp_path):
    path, rec, data_start, _ = _gptoss(tmp_path, 64)
    man = tmp_path / "manifest.txt"
    with GgufFile(path) as g:
        g.write_manifest(man)
    # setup_model.sh:45-51: "data_start N", then "name type offset n_elements"
    want = [f"data_start {data_start}"] + [f"{n} {t} {o} {e}" for n, t, o, e, _ in rec]
    assert man.read_text().splitlines() == want


def test_corrupt_files_fail_cleanly(tmp_path):
    path, rec, data_start, _ = _gptoss(tmp_path)
    raw = path.read_bytes()
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGUX" + raw[4:])
    with pytest.raises(L.CpbError, match="magic"):
        GgufFile(bad)
    bad.write_bytes(raw[:4] + (7).to_bytes(4, "little") + raw[8:])
    with pytest.raises(L.CpbError, match="version"):
        GgufFile(bad)
    # every truncation inside the header and index fails with an error, as
    # does a cut inside the tensor data
    for cut in list(range(0, data_start, max(1, data_start // 97))) + [data_start + 100, len(raw) - 1]:
        bad.write_bytes(raw[:cut])
        with pytest.raises(L.CpbError):
            GgufFile(bad)
    # an absurd tensor count
    bad.write_bytes(raw[:8] + (1 << 60).to_bytes(8, "little") + raw[16:])
    with pytest.raises(L.CpbError):
        GgufFile(bad)


def test_duplicate_tensor_rejected(tmp_path):
    t = [("a", 0, [4], bytes(16)), ("a", 0, [4], bytes(16))]
    p = tmp_path / "dup.gguf"
    W.write_gguf(p, [], t)
    with pytest.raises(L.CpbError, match="duplicate"):
        GgufFile(p)
