"""Minimal GGUF v3 writer for tests, written from the published format
(ggml's docs/gguf.md): little endian; "GGUF", u32 version, u64 tensor
count, u64 metadata count; metadata = string key, u32 value type, value;
tensor infos = string name, u32 n_dims, u64 dims (fastest first), u32 type,
u64 offset from the data start; data start and every tensor's data aligned
to general.alignment (default 32).  string = u64 length + UTF-8 bytes.
Independent of the library's reader (cpubrrr_amd/csrc/gguf.cpp), which the
tests check against it.
"""
from __future__ import annotations

import struct

import numpy as np

T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64 = range(13)
_FMT = {T_U8: "<B", T_I8: "<b", T_U16: "<H", T_I16: "<h", T_U32: "<I", T_I32: "<i", T_F32: "<f", T_BOOL: "<?",
        T_U64: "<Q", T_I64: "<q", T_F64: "<d"}
# bytes per block, elements per block
BLOCK = {0: (4, 1), 1: (2, 1), 2: (18, 32), 8: (34, 32), 12: (144, 256), 14: (210, 256), 30: (2, 1), 39: (17, 32)}


def _s(b: bytearray, text: str) -> None:
    raw = text.encode()
    b += struct.pack("<Q", len(raw)) + raw


def _val(b: bytearray, t: int, v) -> None:
    if t == T_STR:
        _s(b, v)
    elif t == T_ARR:
        et, items = v
        b += struct.pack("<IQ", et, len(items))
        for it in items:
            _val(b, et, it)
    else:
        b += struct.pack(_FMT[t], v)


def write_gguf(path, meta: list, tensors: list, alignment: int | None = None, version: int = 3) -> list:
    """meta: [(key, type, value)]; tensors: [(name, ggml_type, dims, raw bytes)].
    Returns [(name, type, offset, n_elements, n_bytes)] as written."""
    b = bytearray(b"GGUF")
    b += struct.pack("<IQQ", version, len(tensors), len(meta) + (alignment is not None))
    for k, t, v in meta:
        _s(b, k)
        b += struct.pack("<I", t)
        _val(b, t, v)
    al = 32
    if alignment is not None:
        _s(b, "general.alignment")
        b += struct.pack("<I", T_U32)
        b += struct.pack("<I", alignment)
        al = alignment
    rec, off = [], 0
    for name, t, dims, raw in tensors:
        n = int(np.prod(dims))
        bs, be = BLOCK[t]
        assert dims[0] % be == 0 and len(raw) == n // be * bs, (name, len(raw))
        _s(b, name)
        b += struct.pack("<I", len(dims))
        b += struct.pack(f"<{len(dims)}Q", *dims)
        b += struct.pack("<IQ", t, off)
        rec.append((name, t, off, n, len(raw)))
        off += (len(raw) + al - 1) // al * al
    data_start = (len(b) + al - 1) // al * al
    b += bytes(data_start - len(b))
    for (name, t, dims, raw), (_, _, o, _, _) in zip(tensors, rec):
        assert len(b) == data_start + o
        b += raw
        b += bytes((len(raw) + al - 1) // al * al - len(raw))
    with open(path, "wb") as f:
        f.write(b)
    return rec, data_start


def moe_model(path, family: str, layers: list, d: int, dff: int, ne: int, k: int, eps: float,
              alignment: int | None = None):
    """A GGUF holding the MoE tensors of `layers` (synth.gptoss_layer /
    qwen_layer dicts) under the reference's names, with gpt-oss / qwen3moe
    hparams and a tokenizer-like string array (skipped by the reader)."""
    arch = "gpt-oss" if family == "gptoss" else "qwen3moe"
    meta = [("general.architecture", T_STR, arch), ("general.name", T_STR, "synthetic"),
            (f"{arch}.block_count", T_U32, len(layers)), (f"{arch}.embedding_length", T_U32, d),
            (f"{arch}.expert_count", T_U32, ne), (f"{arch}.expert_used_count", T_U32, k),
            (f"{arch}.attention.layer_norm_rms_epsilon", T_F32, eps),
            (f"{arch}.rope.freq_base", T_F32, 150000.0), (f"{arch}.context_length", T_U64, 131072),
            ("tokenizer.ggml.tokens", T_ARR, (T_STR, ["<s>", "a", "bc", "é"])),
            ("tokenizer.ggml.scores", T_ARR, (T_F32, [0.0, -1.0, -2.0, -3.0])),
            ("general.flag", T_BOOL, True), ("general.i8", T_I8, -5), ("general.f64", T_F64, 2.5)]
    if family == "qwen":
        meta.append((f"{arch}.expert_feed_forward_length", T_U32, dff))   # gpt-oss: derived from the tensor
    tensors = []
    for i, L in enumerate(layers):
        gt = L.get("gate_type", 39)
        dt = L.get("down_type", 39)
        tensors += [(f"blk.{i}.ffn_gate_exps.weight", gt, [d, dff, ne], L["gate"].tobytes()),
                    (f"blk.{i}.ffn_up_exps.weight", gt, [d, dff, ne], L["up"].tobytes()),
                    (f"blk.{i}.ffn_down_exps.weight", dt, [dff, d, ne], L["down"].tobytes()),
                    (f"blk.{i}.ffn_gate_inp.weight", 0, [d, ne], L["router_w"].astype(np.float32).tobytes()),
                    (f"blk.{i}.ffn_norm.weight", 0, [d], L["norm_w"].astype(np.float32).tobytes())]
        if family == "gptoss":
            tensors += [(f"blk.{i}.ffn_gate_exps.bias", 0, [dff, ne], L["gate_b"].tobytes()),
                        (f"blk.{i}.ffn_up_exps.bias", 0, [dff, ne], L["up_b"].tobytes()),
                        (f"blk.{i}.ffn_down_exps.bias", 0, [d, ne], L["down_b"].tobytes()),
                        (f"blk.{i}.ffn_gate_inp.bias", 0, [ne], L["router_b"].tobytes())]
    # a tensor of a type the MoE path never reads (attention weights are BF16)
    tensors.append(("blk.0.attn_q.weight", 30, [d, 64], bytes(2 * d * 64)))
    return write_gguf(path, meta, tensors, alignment)
