"""GGUF v3 model files for the MoE path (ctypes front end of include/cpb_gguf.h).

The reference indexes a GGUF blob with scripts/gguf_index.py (header,
metadata, tensor infos, aligned data start), writes manifest.txt and an
arch-prefix-free config.txt with scripts/setup_model.sh, mmaps the blob and
fetches tensors by name with typed accessors that assert the GGUF type
(engine_gpt2.rs:600-617, 1276-1285).  `GgufFile` does the same through the C
library (the file is mmapped there), `MoeConfig` can be filled from its
hparams, and `MoeBlock.load_gguf_layer` feeds a layer straight from the map.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib as L
from .moe import MoeConfig

F32, F16, Q8_0, Q4_K, Q6_K, BF16, MXFP4 = 0, 1, 8, 12, 14, 30, 39


class GgufFile:
    def __init__(self, path: str):
        self._lib = L.lib()
        h = C.c_void_p()
        L.check(self._lib.cpb_gguf_open(str(path).encode(), C.byref(h)), "cpb_gguf_open")
        self._h = h

    @property
    def handle(self):
        return self._h

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.cpb_gguf_close(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def version(self) -> tuple[int, int, int]:
        v, ds, al = C.c_uint32(), C.c_uint64(), C.c_uint64()
        L.check(self._lib.cpb_gguf_version(self._h, C.byref(v), C.byref(ds), C.byref(al)), "cpb_gguf_version")
        return v.value, ds.value, al.value

    @staticmethod
    def _info(t: L.GgufTensor) -> dict:
        return {"name": t.name.decode(), "type": t.type, "dims": [int(t.dims[k]) for k in range(t.n_dims)],
                "n_elements": int(t.n_elements), "offset": int(t.offset), "n_bytes": int(t.n_bytes),
                "data": t.data}

    def tensors(self) -> list[dict]:
        n = C.c_int64()
        L.check(self._lib.cpb_gguf_n_tensors(self._h, C.byref(n)), "cpb_gguf_n_tensors")
        out = []
        for i in range(n.value):
            t = L.GgufTensor()
            L.check(self._lib.cpb_gguf_tensor_at(self._h, i, C.byref(t)), "cpb_gguf_tensor_at")
            out.append(self._info(t))
        return out

    def tensor(self, name: str) -> dict:
        t = L.GgufTensor()
        L.check(self._lib.cpb_gguf_find(self._h, name.encode(), C.byref(t)), "cpb_gguf_find")
        return self._info(t)

    def data(self, name: str) -> np.ndarray:
        """The tensor's bytes (a copy out of the map), uint8."""
        t = self.tensor(name)
        if not t["data"]:
            raise ValueError(f"{name}: type {t['type']} has no data view")
        return np.ctypeslib.as_array((C.c_uint8 * t["n_bytes"]).from_address(t["data"])).copy()

    def f32v(self, name: str) -> np.ndarray:
        """engine_gpt2.rs:601-605: an F32 tensor (asserts type 0)."""
        t = self.tensor(name)
        if t["type"] != F32:
            raise ValueError(f"{name}: type {t['type']}, expected F32 (0)")
        return self.data(name).view(np.float32)

    def meta_int(self, key: str) -> int:
        v = C.c_int64()
        L.check(self._lib.cpb_gguf_meta_i64(self._h, key.encode(), C.byref(v)), "cpb_gguf_meta_i64")
        return v.value

    def meta_float(self, key: str) -> float:
        v = C.c_double()
        L.check(self._lib.cpb_gguf_meta_f64(self._h, key.encode(), C.byref(v)), "cpb_gguf_meta_f64")
        return v.value

    def meta_str(self, key: str) -> str:
        v = C.c_char_p()
        L.check(self._lib.cpb_gguf_meta_str(self._h, key.encode(), C.byref(v)), "cpb_gguf_meta_str")
        return v.value.decode()

    def hparams(self) -> dict:
        h = L.GgufHparams()
        L.check(self._lib.cpb_gguf_hparams_get(self._h, C.byref(h)), "cpb_gguf_hparams_get")
        out = {k: getattr(h, k) for k, _ in L.GgufHparams._fields_}
        out["arch"] = h.arch.decode()
        return out

    def write_manifest(self, path: str) -> None:
        L.check(self._lib.cpb_gguf_write_manifest(self._h, str(path).encode()), "cpb_gguf_write_manifest")

    def moe_config(self, max_tokens: int = 1) -> MoeConfig:
        """Handle configuration from the file's hparams and tensor types
        (gpt-oss: MXFP4 experts with biases; qwen3moe: Q4_K gate/up)."""
        hp = self.hparams()
        gate = self.tensor("blk.0.ffn_gate_exps.weight")
        down = self.tensor("blk.0.ffn_down_exps.weight")
        d, ne, k, ff, nl = hp["n_embd"], hp["n_expert"], hp["n_expert_used"], hp["n_ff_exp"], hp["n_layer"]
        eps = hp["rms_eps"]
        if gate["type"] == MXFP4:
            return MoeConfig.gptoss(d=d, n_expert=ne, top_k=k, d_ff=ff, n_layer=nl, max_tokens=max_tokens,
                                    rms_eps=eps)
        return MoeConfig.qwen3(d=d, n_expert=ne, top_k=k, d_ff=ff, n_layer=nl, max_tokens=max_tokens,
                               rms_eps=eps, down_type=down["type"])
