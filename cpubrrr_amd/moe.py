"""Host-side mirror of the reference's MoE block, driving the HIP path.

The reference has no operator API for this path: the MoE stage is inline
code in each engine's forward_worker (engine_gpt2.rs:845-923 for gpt-oss,
engine_qwen2.rs:395-433 for Qwen3), configured from config.txt keys
(n_embd, n_expert, n_expert_used, n_ff_exp, n_layer, rms_eps) and fed
tensors by name (blk.{i}.ffn_{gate,up,down}_exps.weight, ..._exps.bias,
ffn_gate_inp.weight/bias, ffn_norm.weight).  `MoeBlock` keeps those names
and that order: construct from the config, load each layer's tensors, then
call `forward(layer, x)`, which updates the residual x in place exactly as
the reference's stage does (x += sum_e w_e * (down_e(act(gate_e, up_e)) + b)).

Every call goes through the C ABI (libcpb_moe.so, include/cpb_moe.h); there
is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _lib as L


@dataclass
class MoeConfig:
    d: int
    n_expert: int
    top_k: int
    d_ff: int
    n_layer: int = 1
    router: int = L.ROUTER_TOPK_SOFTMAX
    act: int = L.ACT_SWIGLU_OAI
    norm: int = L.NORM_GPTOSS
    norm_nt: int = 12
    alpha: float = 1.702
    limit: float = 7.0
    rms_eps: float = 1e-5
    wtype_gate_up: int = L.GGUF_MXFP4
    wtype_down: int = L.GGUF_MXFP4
    has_bias: bool = True
    max_tokens: int = 1

    @staticmethod
    def gptoss(d=2880, n_expert=32, top_k=4, d_ff=2880, n_layer=1, max_tokens=1, rms_eps=1e-5):
        """gpt-oss-20b/120b MoE semantics (engine_gpt2.rs)."""
        return MoeConfig(d, n_expert, top_k, d_ff, n_layer, max_tokens=max_tokens, rms_eps=rms_eps)

    @staticmethod
    def qwen3(d=2048, n_expert=128, top_k=8, d_ff=768, n_layer=1, max_tokens=1, rms_eps=1e-6,
              down_type=L.GGUF_Q6_K):
        """Qwen3-30B-A3B MoE semantics (engine_qwen2.rs)."""
        return MoeConfig(d, n_expert, top_k, d_ff, n_layer, router=L.ROUTER_SOFTMAX_TOPK, act=L.ACT_SILU,
                         norm=L.NORM_QWEN, norm_nt=12, rms_eps=rms_eps, wtype_gate_up=L.GGUF_Q4_K,
                         wtype_down=down_type, has_bias=False, max_tokens=max_tokens)

    def c(self) -> L.MoeCfg:
        return L.MoeCfg(self.d, self.n_expert, self.top_k, self.d_ff, self.n_layer, self.router, self.act,
                        self.norm, self.norm_nt, self.alpha, self.limit, self.rms_eps, self.wtype_gate_up,
                        self.wtype_down, int(self.has_bias), self.max_tokens)

    @property
    def mx(self) -> bool:
        return self.wtype_gate_up == L.GGUF_MXFP4


def _fp(a, t=L.f32p):
    return C.cast(None, t) if a is None else a.ctypes.data_as(t)


class MoeBlock:
    """One handle = one device + one stream + n_layer MoE layers."""

    def __init__(self, cfg: MoeConfig, device: int = 0):
        self.cfg = cfg
        self._lib = L.lib()
        h = C.c_void_p()
        ccfg = cfg.c()
        L.check(self._lib.cpb_moe_create(C.byref(ccfg), device, C.byref(h)), "cpb_moe_create")
        self._h = h
        self._down_type = {}

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.cpb_moe_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @staticmethod
    def layer_bytes(cfg: MoeConfig) -> int:
        n = C.c_size_t()
        ccfg = cfg.c()
        L.check(L.lib().cpb_moe_layer_bytes(C.byref(ccfg), C.byref(n)), "cpb_moe_layer_bytes")
        return n.value

    def load_layer(self, layer: int, t: dict) -> None:
        """t: gate/up/down (native GGUF bytes), gate_b/up_b/down_b, router_w/router_b, norm_w;
        optional gate_type/up_type/down_type (GGUF type ids, default: the config's)."""
        keep = {k: (np.ascontiguousarray(t[k]) if t.get(k) is not None else None)
                for k in ("gate", "up", "down", "gate_b", "up_b", "down_b", "router_w", "router_b", "norm_w")}
        for k in ("gate_b", "up_b", "down_b", "router_w", "router_b", "norm_w"):
            if keep[k] is not None:
                keep[k] = np.ascontiguousarray(keep[k], np.float32)
        if not self.cfg.has_bias:
            for k in ("gate_b", "up_b", "down_b", "router_b"):
                keep[k] = None
        c = self.cfg
        gt = int(t.get("gate_type", c.wtype_gate_up))
        ut = int(t.get("up_type", c.wtype_gate_up))
        dt = int(t.get("down_type", c.wtype_down))
        rc = self._lib.cpb_moe_load_layer_typed(
            self._h, layer, gt, ut, dt, keep["gate"].ctypes.data, keep["up"].ctypes.data, keep["down"].ctypes.data,
            _fp(keep["gate_b"]), _fp(keep["up_b"]), _fp(keep["down_b"]), _fp(keep["router_w"]),
            _fp(keep["router_b"]), _fp(keep["norm_w"]))
        L.check(rc, "cpb_moe_load_layer_typed")
        self._down_type[layer] = dt

    def load_gguf_layer(self, gguf, layer: int) -> None:
        """Layer `layer` straight from a mapped GGUF file (cpubrrr_amd.gguf.GgufFile):
        tensors by the reference's names, types and shapes checked."""
        L.check(self._lib.cpb_moe_load_gguf_layer(self._h, gguf.handle, layer), "cpb_moe_load_gguf_layer")
        self._down_type[layer] = gguf.tensor(f"blk.{layer}.ffn_down_exps.weight")["type"]

    def forward(self, layer: int, x: np.ndarray, apply_norm: bool = True, trace: bool = False):
        """x: [d] or [n_tok, d] fp32, updated like the reference's residual.
        Returns (x_out, trace_dict or None)."""
        c = self.cfg
        xo = np.array(x, np.float32, copy=True, order="C")
        n_tok = 1 if xo.ndim == 1 else xo.shape[0]
        t = None
        tr_p = C.cast(None, C.POINTER(L.MoeTrace))
        if trace:
            d, ff, k, ne = c.d, c.d_ff, c.top_k, c.n_expert
            mx = c.mx
            t = {
                "xn": np.zeros(d, np.float32), "xq": np.zeros(d, np.int8),
                "xsb": np.zeros(d // 32 if mx else d // 256, np.float32),
                "xsum": np.zeros(d // 32, np.int32), "logits": np.zeros(ne, np.float32),
                "ids": np.zeros(k, np.int32), "wts": np.zeros(k, np.float32),
                "gu": np.zeros((k, 2, ff), np.float32),
                "gu_sums": np.zeros((k, 2, ff, d // 32) if mx else (k, 2, ff, d // 256, 2), np.int32),
                "hq": np.zeros((k, ff), np.int8),
                "hsb": np.zeros((k, ff // 32) if mx else (k, ff // 256), np.float32),
                "hsum": np.zeros((k, ff // 32), np.int32), "dn": np.zeros((k, d), np.float32),
                "dn_sums": np.zeros((k, d, ff // 32) if mx else
                                    ((k, d, ff // 256, 2) if self._down_type.get(layer, c.wtype_down) == L.GGUF_Q4_K
                                     else (k, d, ff // 256)),
                                    np.int32),
                "h": np.zeros((k, ff), np.float32),
            }
            tr = L.MoeTrace()
            types = dict(L.MoeTrace._fields_)
            for name, arr in t.items():
                setattr(tr, name, arr.ctypes.data_as(types[name]))
            tr_p = C.pointer(tr)
        rc = self._lib.cpb_moe_forward(self._h, layer, xo.ctypes.data_as(L.f32p), n_tok, int(bool(apply_norm)), tr_p)
        L.check(rc, "cpb_moe_forward")
        if trace:
            t["exact_router_fallbacks"] = int(tr_p.contents.exact_router_fallbacks)
        return xo, t

    def grouped_sums(self, layer: int, x: np.ndarray, apply_norm: bool = True):
        """Test hook of the grouped (n_tok > 1) path: returns (x_out, gu_sums,
        dn_sums), pair-major; MXFP4: [n_tok*k][2][d_ff][d/32] and
        [n_tok*k][d][d_ff/32]; k-quants: the decode trace's superblock sums."""
        c = self.cfg
        xo = np.array(x, np.float32, copy=True, order="C")
        n_tok = xo.shape[0]
        np_ = n_tok * c.top_k
        if c.mx:
            gs = np.zeros((np_, 2, c.d_ff, c.d // 32), np.int32)
            ds = np.zeros((np_, c.d, c.d_ff // 32), np.int32)
        else:
            gs = np.zeros((np_, 2, c.d_ff, c.d // 256, 2), np.int32)
            q4 = self._down_type.get(layer, c.wtype_down) == L.GGUF_Q4_K
            ds = np.zeros((np_, c.d, c.d_ff // 256, 2) if q4 else (np_, c.d, c.d_ff // 256), np.int32)
        L.check(self._lib.cpb_moe_grouped_sums(self._h, layer, xo.ctypes.data_as(L.f32p), n_tok, int(bool(apply_norm)),
                                               gs.ctypes.data_as(L.i32p), ds.ctypes.data_as(L.i32p)),
                "cpb_moe_grouped_sums")
        return xo, gs, ds

    def forward_device(self, layer0: int, n_layers: int, x_ptr: int, n_tok: int = 1, apply_norm: bool = True):
        """Asynchronous forward over layers on device memory (x_ptr: device address)."""
        L.check(self._lib.cpb_moe_forward_device(self._h, layer0, n_layers, C.c_void_p(x_ptr), n_tok,
                                                 int(bool(apply_norm))), "cpb_moe_forward_device")

    def forward_device_noalloc(self, layer0: int, n_layers: int, x_ptr: int, n_tok: int = 1, apply_norm: bool = True):
        """forward_device without any allocation: per-call scratch in the library's
        static per-GPU array (calls overlapping on one GPU race)."""
        L.check(self._lib.cpb_moe_forward_device_noalloc(self._h, layer0, n_layers, C.c_void_p(x_ptr), n_tok,
                                                         int(bool(apply_norm))), "cpb_moe_forward_device_noalloc")

    def set_stream(self, stream_ptr: int | None) -> None:
        L.check(self._lib.cpb_moe_set_stream(self._h, C.c_void_p(stream_ptr or 0)), "cpb_moe_set_stream")

    def sync(self) -> None:
        L.check(self._lib.cpb_moe_sync(self._h), "cpb_moe_sync")

    def timing(self, enable: bool) -> None:
        L.check(self._lib.cpb_moe_timing(self._h, int(enable)), "cpb_moe_timing")

    def kernel_times(self):
        ms = (C.c_double * 3)()
        n = (C.c_long * 3)()
        L.check(self._lib.cpb_moe_kernel_times(self._h, ms, n), "cpb_moe_kernel_times")
        return {name: (ms[i], n[i]) for i, name in enumerate(("route", "gate_up", "down"))}
