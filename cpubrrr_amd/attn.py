"""The gpt-oss engine's attention block on the GPU, decode (ctypes front end
of include/cpb_attn.h).

Per token and layer the reference (engine_gpt2.rs:772-843) normalises x with
attn_norm and quantises it to Q8, projects q / k / v through Q8 copies of the
bf16 weights plus biases, applies YaRN RoPE from a table built once
(:535-590), appends k / v to the layer's cache, runs each q-head's softmax
over the cached positions (a sliding window on layers 0, 2, ...) with the
head's sink in the denominator, quantises the heads' outputs to Q8 and adds
wo . ao + bo to x.  `Attention` holds the quantised weights and the KV cache
of every layer in HBM and runs that step.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib as L

_U16P = C.POINTER(C.c_uint16)


class Attention:
    def __init__(self, d: int, n_head: int, n_head_kv: int, n_layer: int, max_seq: int = 4096,
                 sliding_window: int = 128, rope_base: float = 150000.0, rms_eps: float = 1e-5,
                 head_dim: int = 64, device: int = 0):
        self._lib = L.lib()
        self.cfg = L.AttnCfg(d, n_head, n_head_kv, head_dim, n_layer, max_seq, sliding_window, rope_base, rms_eps)
        h = C.c_void_p()
        L.check(self._lib.cpb_attn_create(C.byref(self.cfg), device, C.byref(h)), "cpb_attn_create")
        self._h = h

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.cpb_attn_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def load_layer(self, layer: int, t: dict) -> None:
        """t: attn_norm, bq, bk, bv, bo, sinks (float32) and wq, wk, wv, wo
        (bf16 bits as uint16), the shapes of include/cpb_attn.h."""
        c = self.cfg
        nq, nkv = c.n_head * c.head_dim, c.n_head_kv * c.head_dim
        shapes = {"attn_norm": (c.d,), "bq": (nq,), "bk": (nkv,), "bv": (nkv,), "bo": (c.d,), "sinks": (c.n_head,),
                  "wq": (nq, c.d), "wk": (nkv, c.d), "wv": (nkv, c.d), "wo": (c.d, nq)}
        a = {}
        for k, shp in shapes.items():
            a[k] = np.ascontiguousarray(t[k], np.uint16 if k.startswith("w") else np.float32)
            assert a[k].shape == shp, (k, a[k].shape, shp)
        f = lambda k: a[k].ctypes.data_as(L.f32p)  # noqa: E731
        w = lambda k: a[k].ctypes.data_as(_U16P)  # noqa: E731
        L.check(self._lib.cpb_attn_load_layer(self._h, layer, f("attn_norm"), w("wq"), w("wk"), w("wv"), w("wo"),
                                              f("bq"), f("bk"), f("bv"), f("bo"), f("sinks")),
                "cpb_attn_load_layer")

    def forward(self, layer: int, pos: int, x: np.ndarray, trace: bool = False):
        """x + attention(x) for the token at pos; with trace, also a dict of
        xq, xsb, q, k, v, ao, aq, asb."""
        c = self.cfg
        xo = np.array(x, np.float32, copy=True)
        assert xo.shape == (c.d,)
        t = None
        tp = C.cast(None, C.POINTER(L.AttnTrace))
        if trace:
            nq, nkv = c.n_head * c.head_dim, c.n_head_kv * c.head_dim
            t = {"xq": np.zeros(c.d, np.int8), "xsb": np.zeros(c.d // 32, np.float32), "q": np.zeros(nq, np.float32),
                 "k": np.zeros(nkv, np.float32), "v": np.zeros(nkv, np.float32), "ao": np.zeros(nq, np.float32),
                 "aq": np.zeros(nq, np.int8), "asb": np.zeros(nq // 32, np.float32)}
            tr = L.AttnTrace()
            types = dict(L.AttnTrace._fields_)
            for k, v in t.items():
                setattr(tr, k, v.ctypes.data_as(types[k]))
            tp = C.pointer(tr)
        L.check(self._lib.cpb_attn_forward(self._h, layer, pos, xo.ctypes.data_as(L.f32p), tp), "cpb_attn_forward")
        return xo, t

    def forward_device(self, layer: int, pos: int, x_ptr: int) -> None:
        L.check(self._lib.cpb_attn_forward_device(self._h, layer, pos, C.c_void_p(x_ptr)), "cpb_attn_forward_device")

    def reset(self) -> None:
        L.check(self._lib.cpb_attn_reset(self._h), "cpb_attn_reset")

    def set_stream(self, stream_ptr: int | None) -> None:
        L.check(self._lib.cpb_attn_set_stream(self._h, C.c_void_p(stream_ptr or 0)), "cpb_attn_set_stream")

    def sync(self) -> None:
        L.check(self._lib.cpb_attn_sync(self._h), "cpb_attn_sync")
