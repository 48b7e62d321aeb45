"""The gpt-oss engine's two-stage LM head on the GPU (ctypes front end of
include/cpb_head.h).

The reference's head_worker (engine_gpt2.rs:937-1002) normalises the final
hidden state with output_norm and quantises it to Q8, screens every
vocabulary row with a Q4 copy of output.weight (each of NT = 12 workers
keeping the CAND = 8 best rows of its slice), recomputes those rows' logits
exactly from the Q8 copy and takes the greedy maximum.  `LmHead` takes the
same bf16 output.weight and output_norm tensors, builds both copies on the
GPU with the reference's quantisers, and returns the greedy token (and, on
request, the candidates and their logits).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib as L


class LmHead:
    def __init__(self, d: int, n_vocab: int, rms_eps: float = 1e-5, n_slices: int = 12, n_cand: int = 8,
                 device: int = 0):
        self._lib = L.lib()
        self.cfg = L.HeadCfg(d, n_vocab, n_slices, n_cand, rms_eps)
        h = C.c_void_p()
        L.check(self._lib.cpb_head_create(C.byref(self.cfg), device, C.byref(h)), "cpb_head_create")
        self._h = h

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.cpb_head_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def load(self, out_w_bf16: np.ndarray, out_norm: np.ndarray) -> None:
        w = np.ascontiguousarray(out_w_bf16, np.uint16)
        nw = np.ascontiguousarray(out_norm, np.float32)
        assert w.shape == (self.cfg.n_vocab, self.cfg.d) and nw.shape == (self.cfg.d,)
        L.check(self._lib.cpb_head_load(self._h, w.ctypes.data_as(C.POINTER(C.c_uint16)), nw.ctypes.data_as(L.f32p)),
                "cpb_head_load")

    def forward(self, x: np.ndarray, trace: bool = False):
        """Greedy token for hidden state x [d]; with trace, also a dict of the
        candidates (ids, Q4 screen values, Q8 logits), xq / xsb and every
        row's screen value."""
        x = np.ascontiguousarray(x, np.float32)
        ch = C.c_int32()
        t = None
        tp = C.cast(None, C.POINTER(L.HeadTrace))
        if trace:
            nc = self.cfg.n_slices * self.cfg.n_cand
            t = {"cand_ids": np.zeros(nc, np.int32), "cand_screen": np.zeros(nc, np.float32),
                 "cand_logits": np.zeros(nc, np.float32), "xq": np.zeros(self.cfg.d, np.int8),
                 "xsb": np.zeros(self.cfg.d // 32, np.float32), "screen": np.zeros(self.cfg.n_vocab, np.float32)}
            tr = L.HeadTrace()
            types = dict(L.HeadTrace._fields_)
            for k, v in t.items():
                setattr(tr, k, v.ctypes.data_as(types[k]))
            tp = C.pointer(tr)
        L.check(self._lib.cpb_head_forward(self._h, x.ctypes.data_as(L.f32p), C.byref(ch), tp), "cpb_head_forward")
        return int(ch.value), t

    def forward_device(self, x_ptr: int, chosen_ptr: int) -> None:
        L.check(self._lib.cpb_head_forward_device(self._h, C.c_void_p(x_ptr), C.c_void_p(chosen_ptr)),
                "cpb_head_forward_device")

    def set_screen(self, bits: int) -> None:
        """4: Q4 screen (default); 2: Q2 screen (the reference's CPBRR_HEAD2)."""
        L.check(self._lib.cpb_head_set_screen(self._h, int(bits)), "cpb_head_set_screen")

    def set_stream(self, stream_ptr: int | None) -> None:
        L.check(self._lib.cpb_head_set_stream(self._h, C.c_void_p(stream_ptr or 0)), "cpb_head_set_stream")

    def sync(self) -> None:
        L.check(self._lib.cpb_head_sync(self._h), "cpb_head_sync")
