"""ctypes front end of the oracle (oracle.c): the CPU restatement of the
reference's MoE expert-FFN decode path.

TEST INFRASTRUCTURE ONLY.  Imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, where it is the checker (or the timed CPU
baseline), never the thing measured on the GPU.  The product package
cpubrrr_amd/ does not import it.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
_LIB = None

f32p = C.POINTER(C.c_float)
i8p = C.POINTER(C.c_int8)
i32p = C.POINTER(C.c_int32)
u8p = C.POINTER(C.c_uint8)


class Trace(C.Structure):
    _fields_ = [("xn", f32p), ("xq", i8p), ("xsb", f32p), ("xsum", i32p), ("logits", f32p),
                ("ids", i32p), ("wts", f32p), ("gu", f32p), ("gu_sums", i32p), ("h", f32p),
                ("hq", i8p), ("hsb", f32p), ("hsum", i32p), ("dn", f32p), ("dn_sums", i32p)]


class GptossLayer(C.Structure):
    _fields_ = [("d", C.c_int), ("dff", C.c_int), ("ne", C.c_int), ("k", C.c_int),
                ("alpha", C.c_float), ("limit", C.c_float), ("eps", C.c_float),
                ("gate", u8p), ("up", u8p), ("down", u8p),
                ("gate_b", f32p), ("up_b", f32p), ("down_b", f32p),
                ("router_w", f32p), ("router_b", f32p), ("norm_w", f32p)]


class QwenLayer(C.Structure):
    _fields_ = [("d", C.c_int), ("dff", C.c_int), ("ne", C.c_int), ("k", C.c_int), ("nt", C.c_int),
                ("eps", C.c_float), ("gate_type", C.c_int), ("up_type", C.c_int), ("down_type", C.c_int),
                ("gate", u8p), ("up", u8p), ("down", u8p), ("router_w", f32p), ("norm_w", f32p)]


def lib() -> C.CDLL:
    global _LIB
    if _LIB is None:
        path = HERE / "liboracle.so"
        if not path.exists():
            from oracle.build import build
            build()
        L = C.CDLL(str(path))
        L.orc_e8m0_half.restype = C.c_float
        L.orc_e8m0_half.argtypes = [C.c_uint8]
        L.orc_half_to_f32.restype = C.c_float
        L.orc_half_to_f32.argtypes = [C.c_uint16]
        L.orc_ssq_gptoss.restype = C.c_float
        L.orc_ssq_gptoss.argtypes = [f32p, C.c_int]
        L.orc_rmsnorm_gptoss.argtypes = [f32p, f32p, C.c_int, C.c_float, f32p]
        L.orc_rmsnorm_qwen.argtypes = [f32p, f32p, C.c_int, C.c_float, C.c_int, f32p]
        L.orc_qblock32.argtypes = [f32p, C.c_int, i8p, f32p]
        L.orc_qblock_k.argtypes = [f32p, C.c_int, i8p, f32p, i32p]
        L.orc_router.argtypes = [f32p, f32p, f32p, C.c_int, C.c_int, f32p]
        L.orc_topk_gptoss.argtypes = [f32p, C.c_int, C.c_int, i32p, f32p]
        L.orc_topk_qwen.argtypes = [f32p, C.c_int, C.c_int, i32p, f32p]
        L.orc_mx_row_dot.restype = C.c_float
        L.orc_mx_row_dot.argtypes = [u8p, i8p, f32p, C.c_int, i32p]
        L.orc_q4k_dot.restype = C.c_float
        L.orc_q4k_dot.argtypes = [u8p, i8p, f32p, i32p, C.c_int, i32p]
        L.orc_q6k_dot.restype = C.c_float
        L.orc_q6k_dot.argtypes = [u8p, i8p, f32p, C.c_int, i32p]
        L.orc_gptoss_moe.argtypes = [C.POINTER(GptossLayer), f32p, C.c_int, C.POINTER(Trace)]
        L.orc_qwen_moe.argtypes = [C.POINTER(QwenLayer), f32p, C.c_int, C.POINTER(Trace)]
        u16p = C.POINTER(C.c_uint16)
        L.orc_f32_to_bf16.restype = C.c_uint16
        L.orc_f32_to_bf16.argtypes = [C.c_float]
        L.orc_bf16_to_f32.restype = C.c_float
        L.orc_bf16_to_f32.argtypes = [C.c_uint16]
        L.orc_q4_scale_search.restype = C.c_uint16
        L.orc_q4_scale_search.argtypes = [f32p, f32p]
        L.orc_q4_quant_row.argtypes = [u16p, C.c_int, u8p, u16p]
        L.orc_q8_quant_row.argtypes = [u16p, C.c_int, i8p, f32p]
        L.orc_q4_row_dot.restype = C.c_float
        L.orc_q4_row_dot.argtypes = [u8p, u16p, i8p, f32p, C.c_int]
        L.orc_q8_row_dot.restype = C.c_float
        L.orc_q8_row_dot.argtypes = [i8p, f32p, i8p, f32p, C.c_int]
        L.orc_gptoss_moe_f64.argtypes = [C.c_void_p, f32p, C.c_int]
        L.orc_gptoss_moe_f64.restype = None
        L.orc_q2_quant_row.argtypes = [u16p, C.c_int, u8p, u16p]
        L.orc_q2_row_dot.restype = C.c_float
        L.orc_q2_row_dot.argtypes = [u8p, u16p, i8p, f32p, C.c_int]
        L.orc_head_q2.argtypes = [u16p, C.c_int, C.c_int, f32p, f32p, C.c_float, C.c_int, C.c_int, i32p, f32p, f32p,
                                  i8p, f32p, i32p]
        L.orc_head_slice_start.argtypes = [C.c_long, C.c_int, C.c_int]
        L.orc_head_slice_start.restype = C.c_long
        L.orc_head.argtypes = [u16p, C.c_int, C.c_int, f32p, f32p, C.c_float, C.c_int, C.c_int, i32p, f32p, f32p,
                               i8p, f32p, i32p]
        L.orc_q4_quant_rows.argtypes = [u16p, C.c_int, C.c_int, u8p, u16p]
        L.orc_head_pre.argtypes = [u16p, u8p, u16p, C.c_int, C.c_int, f32p, f32p, C.c_float, C.c_int, C.c_int, i32p,
                                   f32p, f32p, i8p, f32p, i32p]
        L.orc_set_threads.argtypes = [C.c_int]
        L.orc_get_threads.restype = C.c_int
        _LIB = L
    return _LIB


def _p(a: np.ndarray | None, t):
    if a is None:
        return C.cast(None, t)
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(t)


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def get_threads() -> int:
    return int(lib().orc_get_threads())


def e8m0_half(e: int) -> float:
    return float(lib().orc_e8m0_half(int(e)))


def half_to_f32(h: int) -> float:
    return float(lib().orc_half_to_f32(int(h)))


def ssq_gptoss(x: np.ndarray) -> np.float32:
    x = np.ascontiguousarray(x, np.float32)
    return np.float32(lib().orc_ssq_gptoss(_p(x, f32p), x.size))


def rmsnorm_gptoss(x, w, eps):
    x = np.ascontiguousarray(x, np.float32); w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    lib().orc_rmsnorm_gptoss(_p(x, f32p), _p(w, f32p), x.size, float(eps), _p(out, f32p))
    return out


def rmsnorm_qwen(x, w, eps, nt=12):
    x = np.ascontiguousarray(x, np.float32); w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    lib().orc_rmsnorm_qwen(_p(x, f32p), _p(w, f32p), x.size, float(eps), int(nt), _p(out, f32p))
    return out


def qblock32(x):
    x = np.ascontiguousarray(x, np.float32)
    xq = np.empty(x.size, np.int8); xsb = np.empty(x.size // 32, np.float32)
    lib().orc_qblock32(_p(x, f32p), x.size, _p(xq, i8p), _p(xsb, f32p))
    return xq, xsb


def qblock_k(x):
    x = np.ascontiguousarray(x, np.float32)
    xq = np.empty(x.size, np.int8); ys = np.empty(x.size // 256, np.float32)
    xsum = np.empty(x.size // 32, np.int32)
    lib().orc_qblock_k(_p(x, f32p), x.size, _p(xq, i8p), _p(ys, f32p), _p(xsum, i32p))
    return xq, ys, xsum


def router(W, b, xn):
    W = np.ascontiguousarray(W, np.float32); xn = np.ascontiguousarray(xn, np.float32)
    ne, d = W.shape
    b = None if b is None else np.ascontiguousarray(b, np.float32)
    out = np.empty(ne, np.float32)
    lib().orc_router(_p(W, f32p), _p(b, f32p), _p(xn, f32p), ne, d, _p(out, f32p))
    return out


def topk_gptoss(logits, k):
    logits = np.ascontiguousarray(logits, np.float32)
    ids = np.empty(k, np.int32); w = np.empty(k, np.float32)
    lib().orc_topk_gptoss(_p(logits, f32p), logits.size, k, _p(ids, i32p), _p(w, f32p))
    return ids, w


def topk_qwen(logits, k):
    logits = np.ascontiguousarray(logits, np.float32)
    ids = np.empty(k, np.int32); w = np.empty(k, np.float32)
    lib().orc_topk_qwen(_p(logits, f32p), logits.size, k, _p(ids, i32p), _p(w, f32p))
    return ids, w


def mx_row_dot(row, xq, xsb):
    row = np.ascontiguousarray(row, np.uint8); xq = np.ascontiguousarray(xq, np.int8)
    xsb = np.ascontiguousarray(xsb, np.float32)
    nb = xsb.size
    sums = np.empty(nb, np.int32)
    v = lib().orc_mx_row_dot(_p(row, u8p), _p(xq, i8p), _p(xsb, f32p), nb, _p(sums, i32p))
    return np.float32(v), sums


def q4k_dot(row, xq, ys, xsum):
    row = np.ascontiguousarray(row, np.uint8); xq = np.ascontiguousarray(xq, np.int8)
    ys = np.ascontiguousarray(ys, np.float32); xsum = np.ascontiguousarray(xsum, np.int32)
    sums = np.empty(2 * ys.size, np.int32)
    v = lib().orc_q4k_dot(_p(row, u8p), _p(xq, i8p), _p(ys, f32p), _p(xsum, i32p), xq.size, _p(sums, i32p))
    return np.float32(v), sums


def q6k_dot(row, xq, ys):
    row = np.ascontiguousarray(row, np.uint8); xq = np.ascontiguousarray(xq, np.int8)
    ys = np.ascontiguousarray(ys, np.float32)
    sums = np.empty(ys.size, np.int32)
    v = lib().orc_q6k_dot(_p(row, u8p), _p(xq, i8p), _p(ys, f32p), xq.size, _p(sums, i32p))
    return np.float32(v), sums


def _trace_bufs(d, dff, ne, k, mx: bool, want_sums: bool, down_pairs: bool = False):
    t = {
        "xn": np.zeros(d, np.float32), "xq": np.zeros(d, np.int8),
        "xsb": np.zeros(d // 32 if mx else d // 256, np.float32),
        "xsum": np.zeros(d // 32, np.int32), "logits": np.zeros(ne, np.float32),
        "ids": np.zeros(k, np.int32), "wts": np.zeros(k, np.float32),
        "gu": np.zeros((k, 2, dff), np.float32), "h": np.zeros((k, dff), np.float32),
        "hq": np.zeros((k, dff), np.int8),
        "hsb": np.zeros((k, dff // 32) if mx else (k, dff // 256), np.float32),
        "hsum": np.zeros((k, dff // 32), np.int32), "dn": np.zeros((k, d), np.float32),
    }
    if want_sums:
        t["gu_sums"] = np.zeros((k, 2, dff, d // 32) if mx else (k, 2, dff, d // 256, 2), np.int32)
        t["dn_sums"] = np.zeros((k, d, dff // 32) if mx else
                                ((k, d, dff // 256, 2) if down_pairs else (k, d, dff // 256)), np.int32)
    return t


def _mk_trace(t) -> Trace:
    tr = Trace()
    types = dict(Trace._fields_)
    for name, arr in t.items():
        setattr(tr, name, _p(arr, types[name]))
    return tr


def gptoss_moe(layer: dict, x: np.ndarray, apply_norm: bool, want_sums: bool = False):
    """One gpt-oss MoE block (engine_gpt2.rs:845-923).  Returns (x_out, trace)."""
    d, dff, ne, k = layer["d"], layer["dff"], layer["ne"], layer["k"]
    keep = {n: np.ascontiguousarray(layer[n]) for n in
            ("gate", "up", "down", "gate_b", "up_b", "down_b", "router_w", "router_b", "norm_w")}
    L = GptossLayer(d, dff, ne, k, layer.get("alpha", 1.702), layer.get("limit", 7.0), layer.get("eps", 1e-5),
                    _p(keep["gate"], u8p), _p(keep["up"], u8p), _p(keep["down"], u8p),
                    _p(keep["gate_b"], f32p), _p(keep["up_b"], f32p), _p(keep["down_b"], f32p),
                    _p(keep["router_w"], f32p), _p(keep["router_b"], f32p), _p(keep["norm_w"], f32p))
    xo = np.array(x, np.float32, copy=True)
    t = _trace_bufs(d, dff, ne, k, True, want_sums)
    tr = _mk_trace(t)
    lib().orc_gptoss_moe(C.byref(L), _p(xo, f32p), int(bool(apply_norm)), C.byref(tr))
    return xo, t


def gptoss_moe_f64(layer: dict, x: np.ndarray, apply_norm: bool):
    """scripts/ffn_reference.py's float64 dequant algorithm (scale 2^(e-128))
    on one gpt-oss layer.  Returns x + the layer's MoE output (fp32)."""
    d, dff, ne, k = layer["d"], layer["dff"], layer["ne"], layer["k"]
    keep = {n: np.ascontiguousarray(layer[n]) for n in
            ("gate", "up", "down", "gate_b", "up_b", "down_b", "router_w", "router_b", "norm_w")}
    L = GptossLayer(d, dff, ne, k, layer.get("alpha", 1.702), layer.get("limit", 7.0), layer.get("eps", 1e-5),
                    _p(keep["gate"], u8p), _p(keep["up"], u8p), _p(keep["down"], u8p),
                    _p(keep["gate_b"], f32p), _p(keep["up_b"], f32p), _p(keep["down_b"], f32p),
                    _p(keep["router_w"], f32p), _p(keep["router_b"], f32p), _p(keep["norm_w"], f32p))
    xo = np.array(x, np.float32, copy=True)
    lib().orc_gptoss_moe_f64(C.byref(L), _p(xo, f32p), int(bool(apply_norm)))
    return xo


def qwen_moe(layer: dict, x: np.ndarray, apply_norm: bool, want_sums: bool = False):
    """One Qwen3 MoE block (engine_qwen2.rs:395-433).  Returns (x_out, trace)."""
    d, dff, ne, k = layer["d"], layer["dff"], layer["ne"], layer["k"]
    keep = {n: np.ascontiguousarray(layer[n]) for n in ("gate", "up", "down", "router_w", "norm_w")}
    L = QwenLayer(d, dff, ne, k, layer.get("nt", 12), layer.get("eps", 1e-6),
                  layer.get("gate_type", 12), layer.get("up_type", 12), layer.get("down_type", 14),
                  _p(keep["gate"], u8p), _p(keep["up"], u8p), _p(keep["down"], u8p),
                  _p(keep["router_w"], f32p), _p(keep["norm_w"], f32p))
    xo = np.array(x, np.float32, copy=True)
    t = _trace_bufs(d, dff, ne, k, False, want_sums, layer.get("down_type", 14) == 12)
    tr = _mk_trace(t)
    lib().orc_qwen_moe(C.byref(L), _p(xo, f32p), int(bool(apply_norm)), C.byref(tr))
    return xo, t


# ---- two-stage LM head (oracle/head.c) ----
u16p = C.POINTER(C.c_uint16)


def f32_to_bf16(v: float) -> int:
    return int(lib().orc_f32_to_bf16(float(v)))


def q4_scale_search(vals):
    vals = np.ascontiguousarray(vals, np.float32)
    idq = C.c_float()
    db = lib().orc_q4_scale_search(_p(vals, f32p), C.byref(idq))
    return int(db), np.float32(idq.value)


def q4_quant_row(w_bf16):
    w = np.ascontiguousarray(w_bf16, np.uint16)
    nib = np.empty(w.size // 2, np.uint8); sc = np.empty(w.size // 32, np.uint16)
    lib().orc_q4_quant_row(_p(w, u16p), w.size, _p(nib, u8p), _p(sc, u16p))
    return nib, sc


def q2_quant_row(w_bf16):
    w = np.ascontiguousarray(w_bf16, np.uint16)
    nib = np.empty(w.size // 4, np.uint8); sc = np.empty(w.size // 32, np.uint16)
    lib().orc_q2_quant_row(_p(w, u16p), w.size, _p(nib, u8p), _p(sc, u16p))
    return nib, sc


def q2_row_dot(nib, sc, xq, xsb):
    nib = np.ascontiguousarray(nib, np.uint8); sc = np.ascontiguousarray(sc, np.uint16)
    xq = np.ascontiguousarray(xq, np.int8); xsb = np.ascontiguousarray(xsb, np.float32)
    return np.float32(lib().orc_q2_row_dot(_p(nib, u8p), _p(sc, u16p), _p(xq, i8p), _p(xsb, f32p), xsb.size))


def q8_quant_row(w_bf16):
    w = np.ascontiguousarray(w_bf16, np.uint16)
    q = np.empty(w.size, np.int8); s = np.empty(w.size // 32, np.float32)
    lib().orc_q8_quant_row(_p(w, u16p), w.size, _p(q, i8p), _p(s, f32p))
    return q, s


def q4_row_dot(nib, sc, xq, xsb):
    nib = np.ascontiguousarray(nib, np.uint8); sc = np.ascontiguousarray(sc, np.uint16)
    xq = np.ascontiguousarray(xq, np.int8); xsb = np.ascontiguousarray(xsb, np.float32)
    return np.float32(lib().orc_q4_row_dot(_p(nib, u8p), _p(sc, u16p), _p(xq, i8p), _p(xsb, f32p), xsb.size))


def q8_row_dot(q, s, xq, xsb):
    q = np.ascontiguousarray(q, np.int8); s = np.ascontiguousarray(s, np.float32)
    xq = np.ascontiguousarray(xq, np.int8); xsb = np.ascontiguousarray(xsb, np.float32)
    return np.float32(lib().orc_q8_row_dot(_p(q, i8p), _p(s, f32p), _p(xq, i8p), _p(xsb, f32p), q.size))


def q4_quant_rows(w_bf16):
    """Q4Mat of every row of [V][d] bf16: (nib [V][d/2], sc [V][d/32])."""
    w = np.ascontiguousarray(w_bf16, np.uint16)
    V, d = w.shape
    nib = np.empty((V, d // 2), np.uint8); sc = np.empty((V, d // 32), np.uint16)
    lib().orc_q4_quant_rows(_p(w, u16p), V, d, _p(nib, u8p), _p(sc, u16p))
    return nib, sc


def head_slice_start(n, nt, wid):
    """First item of worker wid's slice of n items (sl(), engine_gpt2.rs:636-642)."""
    return int(lib().orc_head_slice_start(n, nt, wid))


def head(w_bf16, x, norm_w, eps, nt=12, cand=8, pre=None, q2=False):
    """engine_gpt2.rs:937-1002 (greedy).  Returns dict: chosen, cand_ids,
    cand_screen, cand_logits, xq, xsb.  pre: (nib, sc) of q4_quant_rows, or
    None to quantise the Q4 rows inside the call.  q2: the Q2 screen
    (head2_on(), :953-957) instead of the Q4 one."""
    w = np.ascontiguousarray(w_bf16, np.uint16)
    V, d = w.shape
    x = np.ascontiguousarray(x, np.float32); norm_w = np.ascontiguousarray(norm_w, np.float32)
    out = {"cand_ids": np.zeros(nt * cand, np.int32), "cand_screen": np.zeros(nt * cand, np.float32),
           "cand_logits": np.zeros(nt * cand, np.float32), "xq": np.zeros(d, np.int8),
           "xsb": np.zeros(d // 32, np.float32)}
    ch = C.c_int32()
    if pre is not None:
        nib, sc = (np.ascontiguousarray(pre[0], np.uint8), np.ascontiguousarray(pre[1], np.uint16))
        assert nib.shape == (V, d // 2) and sc.shape == (V, d // 32)
        lib().orc_head_pre(_p(w, u16p), _p(nib, u8p), _p(sc, u16p), V, d, _p(x, f32p), _p(norm_w, f32p), float(eps),
                           nt, cand, _p(out["cand_ids"], i32p), _p(out["cand_screen"], f32p),
                           _p(out["cand_logits"], f32p), _p(out["xq"], i8p), _p(out["xsb"], f32p), C.byref(ch))
        out["chosen"] = int(ch.value)
        return out
    fn = lib().orc_head_q2 if q2 else lib().orc_head
    fn(_p(w, u16p), V, d, _p(x, f32p), _p(norm_w, f32p), float(eps), nt, cand,
       _p(out["cand_ids"], i32p), _p(out["cand_screen"], f32p), _p(out["cand_logits"], f32p),
       _p(out["xq"], i8p), _p(out["xsb"], f32p), C.byref(ch))
    out["chosen"] = int(ch.value)
    return out


# ---- attention block, decode (oracle/attn.c) ----
class AttnLayerC(C.Structure):
    _fields_ = [("d", C.c_int), ("nh", C.c_int), ("nkv", C.c_int), ("hd", C.c_int), ("swa", C.c_int),
                ("eps", C.c_float), ("attn_norm", f32p),
                ("wq", i8p), ("sq", f32p), ("wk", i8p), ("sk", f32p), ("wv", i8p), ("sv", f32p),
                ("wo", i8p), ("so", f32p), ("bq", f32p), ("bk", f32p), ("bv", f32p), ("bo", f32p),
                ("sinks", f32p)]


class AttnTraceC(C.Structure):
    _fields_ = [("xq", i8p), ("xsb", f32p), ("q", f32p), ("k", f32p), ("v", f32p), ("ao", f32p), ("aq", i8p),
                ("asb", f32p)]


def rope_table(hd, max_seq, base):
    tab = np.zeros(max_seq * hd, np.float32)
    lib().orc_rope_table.argtypes = [C.c_int, C.c_int, C.c_float, f32p]
    lib().orc_rope_table(hd, max_seq, float(base), _p(tab, f32p))
    return tab


def q8_rows(w_bf16):
    """Q8Mat::from_bf16 of a [rows][cols] bf16 matrix: (q int8 [rows][cols], s [rows][cols/32])."""
    w = np.ascontiguousarray(w_bf16, np.uint16)
    q = np.empty(w.shape, np.int8)
    s = np.empty((w.shape[0], w.shape[1] // 32), np.float32)
    for r in range(w.shape[0]):
        q[r], s[r] = q8_quant_row(w[r])
    return q, s


def attn_layer(L: dict, il: int, pos: int, x, kc, vc, tab):
    """One decode step of the attention block (engine_gpt2.rs:772-843).
    L: d, nh, nkv, hd, swa, eps, attn_norm, q8 weights wq/sq/wk/sk/wv/sv/wo/so
    (see q8_rows), biases bq/bk/bv/bo, sinks.  kc / vc: this layer's cache
    [max_seq][nkv][hd] (updated at pos).  Returns (x_out, trace)."""
    keep = {k: np.ascontiguousarray(L[k]) for k in ("attn_norm", "wq", "sq", "wk", "sk", "wv", "sv", "wo", "so",
                                                     "bq", "bk", "bv", "bo", "sinks")}
    S = AttnLayerC(L["d"], L["nh"], L["nkv"], L["hd"], L["swa"], L["eps"], _p(keep["attn_norm"], f32p),
                   _p(keep["wq"], i8p), _p(keep["sq"], f32p), _p(keep["wk"], i8p), _p(keep["sk"], f32p),
                   _p(keep["wv"], i8p), _p(keep["sv"], f32p), _p(keep["wo"], i8p), _p(keep["so"], f32p),
                   _p(keep["bq"], f32p), _p(keep["bk"], f32p), _p(keep["bv"], f32p), _p(keep["bo"], f32p),
                   _p(keep["sinks"], f32p))
    d, nh, nkv, hd = L["d"], L["nh"], L["nkv"], L["hd"]
    t = {"xq": np.zeros(d, np.int8), "xsb": np.zeros(d // 32, np.float32), "q": np.zeros(nh * hd, np.float32),
         "k": np.zeros(nkv * hd, np.float32), "v": np.zeros(nkv * hd, np.float32),
         "ao": np.zeros(nh * hd, np.float32), "aq": np.zeros(nh * hd, np.int8),
         "asb": np.zeros(nh * hd // 32, np.float32)}
    tr = AttnTraceC(*[_p(t[n], ty) for n, ty in AttnTraceC._fields_])
    xo = np.array(x, np.float32, copy=True)
    lib().orc_attn_layer.argtypes = [C.POINTER(AttnLayerC), C.c_int, C.c_int, f32p, f32p, f32p, f32p,
                                     C.POINTER(AttnTraceC)]
    assert kc.flags["C_CONTIGUOUS"] and vc.flags["C_CONTIGUOUS"]
    lib().orc_attn_layer(C.byref(S), il, pos, _p(xo, f32p), _p(kc, f32p), _p(vc, f32p), _p(tab, f32p), C.byref(tr))
    return xo, t
