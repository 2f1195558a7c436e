"""ctypes wrapper of the CPU oracle (liboracle_moe.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker, never as the measured or
shipped path. See moe_oracle.h for the semantics and reference citations.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle_moe.so")


class Dims(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("T", "d", "E", "K", "h", "threads")]


_lib = None


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(f"{LIB_PATH} missing; run `make -C oracle`")
        _lib = ctypes.CDLL(LIB_PATH)
        _lib.orc_router_logit.restype = ctypes.c_float
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _tab(arrs):
    return (ctypes.c_void_p * len(arrs))(*[a.ctypes.data for a in arrs])


def _dims(T, d, E, K, h, threads=0):
    return Dims(T, d, E, K, h, threads)


def _c(a, dt):
    return None if a is None else np.ascontiguousarray(a, dtype=dt)


def router_logit(x, w) -> float:
    x = _c(x, np.uint16)
    w = _c(w, np.uint16)
    return float(load().orc_router_logit(_p(x), _p(w), ctypes.c_int32(x.size)))


def router(X, Wr, K, bias=None, threads=0) -> dict:
    X, Wr = _c(X, np.uint16), _c(Wr, np.uint16)
    bias = _c(bias, np.float32)
    T, d = X.shape
    E = Wr.shape[0]
    out = {"logits": np.zeros((T, E), np.float32), "probs": np.zeros((T, E), np.float32),
           "idx": np.zeros((T, K), np.int32), "gate": np.zeros((T, K), np.float32),
           "lse": np.zeros(T, np.float32)}
    dm = _dims(T, d, E, K, 0, threads)
    rc = load().orc_router(ctypes.byref(dm), _p(X), _p(Wr), _p(bias), _p(out["logits"]),
                           _p(out["probs"]), _p(out["idx"]), _p(out["gate"]), _p(out["lse"]))
    assert rc == 0, rc
    return out


def dispatch(idx, E) -> dict:
    idx = _c(idx, np.int32)
    T, K = idx.shape
    out = {"counts": np.zeros(E, np.int32), "offsets": np.zeros(E + 1, np.int32),
           "perm": np.zeros(T * K, np.int32), "slot_of": np.zeros((T, K), np.int32)}
    dm = _dims(T, 1, E, K, 0)
    rc = load().orc_dispatch(ctypes.byref(dm), _p(idx), _p(out["counts"]), _p(out["offsets"]),
                             _p(out["perm"]), _p(out["slot_of"]))
    assert rc == 0, rc
    return out


def aux_z(probs, counts, lse, K):
    probs = _c(probs, np.float32)
    T, E = probs.shape
    aux, z = ctypes.c_float(0), ctypes.c_float(0)
    dm = _dims(T, 1, E, K, 0)
    rc = load().orc_aux_z(ctypes.byref(dm), _p(probs), _p(_c(counts, np.int32)),
                          _p(_c(lse, np.float32)), ctypes.byref(aux), ctypes.byref(z))
    assert rc == 0, rc
    return aux.value, z.value


def forward(X, Wr, W_up, W_down, K, h, bias=None, Y_in=None, beta=0.0, threads=0) -> dict:
    X = _c(X, np.uint16)
    T, d = X.shape
    E = W_up.shape[0]
    ups = [np.ascontiguousarray(W_up[e], dtype=np.uint16) for e in range(E)]
    downs = [np.ascontiguousarray(W_down[e], dtype=np.uint16) for e in range(E)] if h > 0 else None
    Wr = _c(Wr, np.uint16)
    out = {"Y": np.zeros((T, d), np.float32), "logits": np.zeros((T, E), np.float32),
           "probs": np.zeros((T, E), np.float32), "idx": np.zeros((T, K), np.int32),
           "gate": np.zeros((T, K), np.float32), "counts": np.zeros(E, np.int32),
           "offsets": np.zeros(E + 1, np.int32), "perm": np.zeros(T * K, np.int32),
           "slot_of": np.zeros((T, K), np.int32)}
    aux, z = ctypes.c_float(0), ctypes.c_float(0)
    dm = _dims(T, d, E, K, h, threads)
    rc = load().orc_forward(
        ctypes.byref(dm), _p(X), _p(Wr), _p(_c(bias, np.float32)), _tab(ups),
        _tab(downs) if downs else None, _p(_c(Y_in, np.uint16)), ctypes.c_float(beta),
        _p(out["Y"]), _p(out["logits"]), _p(out["probs"]), _p(out["idx"]), _p(out["gate"]),
        _p(out["counts"]), _p(out["offsets"]), _p(out["perm"]), _p(out["slot_of"]),
        ctypes.byref(aux), ctypes.byref(z))
    assert rc == 0, rc
    out["aux"], out["z"] = aux.value, z.value
    return out


def backward(X, Wr, W_up, W_down, dY, K, h, bias=None, aux_coef=0.0, z_coef=0.0,
             threads=0) -> dict:
    X, dY = _c(X, np.uint16), _c(dY, np.uint16)
    T, d = X.shape
    E = W_up.shape[0]
    hn = h if h > 0 else d
    ups = [np.ascontiguousarray(W_up[e], dtype=np.uint16) for e in range(E)]
    downs = [np.ascontiguousarray(W_down[e], dtype=np.uint16) for e in range(E)] if h > 0 else None
    out = {"dX": np.zeros((T, d), np.float32), "dWr": np.zeros((E, d), np.float32),
           "dW_up": np.zeros((E, hn, d), np.float32),
           "dW_down": np.zeros((E, d, h), np.float32) if h > 0 else None}
    dup = [out["dW_up"][e] for e in range(E)]
    ddn = [out["dW_down"][e] for e in range(E)] if h > 0 else None
    dm = _dims(T, d, E, K, h, threads)
    rc = load().orc_backward(
        ctypes.byref(dm), _p(X), _p(_c(Wr, np.uint16)), _p(_c(bias, np.float32)), _tab(ups),
        _tab(downs) if downs else None, _p(dY), ctypes.c_float(aux_coef), ctypes.c_float(z_coef),
        _p(out["dX"]), _p(out["dWr"]), _tab(dup), _tab(ddn) if ddn else None)
    assert rc == 0, rc
    return out


def loss_f64(X, Wr, W_up, W_down, dY, K, h, bias=None, aux_coef=0.0, z_coef=0.0,
             grads=True) -> dict:
    X = _c(X, np.float64)
    dY = _c(dY, np.float64)
    T, d = X.shape
    E = W_up.shape[0]
    hn = h if h > 0 else d
    out = {"loss": ctypes.c_double(0), "idx": np.zeros((T, K), np.int32)}
    g = {}
    if grads:
        g = {"dX": np.zeros((T, d)), "dWr": np.zeros((E, d)), "dW_up": np.zeros((E, hn, d)),
             "dW_down": np.zeros((E, d, h)) if h > 0 else None}
    dm = _dims(T, d, E, K, h)
    rc = load().orc_loss_f64(
        ctypes.byref(dm), _p(X), _p(_c(Wr, np.float64)), _p(_c(bias, np.float64)),
        _p(_c(W_up, np.float64)), _p(_c(W_down, np.float64)), _p(dY),
        ctypes.c_double(aux_coef), ctypes.c_double(z_coef), ctypes.byref(out["loss"]),
        _p(g.get("dX")), _p(g.get("dWr")), _p(g.get("dW_up")), _p(g.get("dW_down")),
        _p(out["idx"]))
    assert rc == 0, rc
    res = {"loss": out["loss"].value, "idx": out["idx"]}
    res.update(g)
    return res


def router_bwd(logits, idx, s, counts, aux_coef, z_coef) -> np.ndarray:
    logits = _c(logits, np.float32)
    T, E = logits.shape
    K = idx.shape[1]
    out = np.zeros((T, E), np.float32)
    dm = _dims(T, 1, E, K, 0)
    rc = load().orc_router_bwd(ctypes.byref(dm), _p(logits), _p(_c(idx, np.int32)),
                               _p(_c(s, np.float32)), _p(_c(counts, np.int32)),
                               ctypes.c_float(aux_coef), ctypes.c_float(z_coef), _p(out))
    assert rc == 0, rc
    return out


def mxfp4_quantize(w: np.ndarray):
    w = _c(w, np.float32)
    rows, n = w.reshape(-1, w.shape[-1]).shape
    packed = np.zeros((rows, n // 2), np.uint8)
    scales = np.zeros((rows, n // 32), np.uint8)
    rc = load().orc_mxfp4_quantize(_p(w), ctypes.c_int64(rows), ctypes.c_int64(n), _p(packed), _p(scales))
    assert rc == 0, rc
    return packed.reshape(*w.shape[:-1], n // 2), scales.reshape(*w.shape[:-1], n // 32)


def mxfp4_dequantize(packed, scales, n: int) -> np.ndarray:
    packed, scales = _c(packed, np.uint8), _c(scales, np.uint8)
    rows = packed.size // (n // 2)
    out = np.zeros((rows, n), np.float32)
    rc = load().orc_mxfp4_dequantize(_p(packed), _p(scales), ctypes.c_int64(rows), ctypes.c_int64(n), _p(out))
    assert rc == 0, rc
    return out.reshape(*packed.shape[:-1], n)


def layernorm(S, gamma, beta):
    """LayerNorm forward: H (bf16 bits), mean, rstd (canonical order)."""
    S = _c(S, np.uint16)
    T, d = S.shape
    g, b = _c(gamma, np.float32), _c(beta, np.float32)
    H = np.empty((T, d), np.uint16)
    mean = np.empty(T, np.float32)
    rstd = np.empty(T, np.float32)
    rc = load().orc_layernorm_fwd(T, d, _p(S), _p(g), _p(b), _p(H), _p(mean), _p(rstd))
    assert rc == 0, rc
    return {"H": H, "mean": mean, "rstd": rstd}


def adamw_step(params, clip, lr, b1, b2, eps, wd, step):
    """One multi-tensor AdamW step in place. params: list of dicts with fp32
    arrays master, m, v, grad (C-contiguous, modified in place), optional
    uint16 work, and int flags (1: in the norm, 2: updated). Returns the
    squared gradient norm in the canonical order."""
    cnt = len(params)
    for q in params:
        for k in ("master", "m", "v", "grad"):
            assert q[k].dtype == np.float32 and q[k].flags["C_CONTIGUOUS"], k
        if q.get("work") is not None:
            assert q["work"].dtype == np.uint16 and q["work"].flags["C_CONTIGUOUS"]
    ptrs = lambda key: (ctypes.c_void_p * max(cnt, 1))(
        *[(q[key].ctypes.data if q.get(key) is not None else None) for q in params])
    n = np.array([q["master"].size for q in params] or [0], np.int64)
    flags = np.array([q["flags"] for q in params] or [0], np.int32)
    s = ctypes.c_double(0)
    f = ctypes.c_float
    rc = load().orc_adamw_step(cnt, ptrs("master"), ptrs("m"), ptrs("v"), ptrs("grad"), ptrs("work"),
                               _p(n), _p(flags), f(clip), f(lr), f(b1), f(b2), f(eps), f(wd),
                               ctypes.c_int32(step), ctypes.byref(s))
    assert rc == 0, rc
    return s.value


def layernorm_bwd(S, dH, gamma, mean, rstd):
    """LayerNorm backward from the fp32 gradient dH of its output."""
    S = _c(S, np.uint16)
    T, d = S.shape
    dH = _c(dH, np.float32)
    dS = np.empty((T, d), np.float32)
    dg = np.empty(d, np.float32)
    db = np.empty(d, np.float32)
    rc = load().orc_layernorm_bwd(T, d, _p(S), _p(dH), _p(_c(gamma, np.float32)), _p(_c(mean, np.float32)),
                                  _p(_c(rstd, np.float32)), _p(dS), _p(dg), _p(db))
    assert rc == 0, rc
    return {"dS": dS, "dgamma": dg, "dbeta": db}

