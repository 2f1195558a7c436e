"""Python binding of the MI355X MoE block (ctypes over include/tmt_moe.h).

The compute path is the C ABI in ``libtmt_moe.so`` (hand-written gfx950 HIP
kernels). This module only passes device pointers and streams from torch
tensors to that library; it has no fallback implementation and raises if the
library is missing.

Mirrors the reference operator interface (tmt-cuda/src/moe.cu:330-545):
``MoE`` owns the arena (MoeKeep + MoeWs), ``forward`` replaces
``moe_forward``, ``backward`` replaces ``moe_backward`` and ``stats``
replaces the host read of aux / z-loss / expert counts.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence, Union

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libtmt_moe.so")

WEIGHTS_BF16 = 0
WEIGHTS_MXFP4 = 1
WEIGHTS_MXFP4_MX = 2
WEIGHTS_MXFP4_MX_PLANES = 3

EXPORTED = (
    "tmt_moe_create",
    "tmt_moe_destroy",
    "tmt_moe_workspace_size",
    "tmt_moe_workspace_sizes",
    "tmt_moe_create_shared",
    "tmt_moe_forward",
    "tmt_moe_forward_mxfp4",
    "tmt_moe_backward",
    "tmt_moe_forward_ln",
    "tmt_moe_backward_ln",
    "tmt_moe_read_stats",
    "tmt_moe_stats_device_ptr",
    "tmt_moe_read_routing",
    "tmt_moe_read_norm",
    "tmt_moe_layernorm_workspace_size",
    "tmt_moe_layernorm_forward",
    "tmt_moe_layernorm_backward",
    "tmt_moe_layernorm_backward_noalloc",
    "tmt_moe_adamw_create",
    "tmt_moe_adamw_destroy",
    "tmt_moe_adamw_step",
    "tmt_moe_adamw_read_sumsq",
    "tmt_moe_adamw_zero_grads",
    "tmt_moe_adamw_chunks",
    "tmt_moe_f32_to_bf16",
    "tmt_moe_mxfp4_planes",
    "tmt_moe_set_profiling",
    "tmt_moe_read_profile",
    "tmt_moe_phase_name",
    "tmt_moe_last_error",
)

NPHASES = 15


class Desc(ctypes.Structure):
    _fields_ = [
        ("max_tokens", ctypes.c_int32),
        ("d", ctypes.c_int32),
        ("experts", ctypes.c_int32),
        ("topk", ctypes.c_int32),
        ("hidden", ctypes.c_int32),
        ("weight_format", ctypes.c_int32),
    ]


_lib = None


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load libtmt_moe.so; raises FileNotFoundError when it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise FileNotFoundError(
            f"{path} is missing: build it with __graft_entry__.build() "
            "(there is no non-HIP implementation)")
    lib = ctypes.CDLL(path)
    vp, i32, f32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_float
    pp = ctypes.POINTER(ctypes.c_void_p)
    lib.tmt_moe_create.argtypes = [ctypes.POINTER(Desc), ctypes.POINTER(vp)]
    lib.tmt_moe_destroy.argtypes = [vp]
    lib.tmt_moe_workspace_size.argtypes = [ctypes.POINTER(Desc), ctypes.POINTER(ctypes.c_size_t)]
    lib.tmt_moe_workspace_sizes.argtypes = [ctypes.POINTER(Desc), ctypes.POINTER(ctypes.c_size_t),
                                            ctypes.POINTER(ctypes.c_size_t)]
    lib.tmt_moe_create_shared.argtypes = [ctypes.POINTER(Desc), vp, ctypes.c_size_t, ctypes.POINTER(vp)]
    lib.tmt_moe_forward.argtypes = [vp, vp, i32, vp, vp, vp, pp, pp, vp, f32]
    lib.tmt_moe_forward_mxfp4.argtypes = [vp, vp, i32, vp, vp, vp, pp, pp, pp, pp, vp, f32]
    lib.tmt_moe_backward.argtypes = [vp, vp, vp, vp, vp, pp, pp, f32, f32, vp, vp, pp, pp]
    lib.tmt_moe_forward_ln.argtypes = [vp, vp, i32, vp, vp, vp, vp, vp, pp, pp, vp, f32]
    lib.tmt_moe_backward_ln.argtypes = [vp, vp, vp, vp, vp, vp, pp, pp, f32, f32, vp, vp, vp, vp,
                                        pp, pp]
    lib.tmt_moe_read_norm.argtypes = [vp, vp, vp, vp, vp]
    lib.tmt_moe_layernorm_workspace_size.argtypes = [i32, i32, ctypes.POINTER(ctypes.c_size_t)]
    lib.tmt_moe_layernorm_forward.argtypes = [vp, i32, i32, vp, vp, vp, vp, vp, vp]
    lib.tmt_moe_layernorm_backward.argtypes = [vp, i32, i32, vp, vp, vp, vp, vp, vp, vp, vp, vp,
                                               ctypes.c_size_t]
    lib.tmt_moe_layernorm_backward_noalloc.argtypes = [vp, i32, i32, vp, vp, vp, vp, vp, vp, vp, vp]
    lib.tmt_moe_adamw_create.argtypes = [vp, i32, ctypes.POINTER(vp)]
    lib.tmt_moe_adamw_destroy.argtypes = [vp]
    lib.tmt_moe_adamw_step.argtypes = [vp, vp, f32, f32, f32, f32, f32, f32, i32]
    lib.tmt_moe_adamw_read_sumsq.argtypes = [vp, vp, ctypes.POINTER(ctypes.c_double)]
    lib.tmt_moe_adamw_zero_grads.argtypes = [vp, vp]
    lib.tmt_moe_adamw_chunks.argtypes = [vp, ctypes.POINTER(i32)]
    lib.tmt_moe_f32_to_bf16.argtypes = [vp, vp, vp, ctypes.c_int64]
    lib.tmt_moe_mxfp4_planes.argtypes = [vp, vp, i32, i32, vp]
    lib.tmt_moe_read_stats.argtypes = [vp, vp, vp, vp, vp]
    lib.tmt_moe_stats_device_ptr.argtypes = [vp, pp]
    lib.tmt_moe_read_routing.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, vp]
    lib.tmt_moe_set_profiling.argtypes = [vp, ctypes.c_int]
    lib.tmt_moe_read_profile.argtypes = [vp, vp, vp, ctypes.c_int]
    lib.tmt_moe_phase_name.argtypes = [ctypes.c_int]
    lib.tmt_moe_phase_name.restype = ctypes.c_char_p
    lib.tmt_moe_last_error.restype = ctypes.c_char_p
    for name in EXPORTED:
        if name not in ("tmt_moe_last_error", "tmt_moe_phase_name"):
            getattr(lib, name).restype = ctypes.c_int
    _lib = lib
    return lib


def last_error() -> str:
    return load_library().tmt_moe_last_error().decode()


class MoeError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"tmt_moe error {code}: {msg}")
        self.code = code


def _check(rc: int) -> None:
    if rc != 0:
        raise MoeError(rc, last_error())


def _ptr(t) -> int:
    return 0 if t is None else int(t.data_ptr())


def _table(ws, n: int) -> Optional[ctypes.Array]:
    """Pointer table from a stacked [E, ...] tensor or a list of tensors."""
    if ws is None:
        return None
    if isinstance(ws, (list, tuple)):
        ptrs = [_ptr(w) for w in ws]
    else:
        stride = ws.stride(0) * ws.element_size()
        base = _ptr(ws)
        ptrs = [base + e * stride for e in range(n)]
    if len(ptrs) != n:
        raise ValueError(f"expected {n} per-expert tensors, got {len(ptrs)}")
    return (ctypes.c_void_p * n)(*ptrs)


def _stream(stream) -> int:
    import torch
    if stream is None:
        stream = torch.cuda.current_stream()
    return int(stream.cuda_stream)


def workspace_size(max_tokens: int, d: int, experts: int, topk: int, hidden: int,
                   weight_format: int = WEIGHTS_BF16) -> int:
    lib = load_library()
    desc = Desc(max_tokens, d, experts, topk, hidden, weight_format)
    out = ctypes.c_size_t(0)
    _check(lib.tmt_moe_workspace_size(ctypes.byref(desc), ctypes.byref(out)))
    return int(out.value)


def workspace_sizes(max_tokens: int, d: int, experts: int, topk: int, hidden: int,
                    weight_format: int = WEIGHTS_BF16) -> tuple:
    """(per-layer bytes, shared bytes) of a handle's device memory."""
    lib = load_library()
    desc = Desc(max_tokens, d, experts, topk, hidden, weight_format)
    a, b = ctypes.c_size_t(0), ctypes.c_size_t(0)
    _check(lib.tmt_moe_workspace_sizes(ctypes.byref(desc), ctypes.byref(a), ctypes.byref(b)))
    return int(a.value), int(b.value)


def layernorm_workspace_size(T: int, d: int) -> int:
    """Bytes of device workspace layernorm_backward needs for [T, d]."""
    out = ctypes.c_size_t(0)
    _check(load_library().tmt_moe_layernorm_workspace_size(T, d, ctypes.byref(out)))
    return int(out.value)


def layernorm_forward(S, gamma, beta, H, mean, rstd, stream=None) -> None:
    """Standalone LayerNorm (the reference's layernorm_fwd): H = LN(S),
    mean / rstd [T] written. S, H: [T, d] bf16; gamma, beta: [d] fp32."""
    T, d = int(S.shape[0]), int(S.shape[1])
    _check(load_library().tmt_moe_layernorm_forward(
        _stream(stream), T, d, _ptr(S), _ptr(gamma), _ptr(beta), _ptr(H), _ptr(mean), _ptr(rstd)))


def layernorm_backward(S, dH, gamma, mean, rstd, dS, dGamma, dBeta, workspace,
                       stream=None) -> None:
    """Standalone LayerNorm backward (the reference's layernorm_bwd) from the
    bf16 gradient dH; workspace is a device buffer of at least
    layernorm_workspace_size(T, d) bytes."""
    T, d = int(S.shape[0]), int(S.shape[1])
    nbytes = workspace.numel() * workspace.element_size()
    _check(load_library().tmt_moe_layernorm_backward(
        _stream(stream), T, d, _ptr(S), _ptr(dH), _ptr(gamma), _ptr(mean), _ptr(rstd), _ptr(dS),
        _ptr(dGamma), _ptr(dBeta), _ptr(workspace), ctypes.c_size_t(nbytes)))


def layernorm_backward_noalloc(S, dH, gamma, mean, rstd, dS, dGamma, dBeta, stream=None) -> None:
    """layernorm_backward over the library's own 4 MiB device scratch (no
    allocation, no workspace argument; calls overlapping on one GPU race)."""
    T, d = int(S.shape[0]), int(S.shape[1])
    _check(load_library().tmt_moe_layernorm_backward_noalloc(
        _stream(stream), T, d, _ptr(S), _ptr(dH), _ptr(gamma), _ptr(mean), _ptr(rstd), _ptr(dS),
        _ptr(dGamma), _ptr(dBeta)))


def mxfp4_planes(codes, planes, stream=None) -> None:
    """MXFP4 weight codes [N, K/2] (uint8, the tmt_moe_forward_mxfp4 layout)
    to the K-plane layout [K/64, N, 32] that WEIGHTS_MXFP4_MX_PLANES handles
    take: one expert matrix, device tensors, enqueued on `stream`."""
    N, half = int(codes.shape[0]), int(codes.shape[1])
    _check(load_library().tmt_moe_mxfp4_planes(_stream(stream), _ptr(codes), N, 2 * half, _ptr(planes)))


class MoE:
    """One MoE layer's device state (the reference's MoeKeep + MoeWs)."""

    def __init__(self, max_tokens: int, d: int, experts: int, topk: int,
                 hidden: int = 0, weight_format: int = WEIGHTS_BF16, workspace=None):
        """workspace: optional device tensor shared with other layers
        (tmt_moe_create_shared; at least workspace_sizes(...)[1] bytes,
        kept alive by the caller while this layer exists)."""
        self.lib = load_library()
        self.desc = Desc(max_tokens, d, experts, topk, hidden, weight_format)
        self.E, self.K, self.d, self.h = experts, topk, d, hidden
        self.hn = hidden if hidden > 0 else d
        h = ctypes.c_void_p(0)
        if workspace is None:
            _check(self.lib.tmt_moe_create(ctypes.byref(self.desc), ctypes.byref(h)))
        else:
            nbytes = workspace.numel() * workspace.element_size()
            _check(self.lib.tmt_moe_create_shared(ctypes.byref(self.desc), _ptr(workspace),
                                                  nbytes, ctypes.byref(h)))
        self._workspace = workspace
        self.handle = h
        self.T = None

    def close(self) -> None:
        if getattr(self, "handle", None) is not None and self.handle.value:
            self.lib.tmt_moe_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def forward(self, X, Wr, W_up, W_down, Y, beta: float = 1.0, bias=None,
                stream=None) -> None:
        """Y <- beta*Y + MoE(X). X, Y: [T, d] bf16; Wr: [E, d] bf16;
        W_up: [E, hn, d] (or list); W_down: [E, d, h] (or list, hidden > 0);
        bias: optional [E] fp32 logit bias."""
        T = int(X.shape[0])
        _check(self.lib.tmt_moe_forward(
            self.handle, _stream(stream), T, _ptr(X), _ptr(Wr), _ptr(bias),
            _table(W_up, self.E), _table(W_down, self.E) if self.h > 0 else None,
            _ptr(Y), ctypes.c_float(beta)))
        self.T = T

    def forward_mxfp4(self, X, Wr, W_up, W_up_scale, W_down, W_down_scale, Y,
                      beta: float = 1.0, bias=None, stream=None) -> None:
        T = int(X.shape[0])
        _check(self.lib.tmt_moe_forward_mxfp4(
            self.handle, _stream(stream), T, _ptr(X), _ptr(Wr), _ptr(bias),
            _table(W_up, self.E), _table(W_up_scale, self.E),
            _table(W_down, self.E), _table(W_down_scale, self.E),
            _ptr(Y), ctypes.c_float(beta)))
        self.T = T

    def backward(self, dY, X, Wr, W_up, W_down, dX, dWr, dW_up, dW_down,
                 aux_coef: float = 0.0, z_coef: float = 0.0, stream=None) -> None:
        """Gradients of <dY, Y> + aux_coef*aux + z_coef*z (outputs overwritten)."""
        _check(self.lib.tmt_moe_backward(
            self.handle, _stream(stream), _ptr(dY), _ptr(X), _ptr(Wr),
            _table(W_up, self.E), _table(W_down, self.E) if self.h > 0 else None,
            ctypes.c_float(aux_coef), ctypes.c_float(z_coef), _ptr(dX), _ptr(dWr),
            _table(dW_up, self.E), _table(dW_down, self.E) if self.h > 0 else None))

    def forward_ln(self, S, ln_gamma, ln_beta, Wr, W_up, W_down, Y, beta: float = 1.0,
                   bias=None, stream=None) -> None:
        """Y <- beta*Y + MoE(LayerNorm(S)). S, Y: [T, d] bf16; ln_gamma,
        ln_beta: [d] fp32 (the recurrent block's layernorm_fwd + moe_forward)."""
        T = int(S.shape[0])
        _check(self.lib.tmt_moe_forward_ln(
            self.handle, _stream(stream), T, _ptr(S), _ptr(ln_gamma), _ptr(ln_beta), _ptr(Wr),
            _ptr(bias), _table(W_up, self.E), _table(W_down, self.E) if self.h > 0 else None,
            _ptr(Y), ctypes.c_float(beta)))
        self.T = T

    def backward_ln(self, dY, S, ln_gamma, Wr, W_up, W_down, dS, dGamma, dBeta, dWr, dW_up,
                    dW_down, aux_coef: float = 0.0, z_coef: float = 0.0, stream=None) -> None:
        """Backward of forward_ln (outputs overwritten): dS [T, d] bf16,
        dGamma / dBeta [d] fp32, and the MoE weight gradients."""
        _check(self.lib.tmt_moe_backward_ln(
            self.handle, _stream(stream), _ptr(dY), _ptr(S), _ptr(ln_gamma), _ptr(Wr),
            _table(W_up, self.E), _table(W_down, self.E) if self.h > 0 else None,
            ctypes.c_float(aux_coef), ctypes.c_float(z_coef), _ptr(dS), _ptr(dGamma),
            _ptr(dBeta), _ptr(dWr), _table(dW_up, self.E),
            _table(dW_down, self.E) if self.h > 0 else None))

    def norm(self, stream=None) -> dict:
        """Host copies of what the last forward_ln kept: H (bf16 bits), mean, rstd."""
        T, d = self.T, self.d
        out = {"H": np.zeros((T, d), np.uint16), "mean": np.zeros(T, np.float32),
               "rstd": np.zeros(T, np.float32)}
        _check(self.lib.tmt_moe_read_norm(self.handle, _stream(stream), out["H"].ctypes.data,
                                          out["mean"].ctypes.data, out["rstd"].ctypes.data))
        return out

    def stats(self, stream=None):
        """(aux, z, counts[E]) of the last forward; synchronises the stream."""
        aux = ctypes.c_float(0)
        z = ctypes.c_float(0)
        counts = np.zeros(self.E, dtype=np.int32)
        _check(self.lib.tmt_moe_read_stats(self.handle, _stream(stream), ctypes.byref(aux),
                                           ctypes.byref(z), counts.ctypes.data))
        return float(aux.value), float(z.value), counts

    def set_profiling(self, enable: bool) -> None:
        """Bracket every kernel launch with HIP events (per-phase timing)."""
        _check(self.lib.tmt_moe_set_profiling(self.handle, 1 if enable else 0))

    def profile(self, reset: bool = True) -> dict:
        """{phase: (total_ms, launches)} since the last reset; waits for events."""
        ms = np.zeros(NPHASES, np.float32)
        cnt = np.zeros(NPHASES, np.int32)
        _check(self.lib.tmt_moe_read_profile(self.handle, ms.ctypes.data, cnt.ctypes.data,
                                             1 if reset else 0))
        return {self.lib.tmt_moe_phase_name(i).decode(): (float(ms[i]), int(cnt[i]))
                for i in range(NPHASES)}

    def routing(self, stream=None) -> dict:
        """Host copies of the last forward's routing."""
        T, E, K = self.T, self.E, self.K
        out = {
            "logits": np.zeros((T, E), np.float32),
            "probs": np.zeros((T, E), np.float32),
            "idx": np.zeros((T, K), np.int32),
            "gate": np.zeros((T, K), np.float32),
            "offsets": np.zeros(E + 1, np.int32),
            "perm": np.zeros(T * K, np.int32),
            "slot_of": np.zeros((T, K), np.int32),
        }
        _check(self.lib.tmt_moe_read_routing(
            self.handle, _stream(stream), *(out[k].ctypes.data for k in
                                            ("logits", "probs", "idx", "gate", "offsets",
                                             "perm", "slot_of"))))
        return out


ADAMW_IN_NORM = 1
ADAMW_UPDATE = 2


class AdamwParam(ctypes.Structure):
    _fields_ = [("master", ctypes.c_void_p), ("m", ctypes.c_void_p), ("v", ctypes.c_void_p),
                ("grad", ctypes.c_void_p), ("work", ctypes.c_void_p), ("n", ctypes.c_int64),
                ("flags", ctypes.c_int32)]


class AdamW:
    """Multi-tensor AdamW with global-norm clipping (the reference's MTParams
    optimizer). params: list of dicts of fp32 CUDA tensors master, m, v, grad
    (same numel), optional bf16 work, and flags (ADAMW_IN_NORM | ADAMW_UPDATE).
    The tensors must stay alive while the optimizer exists."""

    def __init__(self, params):
        self.lib = load_library()
        self._keep = params
        arr = (AdamwParam * max(len(params), 1))()
        for i, q in enumerate(params):
            n = q["master"].numel()
            for k in ("m", "v", "grad"):
                assert q[k].numel() == n, k
            if q.get("work") is not None:
                assert q["work"].numel() == n
            arr[i] = AdamwParam(_ptr(q["master"]), _ptr(q["m"]), _ptr(q["v"]), _ptr(q["grad"]),
                                _ptr(q.get("work")), n, int(q.get("flags", ADAMW_IN_NORM | ADAMW_UPDATE)))
        h = ctypes.c_void_p(0)
        _check(self.lib.tmt_moe_adamw_create(ctypes.cast(arr, ctypes.c_void_p), len(params),
                                             ctypes.byref(h)))
        self.handle = h

    def step(self, step: int, lr: float, clip: float = 0.0, beta1: float = 0.9,
             beta2: float = 0.999, eps: float = 1e-8, weight_decay: float = 0.01,
             stream=None) -> None:
        """Enqueue one update; step is the 1-based update count."""
        f = ctypes.c_float
        _check(self.lib.tmt_moe_adamw_step(self.handle, _stream(stream), f(clip), f(lr), f(beta1),
                                           f(beta2), f(eps), f(weight_decay), int(step)))

    def sumsq(self, stream=None) -> float:
        """Squared gradient norm of the last step (waits for the stream)."""
        out = ctypes.c_double(0)
        _check(self.lib.tmt_moe_adamw_read_sumsq(self.handle, _stream(stream), ctypes.byref(out)))
        return out.value

    def zero_grads(self, stream=None) -> None:
        _check(self.lib.tmt_moe_adamw_zero_grads(self.handle, _stream(stream)))

    @property
    def chunks(self) -> int:
        out = ctypes.c_int32(0)
        _check(self.lib.tmt_moe_adamw_chunks(self.handle, ctypes.byref(out)))
        return out.value

    def close(self) -> None:
        if getattr(self, "handle", None) is not None and self.handle.value:
            self.lib.tmt_moe_adamw_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
