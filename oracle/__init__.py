"""CPU oracle for the HIP kernels: numpy front end of ``oracle/liboracle.so``.

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and bench.py's
``cpu_baseline`` leg, as the checker. The product library never uses it.

The C++ restatement (``hk_oracle.cpp``) follows the reference harnesses' CPU references; see the
file:line citation at each function there. Parity pinning of each function (against the
reference's own checks, closed forms, invariants and brute force) lives in
``tests/test_oracle.py``; no function of this oracle is left unpinned.
"""
from __future__ import annotations

import ctypes
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_i64, _u64, _f, _i = ctypes.c_int64, ctypes.c_uint64, ctypes.c_float, ctypes.c_int


class _NullableF32(object):
    """ndpointer that also accepts None (passed as NULL)."""

    @classmethod
    def from_param(cls, obj):
        if obj is None:
            return ctypes.c_void_p(0)
        return _f32p.from_param(obj)


class _NullableU16(object):
    @classmethod
    def from_param(cls, obj):
        if obj is None:
            return ctypes.c_void_p(0)
        return _u16p.from_param(obj)


_SIGS = {
    "oracle_set_threads": (None, [_i]),
    "oracle_max_threads": (_i, []),
    "oracle_hardware_concurrency": (_i, []),
    "oracle_f32_to_bf16": (None, [_f32p, _u16p, _i64]),
    "oracle_bf16_to_f32": (None, [_u16p, _f32p, _i64]),
    "oracle_rand_uniform": (None, [_f32p, _i64, _u64, _f, _f]),
    "oracle_splitmix_uniform": (None, [_f32p, _i64, _u64, _f, _f]),
    "oracle_normal": (None, [_f32p, _i64, _u64, _f, _f]),
    "oracle_gelu_forward_f32": (None, [_f32p, _f32p, _i64]),
    "oracle_gelu_backward_f32": (None, [_f32p, _f32p, _f32p, _i64]),
    "oracle_gelu_backward_fd_f32": (None, [_f32p, _f32p, _f32p, _i64]),
    "oracle_gelu_forward_bf16": (None, [_u16p, _f32p, _i64]),
    "oracle_gelu_backward_bf16": (None, [_u16p, _u16p, _f32p, _i64]),
    "oracle_layer_norm_forward": (None, [_f32p, _NullableF32, _NullableF32, _f32p, _NullableF32,
                                         _NullableF32, _i64, _i64, _f]),
    "oracle_ln_backward_input": (None, [_f32p, _f32p, _f32p, _f32p, _NullableF32, _f32p, _i64,
                                        _i64]),
    "oracle_ln_backward_gamma_beta": (None, [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _i64,
                                             _i64]),
    "oracle_sparse_ce_forward": (None, [_f32p, _i32p, _f32p, _f32p, _f32p, _i64, _i64]),
    "oracle_sparse_ce_backward": (None, [_f32p, _i32p, _f32p, _f32p, _f32p, _i64, _i64, _f]),
    "oracle_adamw": (None, [_f32p, _f32p, _f32p, _f32p, _i64, _f, _f, _f, _f, _f, _f, _f]),
    "oracle_reduce_inner": (None, [_f32p, _f32p, _i64, _i64, _i64]),
    "oracle_reduce_outer": (None, [_f32p, _f32p, _i64, _i64, _i64, _i64, _i64]),
    "oracle_reduce_selftest_input": (None, [_f32p, _i64]),
    "oracle_attn_forward": (None, [_f32p, _f32p, _f32p, _i, _i, _i, _i, _f, _i, _NullableF32,
                                   _f32p, _f32p]),
    "oracle_attn_precompute_D": (None, [_f32p, _f32p, _f32p, _i64, _i]),
    "oracle_attn_backward": (None, [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _i, _i, _i, _i, _f,
                                    _i, _f32p, _f32p, _f32p, _f32p]),
    "oracle_sgemm": (None, [_i, _i, _i64, _i64, _i64, _f, _f32p, _i64, _f32p, _i64, _f,
                            _NullableF32, _i64, _NullableF32, _f32p, _i64]),
    "oracle_bgemm": (None, [_i, _i, _i64, _i64, _i64, _f, _u16p, _i64, _u16p, _i64, _f,
                            _NullableU16, _i64, _NullableU16, _i64, _f32p, _i64]),
}

_lib = None


def build() -> pathlib.Path:
    """Compiles liboracle.so with the committed Makefile (g++, no GPU needed)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def set_threads(n: int) -> None:
    lib().oracle_set_threads(n)


def max_threads() -> int:
    return lib().oracle_max_threads()


def hardware_concurrency() -> int:
    """std::thread::hardware_concurrency() of this host (hardware threads, not the affinity)."""
    return lib().oracle_hardware_concurrency()


# ---- conversions and generators ----------------------------------------------------------------
def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_f32_to_bf16(x.reshape(-1), out.reshape(-1), x.size)
    return out


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().oracle_bf16_to_f32(h.reshape(-1), out.reshape(-1), h.size)
    return out


def rand_uniform(n: int, seed: int, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    """kernels_test.cu rand_vec: mt19937_64(seed) + uniform_real_distribution<float>(lo, hi)."""
    out = np.empty(n, dtype=np.float32)
    lib().oracle_rand_uniform(out, n, seed, lo, hi)
    return out


def splitmix_uniform(n: int, seed: int, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    """sgemm_test.cu / bgemm_test.cu fill_random_kernel stream."""
    out = np.empty(n, dtype=np.float32)
    lib().oracle_splitmix_uniform(out, n, seed, lo, hi)
    return out


def normal(n: int, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().oracle_normal(out, n, seed, mean, std)
    return out


# ---- kernels ---------------------------------------------------------------------------------
def _c(x, dt=np.float32):
    return np.ascontiguousarray(x, dtype=dt)


def gelu_forward(x: np.ndarray) -> np.ndarray:
    if x.dtype == np.uint16:
        out = np.empty(x.shape, np.float32)
        lib().oracle_gelu_forward_bf16(_c(x, np.uint16).reshape(-1), out.reshape(-1), x.size)
        return out
    x = _c(x)
    out = np.empty_like(x)
    lib().oracle_gelu_forward_f32(x.reshape(-1), out.reshape(-1), x.size)
    return out


def gelu_backward(g: np.ndarray, x: np.ndarray) -> np.ndarray:
    if x.dtype == np.uint16:
        out = np.empty(x.shape, np.float32)
        lib().oracle_gelu_backward_bf16(_c(g, np.uint16).reshape(-1), _c(x, np.uint16).reshape(-1),
                                        out.reshape(-1), x.size)
        return out
    g, x = _c(g), _c(x)
    out = np.empty_like(x)
    lib().oracle_gelu_backward_f32(g.reshape(-1), x.reshape(-1), out.reshape(-1), x.size)
    return out


def gelu_backward_fd(g: np.ndarray, x: np.ndarray) -> np.ndarray:
    g, x = _c(g), _c(x)
    out = np.empty_like(x)
    lib().oracle_gelu_backward_fd_f32(g.reshape(-1), x.reshape(-1), out.reshape(-1), x.size)
    return out


def layer_norm_forward(x, gamma, beta, eps):
    x = _c(x)
    rows, cols = x.shape
    y = np.empty_like(x)
    mean = np.empty(rows, np.float32)
    rstd = np.empty(rows, np.float32)
    lib().oracle_layer_norm_forward(x, None if gamma is None else _c(gamma),
                                    None if beta is None else _c(beta), y, mean, rstd, rows, cols,
                                    eps)
    return y, mean, rstd


def ln_backward_input(dy, x, mean, rstd, gamma):
    x = _c(x)
    rows, cols = x.shape
    dx = np.empty_like(x)
    lib().oracle_ln_backward_input(_c(dy), x, _c(mean), _c(rstd),
                                   None if gamma is None else _c(gamma), dx, rows, cols)
    return dx


def ln_backward_gamma_beta(dy, x, mean, rstd):
    x = _c(x)
    rows, cols = x.shape
    dg = np.empty(cols, np.float32)
    db = np.empty(cols, np.float32)
    lib().oracle_ln_backward_gamma_beta(_c(dy), x, _c(mean), _c(rstd), dg, db, rows, cols)
    return dg, db


def sparse_ce_forward(logits, targets):
    logits = _c(logits)
    rows, vocab = logits.shape
    loss, mx, sm = (np.empty(rows, np.float32) for _ in range(3))
    lib().oracle_sparse_ce_forward(logits, _c(targets, np.int32), loss, mx, sm, rows, vocab)
    return loss, mx, sm


def sparse_ce_backward(logits, targets, mx, sm, scale=1.0, out=None):
    logits = _c(logits)
    rows, vocab = logits.shape
    grad = np.empty_like(logits) if out is None else out
    lib().oracle_sparse_ce_backward(logits, _c(targets, np.int32), _c(mx), _c(sm), grad, rows,
                                    vocab, scale)
    return grad


def adamw(p, g, m, v, lr, b1, b2, eps, wd, bc1, bc2):
    """Returns updated copies (p, m, v)."""
    p, m, v = _c(p).copy(), _c(m).copy(), _c(v).copy()
    lib().oracle_adamw(p.reshape(-1), _c(g).reshape(-1), m.reshape(-1), v.reshape(-1), p.size, lr,
                       b1, b2, eps, wd, bc1, bc2)
    return p, m, v


def adamw_(p, g, m, v, lr, b1, b2, eps, wd, bc1, bc2):
    """In-place form of adamw on contiguous float32 arrays (no copies)."""
    for a in (p, g, m, v):
        assert a.dtype == np.float32 and a.flags.c_contiguous
    lib().oracle_adamw(p.reshape(-1), g.reshape(-1), m.reshape(-1), v.reshape(-1), p.size, lr,
                       b1, b2, eps, wd, bc1, bc2)


def reduce_inner(src, nout, length, row_stride=None):
    out = np.empty(nout, np.float32)
    lib().oracle_reduce_inner(_c(src).reshape(-1), out, nout, length,
                              length if row_stride is None else row_stride)
    return out


def reduce_outer(src, nout, inner, outer_stride, row_stride, length):
    out = np.empty(nout, np.float32)
    lib().oracle_reduce_outer(_c(src).reshape(-1), out, nout, inner, outer_stride, row_stride,
                              length)
    return out


def reduce_selftest_input(n):
    out = np.empty(n, np.float32)
    lib().oracle_reduce_selftest_input(out, n)
    return out


def attn_forward(q, k, v, scale, causal, mask=None):
    """O, LSE of softmax attention; `mask` ([B, H, T, T] fp32 or None) is the reference's
    dropout mask, applied to the exp terms before the row sum."""
    q, k, v = _c(q), _c(k), _c(v)
    B, H, T, D = q.shape
    o = np.empty_like(q)
    lse = np.empty((B, H, T), np.float32)
    lib().oracle_attn_forward(q, k, v, B, H, T, D, scale, int(bool(causal)),
                              None if mask is None else _c(mask).reshape(-1), o, lse)
    return o, lse


def attn_precompute_D(do, o):
    do, o = _c(do), _c(o)
    D = np.empty(do.shape[:-1], np.float32)
    lib().oracle_attn_precompute_D(do.reshape(-1), o.reshape(-1), D.reshape(-1),
                                   do.size // do.shape[-1], do.shape[-1])
    return D


def attn_backward(q, k, v, o, do, lse, scale, causal):
    q, k, v, o, do, lse = (_c(a) for a in (q, k, v, o, do, lse))
    B, H, T, Dh = q.shape
    D = np.empty((B, H, T), np.float32)
    dq, dk, dv = np.empty_like(q), np.empty_like(k), np.empty_like(v)
    lib().oracle_attn_backward(q, k, v, o, do, lse, B, H, T, Dh, scale, int(bool(causal)), D, dq,
                               dk, dv)
    return D, dq, dk, dv


def sgemm(transA, transB, A, B, alpha=1.0, beta=0.0, C0=None, bias=None):
    """C = alpha op(A) op(B) + beta C0 + bias, row-major; A [M,K] or [K,M] (transA)."""
    A, B = _c(A), _c(B)
    M = A.shape[1] if transA else A.shape[0]
    K = A.shape[0] if transA else A.shape[1]
    N = B.shape[0] if transB else B.shape[1]
    C = np.empty((M, N), np.float32)
    lib().oracle_sgemm(int(transA), int(transB), M, N, K, alpha, A, A.shape[1], B, B.shape[1], beta,
                       None if C0 is None else _c(C0), N, None if bias is None else _c(bias), C, N)
    return C


def bgemm(transA, transB, A, B, alpha=1.0, beta=0.0, C0=None, bias=None):
    """bf16 (uint16) operands, fp32 result = alpha acc + beta C0 (+ beta bias). The bias
    element is chosen by its size: N per column, M per row, 1 scalar, M*N full."""
    A, B = _c(A, np.uint16), _c(B, np.uint16)
    M = A.shape[1] if transA else A.shape[0]
    K = A.shape[0] if transA else A.shape[1]
    N = B.shape[0] if transB else B.shape[1]
    C = np.empty((M, N), np.float32)
    lib().oracle_bgemm(int(transA), int(transB), M, N, K, alpha, A, A.shape[1], B, B.shape[1], beta,
                       None if C0 is None else _c(C0, np.uint16), N,
                       None if bias is None else _c(bias, np.uint16).reshape(-1),
                       0 if bias is None else int(np.asarray(bias).size), C, N)
    return C
