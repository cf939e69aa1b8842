"""Host-side mirror of the reference kernel surface over torch device tensors.

Each function wraps one C-ABI entry point of ``include/hk.h`` and keeps the argument meaning of
the reference kernel it replaces (cited per function). Tensors must be HIP device tensors;
outputs may be passed in (as the reference caller does) or are allocated here. Launches go on
torch's current stream. Errors from the library raise ``HKError``; nothing falls back to a CPU
path.
"""
from __future__ import annotations

import ctypes
from typing import Sequence

import torch

from ._lib import HKError, call, lib  # noqa: F401

__all__ = [
    "HKError", "gelu_forward", "gelu_backward", "layer_norm_forward", "ln_backward_input",
    "ln_backward_gamma_beta", "layer_norm_backward", "sparse_ce_forward", "sparse_ce_backward",
    "AdamLaunchMetadata", "multi_tensor_adam", "AdamPlan", "ReductionLayout",
    "unified_reduce_sum", "reduce_generic", "REDUCE_INNER", "REDUCE_OUTER", "REDUCE_GENERIC",
]


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _dev(*ts: torch.Tensor | None) -> None:
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("hyperkernels_amd kernels take device tensors only")
        if not t.is_contiguous():
            raise ValueError("hyperkernels_amd kernels take contiguous tensors")


# ----------------------------------------------------------------------------------------------
# GELU: gelu_forward_sm89_kernel<T> (kernels/gelu/gelu_forward_sm89_kernel.cu:35-37),
#       gelu_backward_sm89_kernel<T> (kernels/gelu/gelu_backward_sm89_kernel.cu:44-47)
# ----------------------------------------------------------------------------------------------
# storage dtype -> entry-point suffix (the reference's float / __nv_bfloat16 / __half
# instantiations of the GELU and LayerNorm kernels)
_SUFFIX = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}


def gelu_forward(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    _dev(x, out)
    out = torch.empty_like(x) if out is None else out
    if x.dtype not in _SUFFIX or out.dtype != x.dtype or out.numel() != x.numel():
        raise ValueError("gelu_forward: fp32, bf16 or fp16 tensors of equal size")
    call(f"hk_gelu_forward_{_SUFFIX[x.dtype]}", _ptr(x), _ptr(out), x.numel(), _stream())
    return out


def gelu_backward(grad: torch.Tensor, x: torch.Tensor,
                  grad_in: torch.Tensor | None = None) -> torch.Tensor:
    _dev(grad, x, grad_in)
    grad_in = torch.empty_like(x) if grad_in is None else grad_in
    if x.dtype not in _SUFFIX or not (grad.dtype == x.dtype == grad_in.dtype) or not (
            grad.numel() == x.numel() == grad_in.numel()):
        raise ValueError("gelu_backward: fp32, bf16 or fp16 tensors of equal size")
    call(f"hk_gelu_backward_{_SUFFIX[x.dtype]}", _ptr(grad), _ptr(x), _ptr(grad_in),
         x.numel(), _stream())
    return grad_in


# ----------------------------------------------------------------------------------------------
# LayerNorm (kernels/layernorm/*.cu)
# ----------------------------------------------------------------------------------------------
def _rows_cols(x: torch.Tensor) -> tuple[int, int]:
    if x.dim() < 1:
        raise ValueError("layer norm needs at least one dimension")
    cols = x.shape[-1]
    return (x.numel() // cols if cols else 0), cols


def _ln_suffix(data, stats) -> str:
    """Entry-point suffix for LayerNorm: `data` tensors (x, gamma, beta, y, dy, dx) share one
    storage dtype; `stats` tensors (mean, rstd, grad_gamma, grad_beta) are fp32."""
    dt = data[0].dtype
    if dt not in _SUFFIX or any(t is not None and t.dtype != dt for t in data):
        raise ValueError("layer norm: x, gamma, beta, y, dy and dx must share one dtype "
                         "(fp32, bf16 or fp16)")
    if any(t is not None and t.dtype != torch.float32 for t in stats):
        raise ValueError("layer norm: mean, rstd, grad_gamma and grad_beta are fp32")
    return _SUFFIX[dt]


def layer_norm_forward(x, gamma=None, beta=None, eps: float = 1e-5, y=None, mean=None, rstd=None):
    """layer_norm_forward_sm89_kernel<T,float> (layer_norm_forward_sm89_kernel.cu:27-32).

    Returns (y, mean, rstd); mean/rstd are [rows] fp32."""
    _dev(x, gamma, beta, y, mean, rstd)
    rows, cols = _rows_cols(x)
    y = torch.empty_like(x) if y is None else y
    mean = torch.empty(rows, device=x.device, dtype=torch.float32) if mean is None else mean
    rstd = torch.empty(rows, device=x.device, dtype=torch.float32) if rstd is None else rstd
    sfx = _ln_suffix([x, gamma, beta, y], [mean, rstd])
    call(f"hk_layer_norm_forward_{sfx}", _ptr(x), _ptr(gamma), _ptr(beta), _ptr(y), _ptr(mean),
         _ptr(rstd), rows, cols, ctypes.c_float(eps), _stream())
    return y, mean, rstd


def ln_backward_input(grad_y, x, mean, rstd, gamma=None, grad_x=None):
    """OwnTensor::cuda::ln_backward_input_sm89_kernel<T> (ln_backward_input_sm89_kernel.cu:33-38)."""
    _dev(grad_y, x, mean, rstd, gamma, grad_x)
    rows, cols = _rows_cols(x)
    grad_x = torch.empty_like(x) if grad_x is None else grad_x
    sfx = _ln_suffix([x, grad_y, gamma, grad_x], [mean, rstd])
    call(f"hk_ln_backward_input_{sfx}", _ptr(grad_y), _ptr(x), _ptr(mean), _ptr(rstd),
         _ptr(gamma), _ptr(grad_x), rows, cols, _stream())
    return grad_x


def ln_backward_gamma_beta(grad_y, x, mean, rstd, grad_gamma, grad_beta):
    """ln_backward_gamma_beta_sm89_kernel<T> (ln_backward_gamma_beta_sm89_kernel.cu:15-21).

    ADDS the column sums into grad_gamma / grad_beta (the reference's atomics into caller-zeroed
    buffers), in a fixed order."""
    _dev(grad_y, x, mean, rstd, grad_gamma, grad_beta)
    rows, cols = _rows_cols(x)
    sfx = _ln_suffix([x, grad_y], [mean, rstd, grad_gamma, grad_beta])
    call(f"hk_ln_backward_gamma_beta_{sfx}", _ptr(grad_y), _ptr(x), _ptr(mean), _ptr(rstd),
         _ptr(grad_gamma), _ptr(grad_beta), rows, cols, _stream())
    return grad_gamma, grad_beta


def layer_norm_backward(grad_y, x, mean, rstd, gamma, grad_gamma, grad_beta, grad_x=None):
    """Fused backward: grad_x written, grad_gamma / grad_beta added into, one pass over dy, x."""
    _dev(grad_y, x, mean, rstd, gamma, grad_gamma, grad_beta, grad_x)
    rows, cols = _rows_cols(x)
    grad_x = torch.empty_like(x) if grad_x is None else grad_x
    sfx = _ln_suffix([x, grad_y, gamma, grad_x], [mean, rstd, grad_gamma, grad_beta])
    call(f"hk_layer_norm_backward_{sfx}", _ptr(grad_y), _ptr(x), _ptr(mean), _ptr(rstd),
         _ptr(gamma), _ptr(grad_x), _ptr(grad_gamma), _ptr(grad_beta), rows, cols, _stream())
    return grad_x


# ----------------------------------------------------------------------------------------------
# Sparse cross-entropy (kernels/loss/*.cu)
# ----------------------------------------------------------------------------------------------
# target dtype -> entry-point suffix: the reference's <float, int32_t | int64_t | uint16_t>
# instantiations (sparse_ce_forward_...cu:108-113; sparseCENormalize_from_stats.cu:52-60)
_CE_INDEX = {torch.int32: "i32", torch.int64: "i64", torch.uint16: "u16"}


def sparse_ce_forward(logits, targets, losses=None, saved_max=None, saved_sum=None):
    """sparse_ce_forward_kernel_vec_save_stats<float,TIdx> (sparse_ce_forward_...cu:14-23).

    Returns (losses, saved_max, saved_sum), each [rows] fp32."""
    _dev(logits, targets, losses, saved_max, saved_sum)
    if logits.dtype != torch.float32 or targets.dtype not in _CE_INDEX or logits.dim() != 2:
        raise ValueError("sparse_ce_forward: fp32 logits [rows, vocab] and int32/int64/uint16 "
                         "targets")
    rows, vocab = logits.shape
    mk = lambda: torch.empty(rows, device=logits.device, dtype=torch.float32)  # noqa: E731
    losses = mk() if losses is None else losses
    saved_max = mk() if saved_max is None else saved_max
    saved_sum = mk() if saved_sum is None else saved_sum
    call("hk_sparse_ce_forward_f32_" + _CE_INDEX[targets.dtype], _ptr(logits), _ptr(targets),
         _ptr(losses), _ptr(saved_max), _ptr(saved_sum), rows, vocab, _stream())
    return losses, saved_max, saved_sum


def sparse_ce_backward(logits, targets, saved_max, saved_sum, grad_output=None,
                       host_scale: float = 1.0, grad=None):
    """sparseCENormalize_from_stats<float,TIdx> (sparseCENormalize_from_stats.cu:7-17).

    grad_output is a 1-element device tensor (or None for 1.0)."""
    _dev(logits, targets, saved_max, saved_sum, grad_output, grad)
    if logits.dtype != torch.float32 or targets.dtype not in _CE_INDEX or logits.dim() != 2:
        raise ValueError("sparse_ce_backward: fp32 logits [rows, vocab] and int32/int64/uint16 "
                         "targets")
    rows, vocab = logits.shape
    grad = torch.empty_like(logits) if grad is None else grad
    call("hk_sparse_ce_backward_f32_" + _CE_INDEX[targets.dtype], _ptr(logits), _ptr(targets),
         _ptr(grad), _ptr(saved_max), _ptr(saved_sum), rows, vocab, _ptr(grad_output),
         ctypes.c_float(host_scale), _stream())
    return grad


# ----------------------------------------------------------------------------------------------
# Multi-tensor AdamW (kernels/optimizer/multi_tensor_adam_sm89_kernel.cu)
# ----------------------------------------------------------------------------------------------
ADAM_CHUNK_SIZE = 32768
ADAM_MAX_BLOCKS = 320
ADAM_MAX_TENSORS = 48


class AdamLaunchMetadata(ctypes.Structure):
    """Byte-for-byte the reference's AdamLaunchMetadata (multi_tensor_adam_sm89_kernel.cu:13-21)."""

    _fields_ = [
        ("params", ctypes.c_void_p * ADAM_MAX_TENSORS),
        ("grads", ctypes.c_void_p * ADAM_MAX_TENSORS),
        ("ms", ctypes.c_void_p * ADAM_MAX_TENSORS),
        ("vs", ctypes.c_void_p * ADAM_MAX_TENSORS),
        ("sizes", ctypes.c_int64 * ADAM_MAX_TENSORS),
        ("block_to_tensor", ctypes.c_ubyte * ADAM_MAX_BLOCKS),
        ("block_to_chunk", ctypes.c_int * ADAM_MAX_BLOCKS),
    ]


def multi_tensor_adam(params: Sequence[torch.Tensor], grads, ms, vs, lr, beta1, beta2, eps,
                      weight_decay, bias_correction1, bias_correction2) -> None:
    """One launch of the reference ABI: <= 48 tensors, <= 320 chunks of 32768 elements."""
    if not (len(params) == len(grads) == len(ms) == len(vs)) or len(params) > ADAM_MAX_TENSORS:
        raise ValueError("multi_tensor_adam: at most 48 tensors, equal list lengths")
    meta = AdamLaunchMetadata()
    blk = 0
    for t, (p, g, m, v) in enumerate(zip(params, grads, ms, vs)):
        _dev(p, g, m, v)
        meta.params[t], meta.grads[t] = p.data_ptr(), g.data_ptr()
        meta.ms[t], meta.vs[t] = m.data_ptr(), v.data_ptr()
        meta.sizes[t] = p.numel()
        for c in range((p.numel() + ADAM_CHUNK_SIZE - 1) // ADAM_CHUNK_SIZE):
            if blk >= ADAM_MAX_BLOCKS:
                raise ValueError("multi_tensor_adam: more than 320 chunks")
            meta.block_to_tensor[blk], meta.block_to_chunk[blk] = t, c
            blk += 1
    f = ctypes.c_float
    call("hk_multi_tensor_adam", ctypes.byref(meta), blk, f(lr), f(beta1), f(beta2), f(eps),
         f(weight_decay), f(bias_correction1), f(bias_correction2), _stream())


class AdamPlan:
    """Device-resident tensor/chunk table: one launch per step over any number of tensors."""

    def __init__(self, params, grads, ms, vs):
        n = len(params)
        if not (n == len(grads) == len(ms) == len(vs)):
            raise ValueError("AdamPlan: equal list lengths")
        for ts in zip(params, grads, ms, vs):
            _dev(*ts)
            if len({t.numel() for t in ts}) != 1 or any(t.dtype != torch.float32 for t in ts):
                raise ValueError("AdamPlan: p, g, m, v of one tensor are fp32 of equal size")
        arr = lambda ts: (ctypes.c_void_p * n)(*[t.data_ptr() for t in ts])  # noqa: E731
        self._keep = (list(params), list(grads), list(ms), list(vs))
        sizes = (ctypes.c_int64 * n)(*[p.numel() for p in params])
        self._plan = ctypes.c_void_p()
        call("hk_adam_plan_create", n, arr(params), arr(grads), arr(ms), arr(vs), sizes,
             ctypes.byref(self._plan))
        self.num_chunks = lib().hk_adam_plan_num_chunks(self._plan)

    def step(self, lr, beta1, beta2, eps, weight_decay, bias_correction1, bias_correction2):
        f = ctypes.c_float
        call("hk_adam_plan_step", self._plan, f(lr), f(beta1), f(beta2), f(eps),
             f(weight_decay), f(bias_correction1), f(bias_correction2), _stream())

    def close(self):
        if self._plan:
            call("hk_adam_plan_destroy", self._plan)
            self._plan = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ----------------------------------------------------------------------------------------------
# Attention (kernels/attention/*.cu), fp32, head_dim 64, tensors [B, nh, T, d] (any strides
# with a unit last dimension), LSE / D [B, nh, T]
# ----------------------------------------------------------------------------------------------
_I64 = ctypes.c_int64


class AttnFwdParams(ctypes.Structure):
    """MemEfficientFwdParams (fused_attn_forward_kernel_tc_sm89.cu:8-29), field for field."""

    _fields_ = [("Q", ctypes.c_void_p), ("K", ctypes.c_void_p), ("V", ctypes.c_void_p),
                ("O", ctypes.c_void_p), ("LSE", ctypes.c_void_p), ("B", ctypes.c_int),
                ("nh", ctypes.c_int), ("T", _I64), ("scale", ctypes.c_float),
                ("is_causal", ctypes.c_bool), ("dropout_p", ctypes.c_float),
                ("dropout_mask", ctypes.c_void_p)] + [
        (f"{t}_stride{s}", _I64) for t in ("q", "k", "v", "o") for s in ("B", "M", "H")] + [
        ("lse_strideB", _I64), ("lse_strideH", _I64)]


class AttnBwdParams(ctypes.Structure):
    """MemEfficientBwdParams (mem_efficient_bwd_precompute_D_sm89.cu:7-33), field for field."""

    _fields_ = [(n, ctypes.c_void_p) for n in ("Q", "K", "V", "O", "dO", "LSE", "D", "dQ", "dK",
                                               "dV")] + [
        ("B", ctypes.c_int), ("nh", ctypes.c_int), ("T", ctypes.c_int), ("scale", ctypes.c_float),
        ("is_causal", ctypes.c_bool)] + [
        (f"{t}_stride{s}", _I64) for t in ("q", "k", "v", "o", "do", "dq", "dk", "dv")
        for s in ("B", "M", "H")] + [
        ("lse_strideB", _I64), ("lse_strideH", _I64), ("d_strideB", _I64), ("d_strideH", _I64)]


def _set_strides(params, prefix: str, t: torch.Tensor) -> None:
    if t.dim() != 4 or t.stride(-1) != 1:
        raise ValueError("attention tensors are [B, nh, T, d] with a unit last-dim stride")
    setattr(params, f"{prefix}_strideB", t.stride(0))
    setattr(params, f"{prefix}_strideH", t.stride(1))
    setattr(params, f"{prefix}_strideM", t.stride(2))


def fused_attn_forward(q, k, v, causal: bool, scale: float | None = None, o=None, lse=None,
                       dropout_p: float = 0.0, dropout_mask=None):
    """fused_attn_forward_kernel_tc_sm89<64,64,64,1>: returns (O, LSE).

    With dropout_p > 0 and a dropout_mask (contiguous fp32 [B, nh, T, T], the factor of each
    score, e.g. 0 or 1 / (1 - p)), the exp terms are multiplied by the mask and normalised by
    their post-dropout sum, as the reference kernel does (fused_attn_forward...:316-334)."""
    for t in (q, k, v):
        if not t.is_cuda or t.dtype != torch.float32:
            raise ValueError("fused_attn_forward: fp32 device tensors")
    B, H, T, D = q.shape
    if dropout_mask is not None and (
            not dropout_mask.is_cuda or dropout_mask.dtype != torch.float32
            or tuple(dropout_mask.shape) != (B, H, T, T) or not dropout_mask.is_contiguous()):
        raise ValueError("fused_attn_forward: dropout_mask is a contiguous fp32 [B, nh, T, T] "
                         "device tensor")
    scale = D ** -0.5 if scale is None else scale
    o = torch.empty_like(q) if o is None else o
    lse = torch.empty(B, H, T, device=q.device, dtype=torch.float32) if lse is None else lse
    p = AttnFwdParams()
    p.Q, p.K, p.V, p.O, p.LSE = (t.data_ptr() for t in (q, k, v, o, lse))
    p.B, p.nh, p.T, p.scale, p.is_causal = B, H, T, scale, bool(causal)
    p.dropout_p = dropout_p
    p.dropout_mask = None if dropout_mask is None else dropout_mask.data_ptr()
    for name, t in (("q", q), ("k", k), ("v", v), ("o", o)):
        _set_strides(p, name, t)
    p.lse_strideB, p.lse_strideH = lse.stride(0), lse.stride(1)
    call("hk_fused_attn_forward", ctypes.byref(p), D, _stream())
    return o, lse


def _bwd_params(q, k, v, o, do, lse, D, dq, dk, dv, causal, scale):
    B, H, T, _ = q.shape
    p = AttnBwdParams()
    p.Q, p.K, p.V, p.O, p.dO, p.LSE, p.D, p.dQ, p.dK, p.dV = (
        None if t is None else t.data_ptr() for t in (q, k, v, o, do, lse, D, dq, dk, dv))
    p.B, p.nh, p.T, p.scale, p.is_causal = B, H, T, scale, bool(causal)
    for name, t in (("q", q), ("k", k), ("v", v), ("o", o), ("do", do), ("dq", dq), ("dk", dk),
                    ("dv", dv)):
        if t is not None:
            _set_strides(p, name, t)
    if lse is not None:
        p.lse_strideB, p.lse_strideH = lse.stride(0), lse.stride(1)
    p.d_strideB, p.d_strideH = D.stride(0), D.stride(1)
    return p


def attn_bwd_precompute_D(do, o, D=None):
    """mem_efficient_bwd_precompute_D_sm89<HD>: D = rowsum(dO * O), [B, nh, T]."""
    B, H, T, Dh = o.shape
    D = torch.empty(B, H, T, device=o.device, dtype=torch.float32) if D is None else D
    p = _bwd_params(o, None, None, o, do, None, D, None, None, None, False, 1.0)
    p.Q = None
    call("hk_attn_bwd_precompute_D", ctypes.byref(p), Dh, _stream())
    return D


def attn_backward(q, k, v, do, lse, D, causal: bool, scale: float | None = None, dq=None, dk=None,
                  dv=None, o=None):
    """OwnTensor::mem_efficient_bwd_unified_kernel_exp12<64, Causal>: returns (dQ, dK, dV).

    dK and dV are written; dQ is ADDED into (zeroed here when not passed in), as in the
    reference where the caller zeroes dQ before the launch."""
    B, H, T, Dh = q.shape
    scale = Dh ** -0.5 if scale is None else scale
    dq = torch.zeros_like(q) if dq is None else dq
    dk = torch.empty_like(k) if dk is None else dk
    dv = torch.empty_like(v) if dv is None else dv
    p = _bwd_params(q, k, v, o, do, lse, D, dq, dk, dv, causal, scale)
    call("hk_attn_backward", ctypes.byref(p), Dh, _stream())
    return dq, dk, dv


# ----------------------------------------------------------------------------------------------
# Unified reduce (kernels/reduction/unified_reduce_standalone.cu)
# ----------------------------------------------------------------------------------------------
REDUCE_INNER, REDUCE_OUTER, REDUCE_GENERIC = 0, 1, 2


class ReductionLayout(ctypes.Structure):
    """detail::ReductionLayout (unified_reduce_standalone.cu:46-56), path as int32."""

    _fields_ = [
        ("path", ctypes.c_int32),
        ("num_outputs", ctypes.c_int64),
        ("reduced_count", ctypes.c_int64),
        ("input_outer_stride", ctypes.c_int64),
        ("inner_count", ctypes.c_int64),
        ("input_row_stride", ctypes.c_int64),
    ]


def unified_reduce_sum(src: torch.Tensor, layout: ReductionLayout,
                       dst: torch.Tensor | None = None) -> torch.Tensor:
    _dev(src, dst)
    dst = torch.empty(layout.num_outputs, device=src.device, dtype=torch.float32) if dst is None else dst
    call("hk_unified_reduce_sum_f32", ctypes.byref(layout), _ptr(src), _ptr(dst), _stream())
    return dst


def reduce_generic(src: torch.Tensor, out_sizes, out_strides, red_sizes, red_strides,
                   dst: torch.Tensor | None = None) -> torch.Tensor:
    """Sum with explicit strided offset maps (the reference's OffsetCalculator pair)."""
    _dev(dst)
    if not src.is_cuda:
        raise ValueError("reduce_generic: device tensor")
    nout = 1
    for s in out_sizes:
        nout *= s
    dst = torch.empty(nout, device=src.device, dtype=torch.float32) if dst is None else dst
    a = lambda xs: (ctypes.c_int64 * max(len(xs), 1))(*xs)  # noqa: E731
    call("hk_reduce_generic_f32", _ptr(src), _ptr(dst), len(out_sizes), a(out_sizes),
         a(out_strides), len(red_sizes), a(red_sizes), a(red_strides), _stream())
    return dst
