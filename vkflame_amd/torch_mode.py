"""PyTorch front end: aten matmuls on GPU tensors routed to the C ABI.

The reference's torch backend (torch_backend/mode.py:22-45,
torch_backend/ops.py:270-313) is a ``TorchDispatchMode`` whose handlers for
``aten.mm`` / ``aten.addmm`` / ``aten.linear`` stage fp16/int8 tensors into
Vulkan buffers and call ``vkflame_dispatch_linear``, adding the bias with a
separate torch op; float32 falls through to PyTorch.  Here the handlers pass
the tensors' device pointers straight to the library on torch's current
stream:

* fp16 ``mm`` / ``addmm`` / ``linear`` -> ``vkflame_dispatch_linear`` (fp16
  MFMA GEMM, fp32 accumulation, fp16 out).  A transposed view (``w.t()`` of a
  row-major weight) is passed as ``transB`` / ``transA`` instead of being
  copied; ``addmm`` with a full [M, N] input uses the GEMM's ``beta * C``
  epilogue, a bias vector is added by torch as in the reference;
* ``aten._int_mm`` (int8 x int8 -> int32) -> the exact int8 MFMA GEMM;
* ``Int8Linear``: the layer form of the reference's quantised checkpoints
  (``weight_int8`` int8 [N, K] + ``weight_scale`` fp16 [N], written by
  tools/quantise.py:35-43).  Its forward quantises the activations per token
  (``vkflame_quantize_rows_i8``) and runs ``vkflame_dispatch_linear_int8``
  (exact int32 products, then ``acc * a_scale * w_scale + bias`` in fp32,
  fp16 out) -- two library launches.

Anything else (CPU tensors, fp32 / bf16, batched or strided operands the
GEMM does not take) falls through to PyTorch unchanged, as in the
reference.  Unlike the reference, a library error is raised, not swallowed.
"""
from __future__ import annotations

import torch
from torch.utils._python_dispatch import TorchDispatchMode

from . import _lib as L
from . import ops

aten = torch.ops.aten


def _gpu_f16(*ts) -> bool:
    return all(t is not None and t.is_cuda and t.dtype == torch.float16 for t in ts)


def _as_op(t: torch.Tensor):
    """(tensor to pass, trans flag) for a 2-D operand the row-major GEMM takes
    without a copy: packed row-major (trans 0) or the transpose of a packed
    row-major tensor (trans 1); None otherwise."""
    if t.dim() != 2:
        return None
    if t.is_contiguous():
        return t, 0
    if t.t().is_contiguous():
        return t.t(), 1
    return None


class VkflameMode(TorchDispatchMode):
    """Routes the aten matmuls listed in the module docstring to the library.
    ``calls`` counts the routed calls per op name (a test and debugging aid)."""

    def __init__(self):
        super().__init__()
        self.calls: dict[str, int] = {}

    def __torch_dispatch__(self, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        handler = _HANDLERS.get(func)
        if handler is not None:
            out = handler(*args, **kwargs)
            if out is not NotImplemented:
                name = func.overloadpacket.__name__
                self.calls[name] = self.calls.get(name, 0) + 1
                return out
        return func(*args, **kwargs)


def _mm_f16(a: torch.Tensor, b: torch.Tensor, C=None, alpha=1.0, beta=0.0):
    """D[M, N] = alpha * a @ b (+ beta * C), fp16 in and out, or NotImplemented."""
    if not _gpu_f16(a, b) or a.dim() != 2 or b.dim() != 2 or a.shape[1] != b.shape[0]:
        return NotImplemented
    if a.device != b.device:
        return NotImplemented
    oa, ob = _as_op(a), _as_op(b)
    if oa is None or ob is None:
        return NotImplemented
    M, K = a.shape
    N = b.shape[1]
    if M == 0 or N == 0 or K == 0:
        return NotImplemented
    with torch.cuda.device(a.device):
        return ops.linear(oa[0], ob[0], M, N, K, L.DTYPE_FP16, transA=oa[1], transB=ob[1], C=C,
                          alpha=alpha, beta=beta)


def _mm(a, b):
    return _mm_f16(a, b)


def _addmm(bias, a, b, *, beta=1, alpha=1):
    if not _gpu_f16(bias):
        return NotImplemented
    M, N = a.shape[0], b.shape[1] if b.dim() == 2 else -1
    if bias.dim() == 2 and bias.shape == (M, N) and bias.is_contiguous():
        return _mm_f16(a, b, C=bias, alpha=float(alpha), beta=float(beta))
    out = _mm_f16(a, b, alpha=float(alpha))
    if out is NotImplemented:
        return out
    if beta != 0:
        out.add_(bias, alpha=beta)  # broadcast bias, as the reference's handler does
    return out


def _linear(x, weight, bias=None):
    if not _gpu_f16(x, weight) or weight.dim() != 2 or x.dim() < 1 or x.shape[-1] != weight.shape[1]:
        return NotImplemented
    if bias is not None and not _gpu_f16(bias):
        return NotImplemented
    x2 = x.reshape(-1, x.shape[-1])
    out = _mm_f16(x2, weight.t())  # weight [N, K] row-major: transB = 1, no copy
    if out is NotImplemented:
        return out
    if bias is not None:
        out.add_(bias)
    return out.reshape(*x.shape[:-1], weight.shape[0])


def _int_mm(a, b):
    if not (a.is_cuda and b.is_cuda and a.dtype == torch.int8 and b.dtype == torch.int8):
        return NotImplemented
    if a.dim() != 2 or b.dim() != 2 or a.shape[1] != b.shape[0]:
        return NotImplemented
    oa, ob = _as_op(a), _as_op(b)
    if oa is None or ob is None:
        return NotImplemented
    M, K = a.shape
    N = b.shape[1]
    if M == 0 or N == 0 or K == 0:
        return NotImplemented
    with torch.cuda.device(a.device):
        return ops.linear(oa[0], ob[0], M, N, K, L.DTYPE_INT8_INT32OUT, transA=oa[1], transB=ob[1])


_HANDLERS = {
    aten.mm.default: _mm,
    aten.addmm.default: _addmm,
    aten.linear.default: _linear,
    aten._int_mm.default: _int_mm,
}


def install() -> VkflameMode:
    """A mode instance to use as a context manager: ``with install(): ...``."""
    return VkflameMode()


# ---------------------------------------------------------------------------
# int8 weights (the reference's quantised checkpoint layout)
# ---------------------------------------------------------------------------

def quantise_weight(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(weight_int8 [N, K], weight_scale fp16 [N]) by the rule of
    tools/quantise.py:35-41: per output channel scale = max|w|/127 (>= 1e-8,
    in fp32), w_int8 = round(w / scale) clamped to +-127; the scale is stored
    as fp16.  On a GPU tensor this is one library launch
    (vkflame_quantize_rows_i8); on the CPU, torch ops with the same rule."""
    if w.is_cuda:
        q, s = ops.quantize_rows_i8(w.contiguous() if w.dtype in (torch.float16, torch.float32)
                                    else w.float().contiguous())
        return q, s.half()
    wf = w.detach().float()
    scale = (wf.abs().amax(dim=1) / 127.0).clamp(min=1e-8)
    q = (wf / scale.unsqueeze(1)).round().clamp(-127, 127).to(torch.int8)
    return q, scale.half()


class Int8Linear(torch.nn.Module):
    """nn.Linear with int8 per-output-channel weights: buffers ``weight_int8``
    [N, K] and ``weight_scale`` fp16 [N] (the reference's quantised
    checkpoint layout), optional fp16 ``bias``.  Forward on GPU tensors:
    activations quantised per token to int8 (scale max|row|/127), exact int8
    MFMA products, ``float(acc) * a_scale * w_scale + bias`` in fp32, fp16
    out (two library launches)."""

    def __init__(self, weight_int8: torch.Tensor, weight_scale: torch.Tensor, bias: torch.Tensor | None = None):
        super().__init__()
        assert weight_int8.dtype == torch.int8 and weight_int8.dim() == 2
        assert weight_scale.shape == (weight_int8.shape[0],)
        self.register_buffer("weight_int8", weight_int8.contiguous())
        self.register_buffer("weight_scale", weight_scale.to(torch.float16))
        self.register_buffer("bias", None if bias is None else bias.to(torch.float16))
        self.in_features = weight_int8.shape[1]
        self.out_features = weight_int8.shape[0]

    @classmethod
    def from_linear(cls, lin: torch.nn.Linear) -> "Int8Linear":
        q, s = quantise_weight(lin.weight.detach())
        b = None if lin.bias is None else lin.bias.detach()
        return cls(q, s, b)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if not x.is_cuda:
            raise L.VkflameError("Int8Linear runs on GPU tensors only")
        x2 = x.reshape(-1, self.in_features)
        if x2.dtype not in (torch.float16, torch.float32):
            x2 = x2.float()
        x2 = x2.contiguous()
        a_q, a_s = ops.quantize_rows_i8(x2)
        w_s = self.weight_scale.float()
        out = ops.linear_int8(a_q, a_s, self.weight_int8, w_s, bias=self.bias, out_dtype=torch.float16)
        return out.reshape(*x.shape[:-1], self.out_features)


def quantise_linears_(model: torch.nn.Module) -> int:
    """Replace every nn.Linear of ``model`` by an Int8Linear (in place, the
    layer walk of tools/quantise.py:29-48); returns how many were replaced."""
    n = 0
    for name, mod in list(model.named_modules()):
        for cname, child in list(mod.named_children()):
            if isinstance(child, torch.nn.Linear):
                setattr(mod, cname, Int8Linear.from_linear(child))
                n += 1
    return n
