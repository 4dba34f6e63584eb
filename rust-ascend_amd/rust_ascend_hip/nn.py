"""Autograd entry points mirroring the reference's `rust_ascend::nn` functions on
`Autodiff<Ascend>` (src/nn.rs, src/nn/{attention,rotary}.rs), with torch.autograd standing in
for RUDA's autodiff graph. Saved state matches the reference's Backward nodes:

* linear_bf16_fp32 / matmul_bf16_fp32 save the BF16 snapshots of both operands
  (src/nn.rs:375-453), and their backward rounds dY to BF16 before the two GEMMs; the padded
  forms save the zero-padded snapshots and the original shapes (src/nn/padded.rs:29-57);
* rms_norm saves (x, w, rstd) and the backward reuses rstd (src/nn.rs:203-232);
* rotary/rotary_prefix save nothing but the fixed tables (src/nn/rotary.rs:32-105);
* the fused attention saves (q, k, v, o, lse) instead of the materialized score,
  mask and probability tensors of the composed reference (src/nn/attention.rs:10-80); the
  materialized (additive-mask) attention saves (q, k, v, mask) and recomputes the probabilities.
"""
from __future__ import annotations

import torch

from . import _lib
from ._lib import HkError
from .runtime import HipRuntime, LossReduction, RotaryLayout, Transpose


class _LinearBf16Fp32(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w):
        y, xb, wb = HipRuntime.linear_bf16_fp32(x.contiguous(), w.contiguous())
        ctx.save_for_backward(xb, wb)
        return y

    @staticmethod
    def backward(ctx, dy):
        xb, wb = ctx.saved_tensors
        dx, dw = HipRuntime.linear_bf16_fp32_backward(xb, wb, dy.contiguous().float())
        return dx, dw


def linear_bf16_fp32(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """Y = bf16(X) bf16(W)^T with F32 storage. Reference: nn::linear_bf16_fp32 (src/nn.rs:80-88)."""
    return _LinearBf16Fp32.apply(x, w)


class _MatmulBf16Fp32(torch.autograd.Function):
    @staticmethod
    def forward(ctx, a, b, ta, tb):
        out, ab, bb = HipRuntime.gemm_bf16_fp32(a.contiguous(), b.contiguous(), ta, tb)
        ctx.save_for_backward(ab, bb)
        ctx.ta, ctx.tb = ta, tb
        return out

    @staticmethod
    def backward(ctx, dy):
        ab, bb = ctx.saved_tensors
        da, db = HipRuntime.gemm_bf16_fp32_backward(ab, bb, dy.contiguous().float(), ctx.ta, ctx.tb)
        return da, db, None, None


def matmul_bf16_fp32(a, b, ta=Transpose.No, tb=Transpose.No) -> torch.Tensor:
    """op(A) op(B) with BF16 compute and F32 storage. Reference: nn::matmul_bf16_fp32 (src/nn.rs:70-78)."""
    return _MatmulBf16Fp32.apply(a, b, Transpose(ta), Transpose(tb))


class _FloatMatmul(torch.autograd.Function):
    @staticmethod
    def forward(ctx, a, b):
        a, b = a.contiguous(), b.contiguous()
        ctx.save_for_backward(a, b)
        return HipRuntime.tensor_matmul(a, b)

    @staticmethod
    def backward(ctx, dy):
        a, b = ctx.saved_tensors
        return HipRuntime.tensor_matmul_backward(a, b, dy.contiguous().to(a.dtype))


def float_matmul(a, b) -> torch.Tensor:
    """A @ B in the inputs' own dtype (F32, F16, BF16), batch dims broadcast; the backend op
    RudaAscend::float_matmul (src/backend.rs:692-703) with its autodiff (dY B^T, A^T dY, summed
    over broadcast batch dims)."""
    return _FloatMatmul.apply(a, b)


class _SwapLast(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x):
        return HipRuntime.swap_last_dims(x.contiguous())

    @staticmethod
    def backward(ctx, dy):
        return HipRuntime.swap_last_dims(dy.contiguous())


class _AttentionScores(torch.autograd.Function):
    @staticmethod
    def forward(ctx, s, bias, mask, scale, softcap, causal):
        s = s.contiguous()
        bias = None if bias is None else bias.contiguous()
        mask = None if mask is None else mask.contiguous()
        ctx.save_for_backward(s, mask)
        ctx.args = (scale, softcap, causal, None if bias is None else tuple(bias.shape))
        return HipRuntime.attention_scores(s, scale, softcap, bias, mask, causal)

    @staticmethod
    def backward(ctx, dout):
        s, mask = ctx.saved_tensors
        scale, softcap, causal, bias_shape = ctx.args
        need_bias = bias_shape is not None and ctx.needs_input_grad[1]
        ds, dbias = HipRuntime.attention_scores_backward(s, dout.contiguous().float(), scale, softcap, mask, causal,
                                                         bias_shape if need_bias else None)
        return ds, dbias, None, None, None, None


def module_attention(query, key, value, mask=None, attn_bias=None, scale=None, softcap=None, is_causal=False):
    """RudaAscend's ModuleOps::attention (src/backend.rs:1323-1333): the tensor library's fallback
    composed from the backend's own ops, here libhk.so's -- scores = Q swap(K) * scale (scale
    defaults to 1/sqrt(head width)), softcap c tanh(s/c), + attn_bias, -inf where is_causal (key >
    query) or mask (True = masked) excludes a key, softmax over the keys, then P V. Q [B, H, Sq, D],
    K [B, H, Sk, D], V [B, H, Sk, Dv], F32; mask (bool) and attn_bias (F32) [B, H, Sq, Sk] or
    broadcast along dims of size 1. Gradients flow to Q, K, V and the bias."""
    for name, t in (("query", query), ("key", key), ("value", value)):
        if t.dtype != torch.float32 or t.dim() != 4:
            raise HkError(_lib.INVALID_ARGUMENT, f"module attention takes F32 rank-4 tensors ({name})")
    if scale is None:
        scale = 1.0 / float(query.shape[-1]) ** 0.5
    scores = float_matmul(query, _SwapLast.apply(key))
    scores = _AttentionScores.apply(scores, attn_bias, mask, float(scale), float(softcap or 0.0), bool(is_causal))
    return float_matmul(softmax(scores), value)


class _MatmulPaddedBf16Fp32(torch.autograd.Function):
    @staticmethod
    def forward(ctx, a, b, ta, tb):
        out, ap, bp = HipRuntime.gemm_padded_bf16_fp32(a.contiguous(), b.contiguous(), ta, tb)
        ctx.save_for_backward(ap, bp)
        ctx.shapes = (tuple(a.shape), tuple(b.shape))
        ctx.ta, ctx.tb = ta, tb
        return out

    @staticmethod
    def backward(ctx, dy):
        ap, bp = ctx.saved_tensors
        da, db = HipRuntime.gemm_padded_bf16_fp32_backward(ap, bp, dy.contiguous().float(), ctx.shapes[0],
                                                           ctx.shapes[1], ctx.ta, ctx.tb)
        return da, db, None, None


def matmul_padded_bf16_fp32(a, b, ta=Transpose.No, tb=Transpose.No) -> torch.Tensor:
    """op(A) op(B) for any positive M/N/K, BF16 compute with on-device zero padding and an F32
    crop. Saves the padded BF16 snapshots and the original shapes. Reference:
    nn::matmul_padded_bf16_fp32 and PaddedMatmulBackward (src/nn/padded.rs:16-57)."""
    return _MatmulPaddedBf16Fp32.apply(a, b, Transpose(ta), Transpose(tb))


def linear_padded_bf16_fp32(x, w) -> torch.Tensor:
    """X[M,K] W[N,K]^T with explicit padding. Reference: nn::linear_padded_bf16_fp32 (src/nn/padded.rs:22-25)."""
    return matmul_padded_bf16_fp32(x, w, Transpose.No, Transpose.Yes)


class _LinearFrozen(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight):
        ctx.save_for_backward(weight)  # the fixed BF16 weight itself (frozen.rs:51-70)
        ctx.x_shape = tuple(x.shape)
        return HipRuntime.linear_frozen_bf16_fp32(x, weight)

    @staticmethod
    def backward(ctx, dy):
        (weight,) = ctx.saved_tensors
        return HipRuntime.linear_frozen_bf16_fp32_backward(ctx.x_shape, weight, dy.contiguous().float()), None


def linear_frozen_bf16_fp32(x, weight) -> torch.Tensor:
    """F32 X[M,K] and a fixed BF16 W[N,K] (aligned to 16): input-only differentiation, the weight
    never receives a gradient. Reference: nn::linear_frozen_bf16_fp32 (src/nn/frozen.rs:44-70)."""
    return _LinearFrozen.apply(x.contiguous(), weight.contiguous())


class _LinearFrozenPadded(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight):
        y, wp = HipRuntime.linear_frozen_padded_bf16_fp32(x.contiguous(), weight.contiguous())
        ctx.save_for_backward(wp)
        ctx.x_shape = tuple(x.shape)
        return y

    @staticmethod
    def backward(ctx, dy):
        (wp,) = ctx.saved_tensors
        return HipRuntime.linear_frozen_padded_bf16_fp32_backward(wp, dy.contiguous().float(), ctx.x_shape), None


def linear_frozen_padded_bf16_fp32(x, weight) -> torch.Tensor:
    """F32 X and a fixed BF16 W: input-only differentiation with logical tails (the weight never
    receives a gradient). Reference: nn::linear_frozen_padded_bf16_fp32 (src/nn/padded.rs:58-100)."""
    return _LinearFrozenPadded.apply(x, weight)


class _LinearBf16(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w):
        ctx.save_for_backward(x, w)
        return HipRuntime.gemm(x, w, Transpose.No, Transpose.Yes, torch.bfloat16)

    @staticmethod
    def backward(ctx, dy):
        x, w = ctx.saved_tensors
        dx, dw = HipRuntime.linear_nt_backward(x, w, dy.contiguous().to(torch.bfloat16))
        return dx, dw.to(w.dtype)


def linear_bf16(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """BF16 Y = X W^T with F32 accumulation (DeepGemm dense NT); backward through
    AscendRuntime::linear_nt_backward semantics (BF16 dX, F32 dW cast to W's dtype)."""
    return _LinearBf16.apply(x.contiguous(), w.contiguous())


class _RmsNorm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, eps):
        y, rstd = HipRuntime.rms_norm(x, w, eps)
        ctx.save_for_backward(x, w, rstd)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, w, rstd = ctx.saved_tensors
        dx, dw = HipRuntime.rms_norm_backward(x, w, dy.contiguous().to(x.dtype), rstd)
        return dx, dw, None


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """Reference: nn::rms_norm (src/nn.rs:165-174)."""
    return _RmsNorm.apply(x.contiguous(), w.contiguous(), float(eps))


class _Softmax(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, logarithmic):
        y = HipRuntime.log_softmax(x) if logarithmic else HipRuntime.softmax(x)
        ctx.save_for_backward(y)  # the backward needs only the output
        ctx.logarithmic = logarithmic
        return y

    @staticmethod
    def backward(ctx, dy):
        (y,) = ctx.saved_tensors
        dy = dy.contiguous().to(y.dtype)
        dx = HipRuntime.log_softmax_backward(y, dy) if ctx.logarithmic else HipRuntime.softmax_backward(y, dy)
        return dx, None


def softmax(x: torch.Tensor) -> torch.Tensor:
    """Last-axis softmax of an F32 tensor. Reference: nn::softmax / SoftmaxBackward (src/nn.rs:141-159, 234-278)."""
    return _Softmax.apply(x.contiguous(), False)


def log_softmax(x: torch.Tensor) -> torch.Tensor:
    """Last-axis log-softmax of an F32 tensor (AscendRuntime::log_softmax, runtime/mod.rs:327-341)."""
    return _Softmax.apply(x.contiguous(), True)


class _SiluMul(torch.autograd.Function):
    @staticmethod
    def forward(ctx, gate, up):
        ctx.save_for_backward(gate, up)
        return HipRuntime.silu_mul(gate, up)

    @staticmethod
    def backward(ctx, dy):
        gate, up = ctx.saved_tensors
        dg, du = HipRuntime.silu_mul_backward(gate, up, dy.contiguous().to(gate.dtype))
        return dg, du


def silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """SiLU(gate) * up (F32 or BF16). Reference: nn::silu_mul / SiluMulBackend (src/nn.rs:109-119,
    334-349); when gate and up are the same tensor autograd adds both gradients, as the
    reference's shared-node case does (examples/silu_mul_tensor.rs:51-53)."""
    return _SiluMul.apply(gate.contiguous(), up.contiguous())


class _BiasAdd(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, bias, residual):
        ctx.has_residual = residual is not None
        return HipRuntime.bias_add(x, bias, residual)

    @staticmethod
    def backward(ctx, dy):
        dy = dy.contiguous()
        # only a bias that needs a gradient pays for the column reduction (affine.rs:52-58)
        db = HipRuntime.bias_add_backward(dy) if ctx.needs_input_grad[1] else None
        return dy, db, (dy if ctx.has_residual else None)


def bias_add(x: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    """X[..., H] + bias[H] (F32; BF16 X also accepted). Reference: nn::bias_add (src/nn/affine.rs:14-20)."""
    return _BiasAdd.apply(x.contiguous(), bias.contiguous(), None)


def residual_bias_add(x: torch.Tensor, residual: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    """(X + residual) + bias in that F32 order; residual must match X exactly. Reference:
    nn::residual_bias_add (src/nn/affine.rs:21-25)."""
    return _BiasAdd.apply(x.contiguous(), bias.contiguous(), residual.contiguous())


class _Embedding(torch.autograd.Function):
    @staticmethod
    def forward(ctx, weight, ids, padding_idx, scale_grad_by_freq):
        out = HipRuntime.embedding(weight, ids)
        ctx.save_for_backward(ids.clone())  # an independent snapshot of the IDs (mod.rs:248-251)
        ctx.rows = weight.shape[0]
        ctx.options = (padding_idx, scale_grad_by_freq)
        return out

    @staticmethod
    def backward(ctx, dy):
        (ids,) = ctx.saved_tensors
        padding_idx, scale = ctx.options
        dw = HipRuntime.embedding_backward(dy.contiguous(), ids, ctx.rows, padding_idx, scale)
        return dw, None, None, None


def embedding(weight: torch.Tensor, ids: torch.Tensor, padding_idx=None, scale_grad_by_freq: bool = False):
    """weight[ids] with a dense weight gradient; padding affects only the derivative. Reference:
    nn::embedding / embedding_nd with EmbeddingOptions (src/nn/embedding.rs:14-31, 54-90)."""
    if padding_idx is not None and not 0 <= padding_idx < weight.shape[0]:
        raise ValueError("embedding padding row is outside its table")
    return _Embedding.apply(weight.contiguous(), ids.contiguous(), padding_idx, bool(scale_grad_by_freq))


def swiglu_bf16_fp32(x: torch.Tensor, gate: torch.Tensor, up: torch.Tensor, down: torch.Tensor) -> torch.Tensor:
    """(SiLU(x gate^T) * (x up^T)) down^T with F32 storage and BF16 linear compute.
    Reference: nn::swiglu_bf16_fp32 (src/nn/feed_forward.rs:24-42): gate/up [H,K], down [N,H],
    every dimension a positive multiple of 16."""
    m, k = x.shape
    h, gk = gate.shape
    n, dh = down.shape
    if gk != k or tuple(up.shape) != (h, k) or dh != h or any(d <= 0 or d % 16 for d in (m, n, k, h)):
        raise ValueError("SwiGLU requires aligned X[M,K], gate/up[H,K] and down[N,H]")
    if any(t.dtype != torch.float32 for t in (x, gate, up, down)):
        raise ValueError("SwiGLU requires FP32 input and weights")
    g = linear_bf16_fp32(x, gate)
    u = linear_bf16_fp32(x, up)
    return linear_bf16_fp32(silu_mul(g, u), down)


class _Rotary(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, cos, sin, layout, width):
        ctx.save_for_backward(cos, sin)
        ctx.layout, ctx.width = layout, width
        if width is None:
            return HipRuntime.rotary(x, cos, sin, layout)
        return HipRuntime.rotary_prefix(x, cos, sin, width, layout)

    @staticmethod
    def backward(ctx, dy):
        cos, sin = ctx.saved_tensors
        dy = dy.contiguous()
        if ctx.width is None:
            dx = HipRuntime.rotary_backward(dy, cos, sin, ctx.layout)
        else:
            dx = HipRuntime.rotary_prefix_backward(dy, cos, sin, ctx.width, ctx.layout)
        return dx, None, None, None, None


def rotary(x, cos, sin, layout=RotaryLayout.SplitHalf) -> torch.Tensor:
    """Reference: nn::rotary (src/nn/rotary.rs:32-53)."""
    return _Rotary.apply(x.contiguous(), cos.contiguous(), sin.contiguous(), RotaryLayout(layout), None)


def rotary_prefix(x, cos, sin, width: int, layout=RotaryLayout.SplitHalf) -> torch.Tensor:
    """Reference: nn::rotary_prefix (src/nn/rotary.rs:55-105)."""
    return _Rotary.apply(x.contiguous(), cos.contiguous(), sin.contiguous(), RotaryLayout(layout), int(width))


class _Attention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, scale, causal, query_start, key_start):
        o, lse = HipRuntime.attention_forward(q, k, v, scale, causal, query_start, key_start)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.args = (scale, causal, query_start, key_start)
        return o

    @staticmethod
    def backward(ctx, dy):
        q, k, v, o, lse = ctx.saved_tensors
        scale, causal, qs, ks = ctx.args
        dq, dk, dv = HipRuntime.attention_backward(q, k, v, o, lse, dy.contiguous().to(torch.bfloat16), scale,
                                                   causal, qs, ks, grad_dtype=q.dtype)
        return dq, dk, dv, None, None, None, None


def grouped_query_attention_bf16(q, k, v, scale: float) -> torch.Tensor:
    """Non-causal GQA, Q[B,Hq,M,D], K/V[B,Hkv,N,D]. Reference:
    nn::grouped_query_attention_bf16_fp32 without a mask (src/nn/attention.rs:49-67)."""
    return _Attention.apply(q.contiguous(), k.contiguous(), v.contiguous(), float(scale), False, 0, 0)


def causal_grouped_query_attention_bf16(q, k, v, scale: float, query_start: int = 0, key_start: int = 0):
    """Causal GQA with absolute query/key starts. Reference:
    nn::causal_grouped_query_attention_bf16_fp32 (src/nn/attention.rs:68-80)."""
    return _Attention.apply(q.contiguous(), k.contiguous(), v.contiguous(), float(scale), True, int(query_start),
                            int(key_start))


class _AttentionF32(torch.autograd.Function):
    """The FP32 surface on the fused kernels: F32 Q/K/V are rounded to BF16 by the library, O is
    written in F32 and enters the backward's row term unrounded; F32 gradients."""

    @staticmethod
    def forward(ctx, q, k, v, scale, causal, query_start, key_start):
        o, lse = HipRuntime.attention_forward(q, k, v, scale, causal, query_start, key_start, out_dtype=torch.float32)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.args = (scale, causal, query_start, key_start)
        return o

    @staticmethod
    def backward(ctx, dy):
        q, k, v, o, lse = ctx.saved_tensors
        scale, causal, qs, ks = ctx.args
        dq, dk, dv = HipRuntime.attention_backward(q, k, v, o, lse, dy.contiguous().float(), scale, causal, qs, ks,
                                                   grad_dtype=torch.float32)
        return dq, dk, dv, None, None, None, None


class _MaskedAttention(torch.autograd.Function):
    """The reference's materialized attention (additive mask, any value width): saves Q, K, V and
    the mask and recomputes the probabilities in the backward."""

    @staticmethod
    def forward(ctx, q, k, v, mask, scale):
        o = HipRuntime.attention_masked_forward(q, k, v, scale, mask)
        ctx.save_for_backward(q, k, v, mask)
        ctx.scale = scale
        return o

    @staticmethod
    def backward(ctx, dy):
        q, k, v, mask = ctx.saved_tensors
        want_dmask = mask is not None and ctx.needs_input_grad[3]
        dq, dk, dv, dmask = HipRuntime.attention_masked_backward(q, k, v, mask, dy.contiguous().float(), ctx.scale,
                                                                 mask_grad=want_dmask)
        return dq, dk, dv, dmask, None


_FUSED_WIDTHS = (16, 32, 64, 128)


def _fused_ok(q, v) -> bool:
    return q.shape[-1] == v.shape[-1] and q.shape[-1] in _FUSED_WIDTHS


def _f32(*ts):
    return [t.contiguous() for t in ts]


def grouped_query_attention_bf16_fp32(q, k, v, scale: float, additive_mask=None) -> torch.Tensor:
    """F32 Q[B,Hq,M,D], K[B,Hkv,N,D], V[B,Hkv,N,Dv] -> F32 O[B,Hq,M,Dv] with an optional F32
    additive mask [B,Hq,M,N] (differentiable). Without a mask and with Dv == D in {16,32,64,128}
    this runs the fused kernels; otherwise the materialized path of the reference. Reference:
    nn::grouped_query_attention_bf16_fp32 (src/nn/attention.rs:49-67)."""
    q, k, v = _f32(q, k, v)
    if additive_mask is None and _fused_ok(q, v):
        return _AttentionF32.apply(q, k, v, float(scale), False, 0, 0)
    mask = None if additive_mask is None else additive_mask.contiguous()
    return _MaskedAttention.apply(q, k, v, mask, float(scale))


def causal_grouped_query_attention_bf16_fp32(q, k, v, scale: float, query_start: int = 0, key_start: int = 0):
    """F32 GQA with the exact-position causal mask (key j excluded when key_start + j >
    query_start + i). Fused when Dv == D in {16,32,64,128}, else the materialized path with the
    device-generated mask. Reference: nn::causal_grouped_query_attention_bf16_fp32
    (src/nn/attention.rs:68-80)."""
    q, k, v = _f32(q, k, v)
    if _fused_ok(q, v):
        return _AttentionF32.apply(q, k, v, float(scale), True, int(query_start), int(key_start))
    b, h, m, _ = q.shape
    mask = HipRuntime.causal_mask(b * h, m, k.shape[2], query_start, key_start, q.device).view(b, h, m, k.shape[2])
    return _MaskedAttention.apply(q, k, v, mask, float(scale))


def scaled_dot_product_attention_bf16_fp32(q, k, v, scale: float, additive_mask=None) -> torch.Tensor:
    """Rank-3 F32 attention Q[B,M,D], K[B,N,D], V[B,N,Dv] with an optional F32 additive mask
    [B,M,N]. Reference: nn::scaled_dot_product_attention_bf16_fp32 (src/nn/attention.rs:10-29)."""
    q, k, v = _f32(q, k, v)
    if additive_mask is None and _fused_ok(q, v):
        return _AttentionF32.apply(q[:, None], k[:, None], v[:, None], float(scale), False, 0, 0)[:, 0]
    mask = None if additive_mask is None else additive_mask.contiguous()
    return _MaskedAttention.apply(q, k, v, mask, float(scale))


def causal_attention_bf16_fp32(q, k, v, scale: float, query_start: int = 0, key_start: int = 0) -> torch.Tensor:
    """Rank-3 F32 causal attention with absolute positions. Reference: nn::causal_attention_bf16_fp32
    (src/nn/attention.rs:30-43)."""
    return causal_grouped_query_attention_bf16_fp32(q[:, None], k[:, None], v[:, None], scale, query_start,
                                                    key_start)[:, 0]


class _NllLoss(torch.autograd.Function):
    @staticmethod
    def forward(ctx, input, target, weight, reduction, ignore_index):
        out, total, t, w = HipRuntime.nll_loss_with_saved_inputs(input.contiguous(), target.contiguous(),
                                                                 weight.contiguous(), reduction, ignore_index)
        ctx.save_for_backward(input, t, w, total)
        ctx.reduction, ctx.ignore_index = reduction, ignore_index
        return out

    @staticmethod
    def backward(ctx, grad):
        input, t, w, total = ctx.saved_tensors
        dx = HipRuntime.nll_loss_backward(grad.contiguous().to(input.dtype), input, t, w, total, ctx.reduction,
                                          ctx.ignore_index)
        return dx, None, None, None, None


def nll_loss(input, target, weight, reduction=LossReduction.Mean, ignore_index=None):
    """NLLLoss of log-probabilities input [N, C] with fixed class weights (no gradient for the
    weights or labels). Returns [N] (None) or [1]. Reference: nn::nll_loss and NllBackward
    (src/nn/loss.rs:34-41, 88-132): the backward saves the input, label and weight snapshots and
    the forward's total weight."""
    return _NllLoss.apply(input, target, weight, LossReduction(reduction), ignore_index)


def weighted_cross_entropy(logits, target, weight, reduction=LossReduction.Mean, ignore_index=None):
    """nll_loss(log_softmax(logits)) with fixed class weights: F32 logits [N, C], integer labels [N],
    F32 weights [C]. Reference: nn::weighted_cross_entropy (src/nn/loss.rs:52-64)."""
    if logits.dim() != 2 or logits.dtype != torch.float32 or weight.dtype != torch.float32 or \
            target.dtype not in (torch.int32, torch.int64) or tuple(target.shape) != (logits.shape[0],) or \
            tuple(weight.shape) != (logits.shape[1],):
        from ._lib import INVALID_ARGUMENT, HkError
        raise HkError(INVALID_ARGUMENT, "cross entropy requires same-device FP32 logits[N,C], integer labels[N] "
                                        "and FP32 weights[C]")
    return nll_loss(log_softmax(logits), target, weight, reduction, ignore_index)


def cross_entropy(logits, target, reduction=LossReduction.Mean, ignore_index=None):
    """Unweighted cross entropy (class weights of one). Reference: nn::cross_entropy (src/nn/loss.rs:42-50)."""
    weight = torch.ones((logits.shape[1],), dtype=torch.float32, device=logits.device)
    return weighted_cross_entropy(logits, target, weight, reduction, ignore_index)
