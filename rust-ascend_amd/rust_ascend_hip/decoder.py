"""One Llama-style decoder layer, forward and backward, composed from libhk.so's entry points.

The reference composes a layer from its nn functions (src/nn/{embedding,attention,rotary,
feed_forward,affine}.rs and nn::rms_norm); this is the same composition for BF16 activations on
one GPU, arranged for MI355X: one fused QKV projection that writes the head planes with RoPE
applied in its epilogue (and an attention backward that writes the projection's gradient rows,
RoPE's transpose applied in its epilogue), causal grouped-query attention in one fused kernel each way,
SwiGLU on two projections, bias-free residual adds, and every activation and gradient buffer
allocated once. A step is a fixed sequence of C-ABI calls with descriptors built at set-up, so
nothing is allocated and no host synchronization happens inside it (with the context in async
mode). Every op is a HIP kernel of libhk.so; PyTorch only owns the device memory.

Forward, tokens T = B*S, width H, heads Hq/Hkv of size D, feed-forward width F:
    x0 = embedding(table, ids)                       [T, H]   BF16
    n1, rstd1 = rms_norm(x0, w1)                              (F32 weight and rstd)
    q, k, v = split(n1 Wqkv^T) with RoPE on q, k      [B, H, S, D]   (one launch)
    o, lse = causal_attention(q, k, v)
    h1 = x0 + rows(o) Wo^T                                    (the add in the GEMM epilogue)
    n2, rstd2 = rms_norm(h1, w2)
    g = n2 Wg^T;  u = n2 Wu^T;  m = silu(g) * u      [T, F]   (one GEMM over [Wg; Wu], silu-mul in
                                                               its epilogue)
    y = h1 + m Wd^T                                           (the add in the GEMM epilogue)
Backward takes dY and produces every parameter gradient (F32 for the projections and norms,
BF16 for the embedding table, as hk_embedding_backward writes the gradient's dtype).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib, runtime
from ._lib import check
from .runtime import RotaryLayout


@dataclass(frozen=True)
class DecoderConfig:
    """hidden 4096, 32/8 heads, SwiGLU 14336, batch 2 x seq 2048, vocab 32000."""
    hidden: int = 4096
    heads: int = 32
    kv_heads: int = 8
    ffn: int = 14336
    vocab: int = 32000
    batch: int = 2
    seq: int = 2048
    eps: float = 1e-5
    theta: float = 5e5
    init_std: float = 0.02

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads

    @property
    def tokens(self) -> int:
        return self.batch * self.seq

    def flops_per_step(self) -> dict:
        """Model FLOPs of one forward + backward: GEMMs 2*T*params forward and twice that
        backward; attention in the causal-useful convention (forward 2*B*Hq*S^2*D, backward 2.5x)."""
        h, f, d = self.hidden, self.ffn, self.head_dim
        proj = h * (self.heads + 2 * self.kv_heads) * d + h * h + 3 * h * f
        gemm_fwd = 2 * self.tokens * proj
        attn_fwd = 2 * self.batch * self.heads * self.seq * self.seq * d
        return {"gemm": 3 * gemm_fwd, "attention": attn_fwd + 2.5 * attn_fwd,
                "total": 3 * gemm_fwd + 3.5 * attn_fwd}


def rope_tables(seq: int, dim: int, theta: float):
    """cos/sin [seq, dim/2] F32 for positions 0..seq-1, angle = s * theta^(-2i/dim), computed in
    float64 (the reference leaves the frequency policy to the caller)."""
    inv = theta ** (-np.arange(0, dim, 2, dtype=np.float64) / dim)
    ang = np.arange(seq, dtype=np.float64)[:, None] * inv[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


class DecoderLayer:
    """Parameters, saved activations, gradients and the C-ABI call sequence of one layer."""

    def __init__(self, cfg: DecoderConfig = DecoderConfig(), seed: int = 0, device="cuda", fused_rope: bool = True,
                 fused_ffn: bool = True):
        self.cfg = c = cfg
        if c.hidden % c.heads or c.heads % c.kv_heads or c.head_dim % 16:
            raise ValueError("hidden must split into heads of a multiple of 16, heads into KV groups")
        # RoPE inside the QKV projection's epilogue and the attention backward's (heads of 128, or
        # 64 for the backward); otherwise the projection writes token rows that qkv_rope_split
        # moves into the head planes, and qkv_rope_merge moves the gradients back
        self.fused_rope = fused_rope and c.head_dim == 128 and c.hidden % 8 == 0
        # the O and down projections add their residual in the GEMM epilogue; gate and up are one GEMM
        # (weights interleaved in blocks of 16 rows) with SiLU-mul in its epilogue, and the SwiGLU
        # backward runs in the epilogue of dY Wd, so dX and dW of gate/up are one GEMM each; the two
        # norms' backward add the residual branch's gradient as they store dX
        self.fused_ffn = fused_ffn and c.ffn % 16 == 0 and c.hidden % 16 == 0
        dev = torch.device(device)
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        bf, f32 = torch.bfloat16, torch.float32
        T, H, F, D = c.tokens, c.hidden, c.ffn, c.head_dim
        W = (c.heads + 2 * c.kv_heads) * D

        def init(*shape):
            return (torch.randn(shape, generator=g, device=dev) * c.init_std).to(bf)

        # parameters (BF16 projections, F32 norm weights)
        self.table = init(c.vocab, H)
        self.wqkv, self.wo = init(W, H), init(H, H)
        wg, wu, self.wd = init(F, H), init(F, H), init(H, F)
        # W_gu row 32 b + r: gate row 16 b + r (r < 16), up row 16 b + r - 16
        self.w_gu = torch.stack([wg.view(F // 16, 16, H), wu.view(F // 16, 16, H)], dim=1).reshape(2 * F, H)
        del wg, wu
        self.w1 = torch.ones(H, device=dev, dtype=f32)
        self.w2 = torch.ones(H, device=dev, dtype=f32)
        cos, sin = rope_tables(c.seq, D, c.theta)
        self.cos, self.sin = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)

        def buf(*shape, dtype=bf):
            return torch.empty(shape, device=dev, dtype=dtype)

        # forward activations (kept for the backward)
        self.ids = torch.zeros((c.batch, c.seq), device=dev, dtype=torch.int64)
        self.x0, self.n1, self.rstd1 = buf(T, H), buf(T, H), buf(T, dtype=f32)
        self.qkv = None if self.fused_rope else buf(c.batch, c.seq, W)
        self.q, self.k, self.v = buf(c.batch, c.heads, c.seq, D), buf(c.batch, c.kv_heads, c.seq, D), \
            buf(c.batch, c.kv_heads, c.seq, D)
        self.o, self.lse = buf(c.batch, c.heads, c.seq, D), buf(c.batch, c.heads, c.seq, dtype=f32)
        self.o_rows, self.h1 = buf(c.batch, c.seq, H), buf(T, H)
        self.n2, self.rstd2 = buf(T, H), buf(T, dtype=f32)
        self.gate, self.up, self.m = buf(T, F), buf(T, F), buf(T, F)
        self.y = buf(T, H)
        # gradients
        self.dy = buf(T, H)
        self.dn2 = buf(T, H)
        if self.fused_ffn:
            self.dgu = buf(T, 2 * F)
        else:
            self._wg, self._wu = self.wg, self.wu  # separate gate and up weights
            self.a, self.ffn_out = buf(T, H), buf(T, H)
            self.dm, self.dgate, self.dup = buf(T, F), buf(T, F), buf(T, F)
            self.dn2_g, self.dn2_u = buf(T, H), buf(T, H)
        self.dh1_norm, self.dh1 = buf(T, H), buf(T, H)
        self.do_rows, self.do = buf(c.batch, c.seq, H), buf(c.batch, c.heads, c.seq, D)
        if not self.fused_rope:
            self.dq, self.dk, self.dv = buf(c.batch, c.heads, c.seq, D), buf(c.batch, c.kv_heads, c.seq, D), \
                buf(c.batch, c.kv_heads, c.seq, D)
        self.dqkv, self.dn1, self.dx0_norm, self.dx0 = buf(c.batch, c.seq, W), buf(T, H), buf(T, H), buf(T, H)
        self.grads = {"table": buf(c.vocab, H), "wqkv": buf(W, H, dtype=f32), "wo": buf(H, H, dtype=f32),
                      "wd": buf(H, F, dtype=f32), "w1": buf(H, dtype=f32), "w2": buf(H, dtype=f32)}
        if self.fused_ffn:
            self.grads["w_gu"] = buf(2 * F, H, dtype=f32)
        else:
            self.grads["wg"], self.grads["wu"] = buf(F, H, dtype=f32), buf(F, H, dtype=f32)
        self._build_calls()

    # ------------------------------------------------------------------ call sequences

    def _build_calls(self):
        c = self.cfg
        lib = _lib.load()
        T, H, W = c.tokens, c.hidden, (c.heads + 2 * c.kv_heads) * c.head_dim
        d = runtime.desc

        def rows(t, width):  # a [T, width] view of a token-major buffer
            return runtime.desc(t.view(T, width))

        gr = self.grads
        eps = ctypes.c_double(c.eps)
        scale = ctypes.c_float(c.head_dim ** -0.5)
        z = ctypes.c_uint64(0)
        sh = int(RotaryLayout.SplitHalf)
        no, yes = 0, 1
        self._forward = [
            (lib.hk_embedding, (d(self.table), d(self.ids), d(self.x0.view(c.batch, c.seq, H)))),
            (lib.hk_rms_norm, (d(self.x0), d(self.w1), eps, d(self.n1), d(self.rstd1))),
            *([(lib.hk_qkv_projection_rope, (d(self.n1), d(self.wqkv), d(self.cos), d(self.sin), sh, d(self.q),
                                               d(self.k), d(self.v)))] if self.fused_rope else
              [(lib.hk_gemm_into, (d(self.n1), d(self.wqkv), no, yes, rows(self.qkv, W))),
               (lib.hk_qkv_rope_split, (d(self.qkv), d(self.cos), d(self.sin), sh, d(self.q), d(self.k),
                                        d(self.v)))]),
            (lib.hk_attention_forward, (d(self.q), d(self.k), d(self.v), scale, 1, z, z, d(self.o), d(self.lse))),
            (lib.hk_heads_to_rows, (d(self.o), d(self.o_rows))),
            *([(lib.hk_linear_residual, (rows(self.o_rows, H), d(self.wo), d(self.x0), d(self.h1))),
               (lib.hk_rms_norm, (d(self.h1), d(self.w2), eps, d(self.n2), d(self.rstd2))),
               (lib.hk_swiglu_projection, (d(self.n2), d(self.w_gu), d(self.gate), d(self.up), d(self.m))),
               (lib.hk_linear_residual, (d(self.m), d(self.wd), d(self.h1), d(self.y)))] if self.fused_ffn else
              [(lib.hk_gemm_into, (rows(self.o_rows, H), d(self.wo), no, yes, d(self.a))),
               (lib.hk_bias_add, (d(self.a), None, d(self.x0), d(self.h1))),
               (lib.hk_rms_norm, (d(self.h1), d(self.w2), eps, d(self.n2), d(self.rstd2))),
               (lib.hk_gemm_into, (d(self.n2), d(self._wg), no, yes, d(self.gate))),
               (lib.hk_gemm_into, (d(self.n2), d(self._wu), no, yes, d(self.up))),
               (lib.hk_silu_mul, (d(self.gate), d(self.up), d(self.m))),
               (lib.hk_gemm_into, (d(self.m), d(self.wd), no, yes, d(self.ffn_out))),
               (lib.hk_bias_add, (d(self.ffn_out), None, d(self.h1), d(self.y)))]),
        ]
        self._backward = [
            # y = h1 + m Wd^T: dh1 gets dY directly; dm = dY Wd, dWd = dY^T m
            *([(lib.hk_gemm_into, (d(self.dy), d(self.m), yes, no, d(gr["wd"]))),
               (lib.hk_swiglu_projection_backward, (d(self.dy), d(self.wd), d(self.gate), d(self.up), d(self.dgu))),
               (lib.hk_linear_nt_backward, (d(self.n2), d(self.w_gu), d(self.dgu), d(self.dn2), d(gr["w_gu"])))]
              if self.fused_ffn else
              [(lib.hk_linear_nt_backward, (d(self.m), d(self.wd), d(self.dy), d(self.dm), d(gr["wd"]))),
               (lib.hk_silu_mul_backward, (d(self.gate), d(self.up), d(self.dm), d(self.dgate), d(self.dup))),
               (lib.hk_linear_nt_backward, (d(self.n2), d(self._wg), d(self.dgate), d(self.dn2_g), d(gr["wg"]))),
               (lib.hk_linear_nt_backward, (d(self.n2), d(self._wu), d(self.dup), d(self.dn2_u), d(gr["wu"]))),
               (lib.hk_bias_add, (d(self.dn2_g), None, d(self.dn2_u), d(self.dn2)))]),
            # dh1 = dY (the residual branch) + the norm's backward: one pass in the fused composition
            *([(lib.hk_rms_norm_backward_residual, (d(self.h1), d(self.w2), d(self.dn2), d(self.rstd2), d(self.dy),
                                                    d(self.dh1), d(gr["w2"])))] if self.fused_ffn else
              [(lib.hk_rms_norm_backward, (d(self.h1), d(self.w2), d(self.dn2), d(self.rstd2), d(self.dh1_norm),
                                           d(gr["w2"]))),
               (lib.hk_bias_add, (d(self.dh1_norm), None, d(self.dy), d(self.dh1)))]),
            # h1 = x0 + rows(o) Wo^T
            (lib.hk_linear_nt_backward, (rows(self.o_rows, H), d(self.wo), d(self.dh1), rows(self.do_rows, H),
                                         d(gr["wo"]))),
            (lib.hk_rows_to_heads, (d(self.do_rows), d(self.do))),
            *([(lib.hk_attention_backward_qkv_rows, (d(self.q), d(self.k), d(self.v), d(self.o), d(self.lse),
                                                     d(self.do), scale, 1, z, z, d(self.cos), d(self.sin), sh,
                                                     d(self.dqkv)))] if self.fused_rope else
              [(lib.hk_attention_backward, (d(self.q), d(self.k), d(self.v), d(self.o), d(self.lse), d(self.do),
                                            scale, 1, z, z, d(self.dq), d(self.dk), d(self.dv))),
               (lib.hk_qkv_rope_merge, (d(self.dq), d(self.dk), d(self.dv), d(self.cos), d(self.sin), sh,
                                        d(self.dqkv)))]),
            (lib.hk_linear_nt_backward, (d(self.n1), d(self.wqkv), rows(self.dqkv, W), d(self.dn1), d(gr["wqkv"]))),
            *([(lib.hk_rms_norm_backward_residual, (d(self.x0), d(self.w1), d(self.dn1), d(self.rstd1), d(self.dh1),
                                                    d(self.dx0), d(gr["w1"])))] if self.fused_ffn else
              [(lib.hk_rms_norm_backward, (d(self.x0), d(self.w1), d(self.dn1), d(self.rstd1), d(self.dx0_norm),
                                           d(gr["w1"]))),
               (lib.hk_bias_add, (d(self.dx0_norm), None, d(self.dh1), d(self.dx0)))]),
            (lib.hk_embedding_backward, (d(self.dx0.view(c.batch, c.seq, H)), d(self.ids), ctypes.c_uint64(c.vocab),
                                         ctypes.c_uint64(_lib.NO_PADDING), 0, d(gr["table"]))),
        ]
        self._lib = lib

    def _run(self, calls):
        ctx = runtime._context()
        check(self._lib.hk_set_stream(ctx, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
        for fn, args in calls:
            check(fn(ctx, *args))

    # ------------------------------------------------------------------ public steps

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        """ids [B, S] (int32/int64, copied into the layer's ID buffer) -> y [B, S, H] BF16 (a view
        of the layer's output buffer, overwritten by the next forward)."""
        c = self.cfg
        if tuple(ids.shape) != (c.batch, c.seq):
            raise ValueError(f"ids must be [{c.batch}, {c.seq}]")
        if ids.data_ptr() != self.ids.data_ptr():
            self.ids.copy_(ids)
        self._run(self._forward)
        return self.y.view(c.batch, c.seq, c.hidden)

    @property
    def wg(self) -> torch.Tensor:
        """The gate projection's weight [F, H] (a copy out of the interleaved W_gu)."""
        return self._gate_up(self.w_gu, 0)

    @property
    def wu(self) -> torch.Tensor:
        """The up projection's weight [F, H] (a copy out of the interleaved W_gu)."""
        return self._gate_up(self.w_gu, 1)

    def _gate_up(self, t: torch.Tensor, which: int) -> torch.Tensor:
        f, h = self.cfg.ffn, t.shape[1]
        return t.view(f // 16, 2, 16, h)[:, which].reshape(f, h)

    def backward(self, dy: torch.Tensor) -> dict:
        """dy [B, S, H] BF16 (copied into the layer's buffer) -> the parameter gradients
        {table, wqkv, wo, wg, wu, wd, w1, w2}, valid until the next backward (wg and wu are
        copies out of the interleaved gradient of W_gu). Uses the activations of the last forward."""
        if dy.data_ptr() != self.dy.data_ptr():
            self.dy.copy_(dy.reshape(self.dy.shape))
        self._run(self._backward)
        if not self.fused_ffn:
            return self.grads
        out = {k: v for k, v in self.grads.items() if k != "w_gu"}
        out["wg"], out["wu"] = self._gate_up(self.grads["w_gu"], 0), self._gate_up(self.grads["w_gu"], 1)
        return out

    def step(self) -> None:
        """Forward + backward on the buffers already in place (the benchmark's timed unit)."""
        self._run(self._forward)
        self._run(self._backward)
