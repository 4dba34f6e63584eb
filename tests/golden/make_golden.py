"""Writes tests/golden/golden.npz: golden vectors for the BF16 transformer kernel path.

Inputs follow the integer formulas of the reference's own tests (cited per case,
paths relative to the shuqi2077/rust-ascend root). Expected outputs are computed here
independently of oracle/ — numpy float64 matmul, torch float64 autograd, or the
reference's closed forms — so the oracle is checked against them, not with itself.

Run: python tests/golden/make_golden.py   (CPU only, a few seconds)
"""
from __future__ import annotations

import os

import numpy as np
import torch

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.npz")


def bf16(x):
    """RNE to BF16 via torch's own conversion (independent of the oracle's C code)."""
    return torch.tensor(np.asarray(x, dtype=np.float32)).to(torch.bfloat16).to(torch.float32).numpy()


def gemm_np(a, b, ta, tb):
    a = a.astype(np.float64)
    b = b.astype(np.float64)
    if a.ndim == 2:
        return (a.T if ta else a) @ (b.T if tb else b)
    return np.stack([(a[i].T if ta else a[i]) @ (b[i].T if tb else b[i]) for i in range(a.shape[0])])


def main():
    g = {}

    # ---- GEMM -------------------------------------------------------------
    # rust-ascend-driver/examples/deepgemm_validate.rs:6,30-43: host(n,seed) = ((i*7+seed)%17)/8-1,
    # m,n,k = 32,64,48; A seed 1, B seed 4; batches 1 and 3; all transposes.
    host = lambda n, seed: ((np.arange(n) * 7 + seed) % 17).astype(np.float32) / 8.0 - 1.0
    for batch in (1, 3):
        m, n, k = 32, 64, 48
        a = host(batch * m * k, 1)
        b = host(batch * k * n, 4)
        for ta in (0, 1):
            for tb in (0, 1):
                ash = (k, m) if ta else (m, k)
                bsh = (n, k) if tb else (k, n)
                if batch != 1:
                    ash = (batch,) + ash
                    bsh = (batch,) + bsh
                A = a.reshape(ash)
                B = b.reshape(bsh)
                key = f"gemm_dv_b{batch}_{'tn'[ta]}{'tn'[tb]}"
                g[key + "_a"] = A
                g[key + "_b"] = B
                g[key + "_out"] = gemm_np(A, B, ta, tb)
    # rust-ascend-kernels/src/tests.rs:91-92,124-128: a = bf16(((i%23)-11)/16), b = bf16(((i%17)-8)/8);
    # dense 80x96x144 (every transpose) and batched 3x16x32x16.
    for (batch, m, n, k) in ((1, 80, 96, 144), (3, 16, 32, 16)):
        a = bf16(((np.arange(batch * m * k) % 23).astype(np.float32) - 11) / 16)
        b = bf16(((np.arange(batch * n * k) % 17).astype(np.float32) - 8) / 8)
        for ta in (0, 1):
            for tb in (0, 1):
                ash = (k, m) if ta else (m, k)
                bsh = (n, k) if tb else (k, n)
                if batch != 1:
                    ash = (batch,) + ash
                    bsh = (batch,) + bsh
                A = a.reshape(ash)
                B = b.reshape(bsh)
                key = f"gemm_vm_{batch}x{m}x{n}x{k}_{'nt'[ta]}{'nt'[tb]}"
                g[key + "_a"] = A
                g[key + "_b"] = B
                g[key + "_out"] = gemm_np(A, B, ta, tb)
    # M-grouped NT, rust-ascend-kernels/src/tests.rs:89-103,130-132: m,n,k = 768,16,144, ends
    # [0,256,256,768] (experts 0 and 2 empty), the formulas above over m*k and groups*n*k values.
    # Expected: numpy float64 per row slice with the slice's own weight matrix.
    def grouped_np(a, w, ends):
        out = np.full((a.shape[0], w.shape[1]), np.nan)
        begin = 0
        for e, end in enumerate(ends):
            out[begin:end] = a[begin:end].astype(np.float64) @ w[e].astype(np.float64).T
            begin = end
        return out
    m, n, k, ends = 768, 16, 144, [0, 256, 256, 768]
    a = bf16(((np.arange(m * k) % 23).astype(np.float32) - 11) / 16).reshape(m, k)
    w = bf16(((np.arange(len(ends) * n * k) % 17).astype(np.float32) - 8) / 8).reshape(len(ends), n, k)
    g["grouped_vm_a"], g["grouped_vm_w"], g["grouped_vm_ends"] = a, w, np.array(ends, dtype=np.int32)
    g["grouped_vm_out"] = grouped_np(a, w, ends)
    # rust-ascend-driver/examples/deepgemm_validate.rs:45-53: m,n,k = 512,64,48, ends [256,256,512],
    # A = host(m*k, 2), W = host(3*n*k, 5) (host as above); rows 256.. use W[2].
    m, n, k, ends = 512, 64, 48, [256, 256, 512]
    a = host(m * k, 2).reshape(m, k)
    w = host(3 * n * k, 5).reshape(3, n, k)
    g["grouped_dv_a"], g["grouped_dv_w"], g["grouped_dv_ends"] = a, w, np.array(ends, dtype=np.int32)
    g["grouped_dv_out"] = np.concatenate([a[:256].astype(np.float64) @ w[0].astype(np.float64).T,
                                          a[256:].astype(np.float64) @ w[2].astype(np.float64).T])

    # Padded BF16-compute GEMM, examples/padded_matrix_tensor.rs:12-45,77-80: (m,n,k) in
    # {(1,1,1),(3,17,7),(17,33,65),(16,32,48)}, all transposes, rank 2 and batch-2 rank 3;
    # a = ((i%17)-8)/59, b = ((i%13)-6)/43, dy = ((i%11)-5)/37 (F32). Expected (the reference's host
    # loop): f64 sums of BF16-rounded products, Y and the gradients of sum(Y * dy).
    for batch in (None, 2):
        nb = batch or 1
        for (m, n, k) in ((1, 1, 1), (3, 17, 7), (17, 33, 65), (16, 32, 48)):
            for ta in (0, 1):
                for tb in (0, 1):
                    a = ((np.arange(nb * m * k) % 17).astype(np.float32) - 8) / 59
                    b = ((np.arange(nb * k * n) % 13).astype(np.float32) - 6) / 43
                    dy = ((np.arange(nb * m * n) % 11).astype(np.float32) - 5) / 37
                    ash = (k, m) if ta else (m, k)
                    bsh = (n, k) if tb else (k, n)
                    A = a.reshape((nb,) + ash)
                    B = b.reshape((nb,) + bsh)
                    DY = dy.reshape(nb, m, n)
                    Ar, Br, Dr = (bf16(t).astype(np.float64) for t in (A, B, DY))
                    opA = Ar.transpose(0, 2, 1) if ta else Ar
                    opB = Br.transpose(0, 2, 1) if tb else Br
                    Y = opA @ opB
                    dopA = Dr @ opB.transpose(0, 2, 1)
                    dopB = opA.transpose(0, 2, 1) @ Dr
                    dA = dopA.transpose(0, 2, 1) if ta else dopA
                    dB = dopB.transpose(0, 2, 1) if tb else dopB
                    sq = (lambda t: t) if batch else (lambda t: t[0])
                    key = f"padded_{nb}_{m}x{n}x{k}_{'nt'[ta]}{'nt'[tb]}"
                    g[key + "_a"], g[key + "_b"], g[key + "_dy"] = sq(A), sq(B), sq(DY)
                    g[key + "_y"], g[key + "_da"], g[key + "_db"] = sq(Y), sq(dA), sq(dB)

    # examples/matrix_runtime.rs:70-77: linear_nt_backward, m,n,k = 32,48,16,
    # x = ((i%17)-8)*0.125, w = ((i%13)-6)*0.25, dy = ((i%11)-5)*0.0625.
    m, n, k = 32, 48, 16
    x = ((np.arange(m * k) % 17).astype(np.float32) - 8) * 0.125
    w = ((np.arange(n * k) % 13).astype(np.float32) - 6) * 0.25
    dy = ((np.arange(m * n) % 11).astype(np.float32) - 5) * 0.0625
    g["linbwd_x"] = x.reshape(m, k)
    g["linbwd_w"] = w.reshape(n, k)
    g["linbwd_dy"] = dy.reshape(m, n)
    g["linbwd_dx"] = dy.reshape(m, n).astype(np.float64) @ w.reshape(n, k).astype(np.float64)
    g["linbwd_dw"] = dy.reshape(m, n).astype(np.float64).T @ x.reshape(m, k).astype(np.float64)

    # ---- RMSNorm ----------------------------------------------------------
    # examples/rms_norm_runtime.rs:37-41: x = (i%31)/7-1, w = 0.5+(i%7)/9, dy = (i%11)/5-0.7, eps 1e-3.
    for rows, width in ((0, 32), (1, 32), (3, 96), (7, 256), (33, 4096), (3, 7), (2, 4100)):
        x = ((np.arange(rows * width) % 31).astype(np.float32) / 7 - 1).reshape(rows, width)
        w = (0.5 + (np.arange(width) % 7).astype(np.float32) / 9).astype(np.float32)
        dy = ((np.arange(rows * width) % 11).astype(np.float32) / 5 - 0.7).reshape(rows, width)
        tx = torch.tensor(x, dtype=torch.float64, requires_grad=True)
        tw = torch.tensor(w, dtype=torch.float64, requires_grad=True)
        rstd = torch.rsqrt(tx.square().mean(-1, keepdim=True) + 1e-3)
        y = tx * rstd * tw
        (y * torch.tensor(dy, dtype=torch.float64)).sum().backward()
        key = f"rms_{rows}x{width}"
        g[key + "_x"] = x
        g[key + "_w"] = w
        g[key + "_dy"] = dy
        g[key + "_y"] = y.detach().numpy()
        g[key + "_rstd"] = rstd.detach().numpy().reshape(rows)
        g[key + "_dx"] = tx.grad.numpy() if rows else np.zeros((0, width))
        g[key + "_dw"] = tw.grad.numpy() if rows else np.zeros(width)
    # examples/gradients.rs:20-37: x = [-2,-1,.5,1,2,3] as [2,3], gamma = [.5,1,2],
    # dy = [1,.5,-.25,-.5,1,.25], eps 1e-5.
    x = np.array([-2.0, -1.0, 0.5, 1.0, 2.0, 3.0], dtype=np.float32).reshape(2, 3)
    w = np.array([0.5, 1.0, 2.0], dtype=np.float32)
    dy = np.array([1.0, 0.5, -0.25, -0.5, 1.0, 0.25], dtype=np.float32).reshape(2, 3)
    tx = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    tw = torch.tensor(w, dtype=torch.float64, requires_grad=True)
    y = tx * torch.rsqrt(tx.square().mean(-1, keepdim=True) + 1e-5) * tw
    (y * torch.tensor(dy, dtype=torch.float64)).sum().backward()
    g["rmsgrad_x"], g["rmsgrad_w"], g["rmsgrad_dy"] = x, w, dy
    g["rmsgrad_y"] = y.detach().numpy()
    g["rmsgrad_dx"] = tx.grad.numpy()
    g["rmsgrad_dw"] = tw.grad.numpy()
    # rust-ascend-compiler/src/ascend/row_tests.rs:280-287: weight contributions dy*(x*rstd) with
    # x = 2, dy = 3, rstd = [0.5, 0.25, 2] -> [3, 1.5, 12].
    g["rmskat_rstd"] = np.array([0.5, 0.25, 2.0], dtype=np.float32)
    g["rmskat_contrib"] = np.array([3.0, 1.5, 12.0])

    # ---- RoPE -------------------------------------------------------------
    # examples/rotary_tensor.rs:23-29: (rows,width) in {(0,6),(1,2),(3,6),(2,96)},
    # x = (i%19)*0.25-2, dy = (i%7)*0.125-0.25, angle = (i%23)*0.125.
    for rows, width in ((0, 6), (1, 2), (3, 6), (2, 96)):
        n = rows * width
        x = ((np.arange(n) % 19).astype(np.float32) * 0.25 - 2).reshape(rows, width)
        dy = ((np.arange(n) % 7).astype(np.float32) * 0.125 - 0.25).reshape(rows, width)
        ang = (np.arange(n // 2) % 23).astype(np.float64) * 0.125
        c = np.cos(ang).astype(np.float32).reshape(rows, width // 2)
        s = np.sin(ang).astype(np.float32).reshape(rows, width // 2)
        for layout in (0, 1):
            tx = torch.tensor(x, dtype=torch.float64, requires_grad=True)
            tc = torch.tensor(c, dtype=torch.float64)
            ts = torch.tensor(s, dtype=torch.float64)
            half = width // 2
            if layout == 0:
                a, b = tx[:, 0::2], tx[:, 1::2]
                ya, yb = a * tc - b * ts, b * tc + a * ts
                y = torch.stack([ya, yb], dim=-1).reshape(rows, width)
            else:
                a, b = tx[:, :half], tx[:, half:]
                y = torch.cat([a * tc - b * ts, b * tc + a * ts], dim=-1)
            (y * torch.tensor(dy, dtype=torch.float64)).sum().backward()
            key = f"rope_{rows}x{width}_l{layout}"
            g[key + "_x"], g[key + "_dy"], g[key + "_cos"], g[key + "_sin"] = x, dy, c, s
            g[key + "_y"] = y.detach().numpy()
            g[key + "_dx"] = tx.grad.numpy() if rows else np.zeros((0, width))
    # rotary_programs.rs:222-260: prefix P=6 over width 11 with broadcast tables; tail values cycle
    # through -0, NaN(0x7fc01234), +Inf, -Inf and must keep their bits.
    for ci, (inp, tab) in enumerate((([11], [3]), ([2, 5, 11], [1, 5, 3]), ([2, 3, 5, 11], [2, 1, 5, 3]),
                                     ([2, 3, 5, 11], [1, 3, 1, 3]), ([2, 3, 5, 6], [1, 1, 5, 3]))):
        p = 6
        n = int(np.prod(inp))
        t = int(np.prod(tab))
        width = inp[-1]
        tails = np.array([0x80000000, 0x7FC01234, 0x7F800000, 0xFF800000], dtype=np.uint32).view(np.float32)
        idx = np.arange(n)
        x = np.where(idx % width >= p, tails[idx % 4], (idx % 17).astype(np.float32) / 8 - 0.75).astype(np.float32)
        c = (0.7 + (np.arange(t) % 3).astype(np.float32) / 8).astype(np.float32)
        s = (-0.3 + (np.arange(t) % 5).astype(np.float32) / 16).astype(np.float32)
        for layout in (0, 1):
            for backward in (0, 1):
                X = x.reshape(inp)
                C = c.reshape(tab)
                S = s.reshape(tab)
                Cb = np.broadcast_to(C, tuple(inp[:-1]) + (p // 2,))
                Sb = np.broadcast_to(S, tuple(inp[:-1]) + (p // 2,))
                Y = X.astype(np.float64).copy()
                half = p // 2
                sign = -1.0 if backward else 1.0
                for pair in range(half):
                    ia, ib = (2 * pair, 2 * pair + 1) if layout == 0 else (pair, half + pair)
                    cc = Cb[..., pair].astype(np.float64)
                    ss = Sb[..., pair].astype(np.float64)
                    xa = X[..., ia].astype(np.float64)
                    xb = X[..., ib].astype(np.float64)
                    Y[..., ia] = xa * cc - sign * xb * ss
                    Y[..., ib] = xb * cc + sign * xa * ss
                key = f"ropepre_{ci}_l{layout}_b{backward}"
                g[key + "_x"], g[key + "_cos"], g[key + "_sin"] = X, C, S
                g[key + "_y"] = Y

    # ---- attention --------------------------------------------------------
    # examples/grouped_attention_tensor.rs:74-90: batch 2, m 32, d = dv = 16, scale 0.25,
    # (kv_heads, group, n, causal) in the five reference cases; q = (i%13)/16-0.375,
    # k = (i%17)/16-0.5, v = (i%11)/8-0.5, dy = (i%7)/8-0.25; additive mask (i%5)/32-0.0625
    # when not causal; causal uses query_start = 2^40 + (n-m), key_start = 2^40.
    for (kvh, group, n, causal) in ((3, 1, 32, False), (1, 3, 96, False), (3, 2, 32, False),
                                    (3, 5, 96, False), (3, 3, 96, True)):
        B, M, D = 2, 32, 16
        H = kvh * group
        q = ((np.arange(B * H * M * D) % 13).astype(np.float32) / 16 - 0.375).reshape(B, H, M, D)
        k = ((np.arange(B * kvh * n * D) % 17).astype(np.float32) / 16 - 0.5).reshape(B, kvh, n, D)
        v = ((np.arange(B * kvh * n * D) % 11).astype(np.float32) / 8 - 0.5).reshape(B, kvh, n, D)
        dy = ((np.arange(B * H * M * D) % 7).astype(np.float32) / 8 - 0.25).reshape(B, H, M, D)
        prefix = n - M
        i = np.arange(B * H * M * n)
        if causal:
            mask = np.where(i % n > prefix + (i // n) % M, -np.inf, 0.0).astype(np.float32)
        else:
            mask = ((i % 5).astype(np.float32) / 32 - 0.0625)
        mask = mask.reshape(B, H, M, n)
        tq = torch.tensor(bf16(q), dtype=torch.float64, requires_grad=True)
        tk = torch.tensor(bf16(k), dtype=torch.float64, requires_grad=True)
        tv = torch.tensor(bf16(v), dtype=torch.float64, requires_grad=True)
        kk = tk.repeat_interleave(group, dim=1)
        vv = tv.repeat_interleave(group, dim=1)
        tm = torch.tensor(mask, dtype=torch.float64, requires_grad=True)
        sc = 0.25 * tq @ kk.transpose(-1, -2) + tm
        p = torch.softmax(sc, dim=-1)
        o = p @ vv
        (o * torch.tensor(bf16(dy), dtype=torch.float64)).sum().backward()
        key = f"attn_kv{kvh}_g{group}_n{n}_c{int(causal)}"
        g[key + "_q"], g[key + "_k"], g[key + "_v"], g[key + "_dy"] = q, k, v, dy
        g[key + "_mask"] = mask
        g[key + "_out"] = o.detach().numpy()
        g[key + "_lse"] = torch.logsumexp(sc, dim=-1).detach().numpy()
        g[key + "_dq"] = tq.grad.numpy()
        g[key + "_dk"] = tk.grad.numpy()
        g[key + "_dv"] = tv.grad.numpy()
        if not causal:  # the mask gradient, checked by the reference at grouped_attention_tensor.rs:95
            g[key + "_dmask"] = tm.grad.numpy()

    # examples/attention_tensor.rs:22-66: orthogonal Q (column 0) and K (column 1) give zero
    # scores -> uniform probabilities; closed forms for out, dQ, dK, dV (no BF16 rounding
    # enters: all values are exactly representable and p = 1/n is a power of two).
    for n in (32, 256):
        B, M, D = 2, 32, 16
        scale = 0.25
        q = np.zeros((B, M, D), np.float32)
        k = np.zeros((B, n, D), np.float32)
        v = np.zeros((B, n, D), np.float32)
        dy = np.zeros((B, M, D), np.float32)
        for row in range(M):
            q[:, row, 0] = ((row % 3) - 1.0) * 0.5
            dy[:, row, 0] = ((row % 3) - 1.0) * 0.25
        for col in range(n):
            k[:, col, 1] = ((col % 5) - 2.0) * 0.25
            v[:, col, 0] = ((col % 5) - 2.0) * 0.125
        p = 1.0 / n
        y = np.zeros((B, M, D))
        gq = np.zeros((B, M, D))
        gk = np.zeros((B, n, D))
        gv = np.zeros((B, n, D))
        for b in range(B):
            for row in range(M):
                mean_v = v[b, :, 0].astype(np.float64).sum() * p
                grad = float(dy[b, row, 0])
                y[b, row, 0] = mean_v
                for col in range(n):
                    ds = p * grad * (float(v[b, col, 0]) - mean_v)
                    gq[b, row, 1] += ds * scale * float(k[b, col, 1])
                    gk[b, col, 0] += ds * scale * float(q[b, row, 0])
                    gv[b, col, 0] += p * grad
        key = f"attnkat_orth_n{n}"
        g[key + "_q"], g[key + "_k"], g[key + "_v"], g[key + "_dy"] = q, k, v, dy
        g[key + "_out"], g[key + "_dq"], g[key + "_dk"], g[key + "_dv"] = y, gq, gk, gv

    # examples/causal_attention_tensor.rs:31-55: Q = K = 0, causal with query_start in {0, n-m}:
    # row i averages the first min(qs+i+1, n) values, p = bf16(1/active) exactly as the
    # reference rounds it; dQ = dK = 0.
    for n in (32, 96):
        for cached in (False, True):
            B, M, D = 2, 32, 16
            qs = (n - M) if cached else 0
            v = ((np.arange(B * n * D) % 7).astype(np.float32) / 8 - 0.375).reshape(B, n, D)
            dy = ((np.arange(B * M * D) % 3).astype(np.float32) / 4 - 0.25).reshape(B, M, D)
            y = np.zeros((B, M, D))
            gv = np.zeros((B, n, D))
            for b in range(B):
                for row in range(M):
                    active = min(qs + row + 1, n)
                    prob = float(bf16(np.float32(1.0 / active)))
                    for col in range(active):
                        y[b, row] += prob * v[b, col].astype(np.float64)
                        gv[b, col] += prob * dy[b, row].astype(np.float64)
            key = f"attnkat_causal_n{n}_c{int(cached)}"
            g[key + "_v"], g[key + "_dy"], g[key + "_qs"] = v, dy, np.array(qs)
            g[key + "_out"], g[key + "_dv"] = y, gv
    # causal_attention_tensor.rs:23-30: exact mask bit patterns.
    for ci, (qn, kn, qs, ks) in enumerate(((3, 7, 0, 0), (3, 7, 5, 0), (3, 7, 1 << 40, 1 << 40))):
        mk = np.zeros((2, qn, kn), np.float32)
        for r in range(qn):
            for c in range(kn):
                if ks + c > qs + r:
                    mk[:, r, c] = -np.inf
        g[f"mask_{ci}"] = mk
        g[f"mask_{ci}_spec"] = np.array([2, qn, kn, qs, ks], dtype=np.uint64)

    np.savez_compressed(OUT, **g)
    print(f"wrote {OUT}: {len(g)} arrays, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
