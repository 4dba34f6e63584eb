"""Attention inputs whose scores rise (or fall) across 64-key tiles, and a replay of the fused
forward kernel's lagging-max rule on them (test infrastructure, numpy only).

The fused forward (hk_attention.hip, tile_softmax) keeps a per-query running max m that may lag
the true max by up to 8 base-2 units: O, l and m are rescaled only when some query of a wave's
32 sees its tile max exceed m + 8. N(0,1) inputs almost never trigger that after the first tile,
so these inputs put Q along one direction and K along the same direction with a magnitude that
grows with the key position: query i's base-2 score against key j is about
rate_i * j / 64, with rate_i chosen per 32-query wave (times a per-query factor in
[0.75, 1.25]):

* "jump": 12 per 64-key tile (every tile rescales);
* "creep": 3 per tile (the max crosses the lag bound every third tile or so);
* "descending": -5 per tile (the first tile holds the max; no later rescale);
* "extreme": 90 per tile (|scale * s| reaches ~1e3 in natural units over 1024 keys).

Noise of std 0.5 on the other components of Q and on every component of K makes the scores
jitter within each tile, so the maxima are not at tile ends only. Everything is rounded to BF16 (the oracle sees the same bits).
"""
import numpy as np

import oracle

PATTERNS = {"jump": 12.0, "creep": 3.0, "descending": -5.0, "extreme": 90.0}
WAVE_ROWS = 32   # queries per wave in both forward kernels
TILE_KEYS = 64   # keys per K/V tile
STALE_MAX = 8.0  # base-2 lag allowed before a rescale (kStaleMax)
LOG2E = 1.4426950408889634


def rising_inputs(batch, heads, kv_heads, m, n, d, seed, patterns=("jump", "creep", "descending", "extreme"),
                  key_step=8.0):
    """q [B,Hq,M,D], k/v [B,Hkv,N,D], do [B,Hq,M,D] float32 holding BF16 values, plus the per-row
    pattern names. Query wave w (rows 32w..32w+31) of every head uses patterns[w % len]; the
    K ramp is key_step per 64 keys along direction e_0."""
    scale = d ** -0.5
    c = scale * LOG2E
    q = oracle.normal((batch, heads, m, d), seed, 1, std=0.5)
    k = oracle.normal((batch, kv_heads, n, d), seed, 2, std=0.5)
    v = oracle.normal((batch, kv_heads, n, d), seed, 3)
    do = oracle.normal((batch, heads, m, d), seed, 4)
    jitter = np.clip(1.0 + 0.2 * oracle.normal((batch, heads, m), seed, 5), 0.75, 1.25)
    names = [patterns[(i // WAVE_ROWS) % len(patterns)] for i in range(m)]
    rate = np.array([PATTERNS[p] for p in names], dtype=np.float64)
    # base-2 score of (i, j) ~ c * a_i * b_j with b_j = key_step * j / 64 -> rate_i = c * a_i * key_step
    a = rate[None, None, :] / (c * key_step) * jitter
    q[..., 0] = a.astype(np.float32)  # the rate itself: no noise along e_0 on the query side
    k[..., 0] += (key_step * np.arange(n) / TILE_KEYS).astype(np.float32)[None, None, :]
    return (oracle.bf16_round(q), oracle.bf16_round(k), oracle.bf16_round(v), oracle.bf16_round(do), names)


def base2_scores(q, k, scale, causal, query_start=0, key_start=0):
    """c * Q K^T per (b, h) in float64 with masked keys at -inf; GQA by head index."""
    B, H, M, D = q.shape
    hkv = k.shape[1]
    s = np.einsum("bhmd,bhnd->bhmn", q.astype(np.float64),
                  np.repeat(k.astype(np.float64), H // hkv, axis=1)) * (abs(scale) * LOG2E)
    if causal:
        i = np.arange(M)[:, None] + query_start
        j = np.arange(k.shape[2])[None, :] + key_start
        s = np.where(j > i, -np.inf, s)
    return s


def rescale_counts(scores):
    """Replays the kernel's rule on base-2 scores [.., M, N]: tiles of 64 keys in ascending
    order, queries in waves of 32 (aligned), a wave rescales when any of its queries' tile max
    exceeds its running max + STALE_MAX, every query then taking max(m, tile max). Returns the
    number of rescales after the first one, per query (a rescale that lowers nothing -- a query
    whose own max did not grow -- is not counted)."""
    *lead, M, N = scores.shape
    s = scores.reshape(-1, M, N)
    counts = np.zeros(s.shape[:2], dtype=np.int64)
    ntiles = (N + TILE_KEYS - 1) // TILE_KEYS
    for w0 in range(0, M, WAVE_ROWS):
        blk = s[:, w0:w0 + WAVE_ROWS]
        m_run = np.full(blk.shape[:2], -np.inf)
        for j in range(ntiles):
            mt = blk[:, :, j * TILE_KEYS:(j + 1) * TILE_KEYS].max(axis=2)
            if np.all(np.isneginf(mt)):
                continue  # the wave skips a tile none of its queries sees
            trig = np.any(mt > m_run + STALE_MAX, axis=1)
            grow = trig[:, None] & (mt > m_run)
            counts[:, w0:w0 + WAVE_ROWS] += grow & np.isfinite(m_run)
            m_run = np.where(trig[:, None], np.maximum(m_run, mt), m_run)
    return counts.reshape(*lead, M)


def lagging_softmax_f64(scores, v, bug=None):
    """O = softmax(scores) V (scores in base 2, [M, N]; v [N, Dv]) evaluated the way the kernel
    does it: tile by tile with the lagging running max above, in float64. `bug` plants a mistake
    in the rescale: "keep_l" (l not multiplied by alpha), "keep_o" (O not multiplied), "alpha_inv"
    (the reciprocal factor). Returns (O, lse in natural units)."""
    M, N = scores.shape
    o = np.zeros((M, v.shape[1]))
    l_run = np.zeros(M)
    m_run = np.full(M, -np.inf)
    for w0 in range(0, M, WAVE_ROWS):
        rows = slice(w0, w0 + WAVE_ROWS)
        for j0 in range(0, N, TILE_KEYS):
            st = scores[rows, j0:j0 + TILE_KEYS]
            mt = st.max(axis=1)
            if np.all(np.isneginf(mt)):
                continue
            if np.any(mt > m_run[rows] + STALE_MAX):
                m_new = np.maximum(m_run[rows], mt)
                with np.errstate(invalid="ignore"):
                    alpha = np.where(np.isneginf(m_new), 1.0, np.exp2(m_run[rows] - m_new))
                if bug == "alpha_inv":
                    alpha = np.where(alpha > 0, 1.0 / np.where(alpha > 0, alpha, 1.0), 0.0)
                m_run[rows] = m_new
                if bug != "keep_l":
                    l_run[rows] *= alpha
                if bug != "keep_o":
                    o[rows] *= alpha[:, None]
            neg_m = np.where(np.isneginf(m_run[rows]), 0.0, -m_run[rows])
            p = np.exp2(st + neg_m[:, None])
            l_run[rows] += p.sum(axis=1)
            o[rows] += p @ v[j0:j0 + TILE_KEYS]
    with np.errstate(divide="ignore", invalid="ignore"):
        out = np.where(l_run[:, None] > 0, o / np.where(l_run > 0, l_run, 1.0)[:, None], 0.0)
        lse = np.where(l_run > 0, (m_run + np.log2(np.where(l_run > 0, l_run, 1.0))) / LOG2E, -np.inf)
    return out, lse
