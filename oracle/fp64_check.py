"""Independent FP64, non-streaming restatement of Piper Attention's recurrence.

TEST INFRASTRUCTURE ONLY (imported by ``tests/`` as a checker of the checker).

The streaming FP32 loop of ``reference.py:76-117`` is, algebraically,

    out_i = sum_t w_ti * (u_t @ v_t)_i / 255  /  sum_t w_ti * sum_k p_tik  +  mean

with per-64-key-block probabilities ``p_tik = exp(s_ik - bm_ti)``, block maxima
``bm_ti = max_k (s_ik + ln vs_k)``, codes ``u_tik = rint(p_tik * vs_k * 255)`` and
block weights ``w_ti = exp(bm_ti - M_i)`` with ``M_i = max_t bm_ti``.  This module
evaluates that closed form directly in FP64 -- no running maximum, no old/current
weights, no rescaled numerator -- so a dropped rescale, a wrong weight or a swapped
operand in the streaming oracle shows up as a disagreement.  Codes can differ from
the FP32 loop only where ``p * vs * 255`` lies within FP32 rounding of a half
integer, so agreement is expected to about 1e-4 relative, not bit for bit.
"""

from __future__ import annotations

import numpy as np

BLOCK = 64


def attention_fp64(prepared: dict, scale: float, is_causal: bool) -> np.ndarray:
    q = prepared["query_code"].astype(np.float64)
    k = prepared["key_code"].astype(np.float64)
    v = prepared["value_code"].astype(np.float64)
    qs = prepared["query_scale"].astype(np.float64)
    ks = prepared["key_scale"].astype(np.float64)
    vs = prepared["value_scale"].astype(np.float64)
    mean = prepared["value_mean"].astype(np.float64)
    batch, heads, sq, width = q.shape
    sk = k.shape[2]
    n_blocks = -(-sk // BLOCK)
    out = np.empty((batch, heads, sq, width))
    for b in range(batch):
        for h in range(heads):
            # full score matrix, then cut into blocks
            s = (q[b, h] @ k[b, h].T) * qs[b, h][:, None] * ks[b, h][None, :] * scale
            if is_causal:
                s[np.arange(sk)[None, :] > np.arange(sq)[:, None]] = -np.inf
            shifted = s + np.log(vs[b, h])[None, :]
            block_max = np.stack(
                [shifted[:, t * BLOCK : (t + 1) * BLOCK].max(axis=1) for t in range(n_blocks)], axis=1
            )  # [sq, n_blocks]
            overall = block_max.max(axis=1)  # [sq]
            num = np.zeros((sq, width))
            den = np.zeros(sq)
            for t in range(n_blocks):
                cols = slice(t * BLOCK, min((t + 1) * BLOCK, sk))
                bm = block_max[:, t]
                finite = np.isfinite(bm)
                with np.errstate(invalid="ignore"):
                    p = np.where(finite[:, None], np.exp(s[:, cols] - bm[:, None]), 0.0)
                    weight = np.where(finite, np.exp(bm - overall), 0.0)
                p = np.nan_to_num(p)
                u = np.clip(np.rint(p * vs[b, h, cols][None, :] * 255.0), 0.0, 255.0)
                num += weight[:, None] * (u @ v[b, h, cols]) / 255.0
                den += weight * p.sum(axis=1)
            out[b, h] = num / np.maximum(den, 1e-30)[:, None] + mean[b, h][None, :]
    return out


def single_tile_zero_query(v_code, v_scale, v_mean) -> np.ndarray:
    """Closed form for Q == 0 and at most 64 keys (one block), non-causal.

    All scores are 0, so ``bm = max_k ln vs_k = ln vs_max``, ``p_k = 1 / vs_max`` for every
    key, ``u_k = rint(255 * vs_k / vs_max)`` and the output row (the same for every query) is
    ``vs_max * sum_k u_k v_k / (255 * n) + mean``.
    Arguments are one head: ``v_code [n, D]``, ``v_scale [n]``, ``v_mean [D]``.
    """
    vs = v_scale.astype(np.float64)
    n = vs.shape[0]
    vs_max = vs.max()
    u = np.clip(np.rint(255.0 * vs / vs_max), 0.0, 255.0)
    return vs_max * (u @ v_code.astype(np.float64)) / (255.0 * n) + v_mean.astype(np.float64)
