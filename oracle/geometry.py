"""Decode-step geometry restated on the CPU (TEST INFRASTRUCTURE ONLY —
see oracle/__init__.py).

The reference builds per-step index tensors in torch
(engine/pyengine/model.py:827-887): the SWA ring map and the padded global
gather. The HIP decode kernel recomputes the same predicates in-kernel from
ctx_lens; these helpers state them for the tests.
"""
import numpy as np


def ring_positions(n, window):
    """decode_batch_ctx #1 (model.py:842-848): ring slot s of a sequence
    holding n tokens holds position p = base + ((s - base) mod W),
    base = max(0, n - W); the slot is live iff p < n."""
    s = np.arange(window)
    base = max(0, n - window)
    p = base + ((s - base) % window)
    return p, p < n


def global_valid(n, L):
    """decode_batch_ctx #2 (model.py:849-857): padded key column j < L is
    live iff j < n; its page index is j // 16, offset j % 16."""
    j = np.arange(L)
    return j // 16, j % 16, j < n


def visible_range(n, window):
    """Keys the decode kernel visits: positions [lo, n),
    lo = max(0, n - W) on windowed layers (attn_swa.py:83-85)."""
    lo = max(0, n - window) if window else 0
    return lo, n


def bucket_len(max_pos, hiwater, bucket=512, cap=None):
    """GraphRunner.step_enqueue #2 (engine/pyengine/graphrun.py:339-343):
    monotone high-water bucket of the padded key length."""
    L = -(-(max_pos + 1) // bucket) * bucket
    L = max(L, hiwater)
    return min(L, cap) if cap is not None else L
