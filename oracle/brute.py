"""Independent float64 loop oracle for slot-indirected causal attention.

TEST INFRASTRUCTURE ONLY. Pure NumPy, explicit loops over requests, query
tokens and heads; meant for small cases (it is O(T * L * Hq * D) in Python).

Semantics (the reference's three ``_slot_based_attention`` branches,
``qwen3_8/full_attention.py:179-283``, collapse to one rule):

* request ``b`` has ``seq_len_b`` tokens in total, of which the last
  ``ext_b`` are new; its prefix is ``P_b = seq_len_b - ext_b``;
* the KV row of context position ``k`` is slot ``req_to_token[row_b, k]`` of the
  pool (slot ids < 0 read slot 0, as the batched branches clamp);
* new token ``t`` (``0 <= t < ext_b``) of request ``b`` attends to context
  positions ``0 .. P_b + t`` inclusive;
* q head ``h`` uses kv head ``h // (Hq // Hkv)``;
* ``out = softmax(scale * q . k) @ v`` over the visible positions.

For ``bsz == 1`` the reference takes ``seq_len`` from ``max_seq_len``; pass
``seq_lens=[max_seq_len]`` for that case.
"""
from __future__ import annotations

import numpy as np


def attention_brute(q, k_pool, v_pool, req_to_token, rows, seq_lens, ext_lens, scale):
    """``q``: ``[T, Hq, D]`` (rows of request 0 first, then request 1, ...);
    ``k_pool``/``v_pool``: ``[S, Hkv, D]``; ``req_to_token``: ``[R, C]`` int;
    ``rows``/``seq_lens``/``ext_lens``: per-request sequences. Returns
    ``[T, Hq, D]`` float64."""
    q = np.asarray(q, dtype=np.float64)
    kp = np.asarray(k_pool, dtype=np.float64)
    vp = np.asarray(v_pool, dtype=np.float64)
    rtt = np.asarray(req_to_token)
    n_tok, n_q, d = q.shape
    n_kv = kp.shape[1]
    group = n_q // n_kv
    out = np.zeros((n_tok, n_q, d), dtype=np.float64)
    base = 0
    for b in range(len(rows)):
        total = int(seq_lens[b])
        ext = int(ext_lens[b])
        prefix = total - ext
        for t in range(ext):
            visible = prefix + t + 1
            for h in range(n_q):
                kvh = h // group
                qv = q[base + t, h]
                scores = np.empty(visible, dtype=np.float64)
                for pos in range(visible):
                    slot = max(int(rtt[rows[b], pos]), 0)
                    scores[pos] = scale * float(np.dot(qv, kp[slot, kvh]))
                top = scores.max()
                w = np.exp(scores - top)
                w /= w.sum()
                acc = np.zeros(d, dtype=np.float64)
                for pos in range(visible):
                    slot = max(int(rtt[rows[b], pos]), 0)
                    acc += w[pos] * vp[slot, kvh]
                out[base + t, h] = acc
        base += ext
    return out


def attention_dense(q, k_pool, v_pool, req_to_token, rows, seq_lens, ext_lens, scale):
    """Same semantics as ``attention_brute`` but vectorised per request in
    float64 (for the mid-sized cases the loop version is too slow for). It is a
    second statement of the rule, checked against ``attention_brute``."""
    q = np.asarray(q, dtype=np.float64)
    kp = np.asarray(k_pool, dtype=np.float64)
    vp = np.asarray(v_pool, dtype=np.float64)
    rtt = np.asarray(req_to_token)
    n_tok, n_q, d = q.shape
    n_kv = kp.shape[1]
    group = n_q // n_kv
    out = np.zeros((n_tok, n_q, d), dtype=np.float64)
    base = 0
    for b in range(len(rows)):
        total = int(seq_lens[b])
        ext = int(ext_lens[b])
        prefix = total - ext
        slots = np.maximum(rtt[rows[b], :total].astype(np.int64), 0)
        keys = kp[slots]                    # [L, Hkv, D]
        vals = vp[slots]
        qb = q[base:base + ext]             # [ext, Hq, D]
        kpos = np.arange(total)[None, :]
        limit = prefix + np.arange(ext)[:, None]
        allowed = kpos <= limit             # [ext, L]
        for h in range(n_q):
            kvh = h // group
            s = scale * (qb[:, h, :] @ keys[:, kvh, :].T)   # [ext, L]
            s = np.where(allowed, s, -np.inf)
            s -= s.max(axis=1, keepdims=True)
            w = np.exp(s)
            w /= w.sum(axis=1, keepdims=True)
            out[base:base + ext, h, :] = w @ vals[:, kvh, :]
        base += ext
    return out
