"""numpy fp32 decode attention -- test infrastructure only.

Restates the reference's ground truth:

* ``default_sm_scale`` / ``expand_kv`` -- ``reference.py:44-53``;
* ``reference_decode_attention`` -- ``reference.py:61-88``: scores
  ``q . k * sm_scale`` in fp32, softmax over the history, ``probs . v``;
* ``reference_grouped`` -- ``l2_sweep.py:196-236``: the same arithmetic with q
  viewed as ``(B, HKV, G, D)`` so K/V are never expanded, history visited in
  chunks (used for the large configurations);
* ``reference_decode_attention_f64`` -- float64 brute force, used to pin the
  fp32 versions on tiny inputs.

Ragged batches: ``seq_lens`` (one length per batch row) restricts batch row b to
its first ``seq_lens[b]`` tokens -- the reference has one S for the whole batch
(``kernels/fused_decode_attn.py:469``); per-row lengths are the extension the
70B-style benchmark configuration needs.
"""

from __future__ import annotations

import math

import numpy as np


def default_sm_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)


def expand_kv(x: np.ndarray, n_rep: int) -> np.ndarray:
    """(B, HKV, S, D) -> (B, HKV*n_rep, S, D), each KV head repeated n_rep times."""
    if n_rep == 1:
        return x
    return np.repeat(x, n_rep, axis=1)


def _softmax_last(x: np.ndarray) -> np.ndarray:
    m = x.max(axis=-1, keepdims=True)
    e = np.exp(x - m)
    return e / e.sum(axis=-1, keepdims=True)


def reference_decode_attention(q, k, v, sm_scale=None) -> np.ndarray:
    """fp32 single-step attention, ``reference.py:61-88``.

    q: (B, HQ, D); k, v: (B, HKV, S, D).  Returns (B, HQ, D) float32.
    """
    B, HQ, D = q.shape
    HKV = k.shape[1]
    if HQ % HKV:
        raise ValueError(f"HQ={HQ} must be a multiple of HKV={HKV}")
    n_rep = HQ // HKV
    sm = np.float32(default_sm_scale(D) if sm_scale is None else sm_scale)
    qf = np.asarray(q, dtype=np.float32)
    kf = expand_kv(np.asarray(k, dtype=np.float32), n_rep)
    vf = expand_kv(np.asarray(v, dtype=np.float32), n_rep)
    scores = np.matmul(kf, qf[..., None])[..., 0] * sm          # (B, HQ, S)
    probs = _softmax_last(scores).astype(np.float32)
    return np.matmul(probs[:, :, None, :], vf)[:, :, 0, :].astype(np.float32)


def reference_grouped(q, k_rows, v_rows, S: int, HKV: int, sm_scale=None,
                      chunk: int = 32768, seq_lens=None) -> np.ndarray:
    """Memory-frugal fp32 attention, ``l2_sweep.py:196-236``.

    ``k_rows(s, e)`` / ``v_rows(s, e)`` return fp32 ``(B, HKV, e-s, D)`` for the
    token range ``[s, e)`` (so a quantized cache is dequantized one chunk at a
    time).  ``seq_lens`` masks each batch row to its own length.
    """
    B, HQ, D = q.shape
    g = HQ // HKV
    sm = np.float32(default_sm_scale(D) if sm_scale is None else sm_scale)
    qg = np.asarray(q, dtype=np.float32).reshape(B, HKV, g, D)
    bounds = [(s, min(S, s + chunk)) for s in range(0, S, chunk)]
    scores = np.concatenate(
        [np.einsum("bhgd,bhsd->bhgs", qg, k_rows(s, e)) for s, e in bounds], axis=-1
    ) * sm
    if seq_lens is not None:
        pos = np.arange(S)[None, None, None, :]
        lens = np.asarray(seq_lens).reshape(B, 1, 1, 1)
        scores = np.where(pos < lens, scores, -np.inf)
    probs = _softmax_last(scores).astype(np.float32)
    out = np.zeros((B, HKV, g, D), dtype=np.float32)
    for s, e in bounds:
        out += np.einsum("bhgs,bhsd->bhgd", probs[..., s:e], v_rows(s, e))
    return out.reshape(B, HQ, D)


def reference_decode_attention_f64(q, k, v, sm_scale=None, seq_lens=None) -> np.ndarray:
    """Float64 brute force (explicit loops over heads), for tiny inputs."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B, HQ, D = q.shape
    HKV, S = k.shape[1], k.shape[2]
    g = HQ // HKV
    sm = default_sm_scale(D) if sm_scale is None else sm_scale
    out = np.zeros((B, HQ, D))
    for b in range(B):
        n = S if seq_lens is None else int(seq_lens[b])
        for h in range(HQ):
            kv = h // g
            s = np.array([float(np.dot(q[b, h], k[b, kv, t])) * sm for t in range(n)])
            w = np.exp(s - s.max())
            w /= w.sum()
            out[b, h] = (w[:, None] * v[b, kv, :n]).sum(axis=0)
    return out


def metrics(got, ref) -> dict:
    """cosine / max-abs / mean-abs / rel-L2, as ``test_correctness.py:62-70``."""
    g = np.asarray(got, dtype=np.float64).ravel()
    r = np.asarray(ref, dtype=np.float64).ravel()
    d = g - r
    denom = max(np.linalg.norm(r), 1e-12)
    cos = float(np.dot(g, r) / max(np.linalg.norm(g) * np.linalg.norm(r), 1e-12))
    return {
        "cosine": cos,
        "max_abs_err": float(np.abs(d).max()) if d.size else 0.0,
        "mean_abs_err": float(np.abs(d).mean()) if d.size else 0.0,
        "rel_l2": float(np.linalg.norm(d) / denom),
    }
