"""Independent numpy restatement of the same reference steps as ts_oracle.c.

TEST INFRASTRUCTURE ONLY.  It exists to cross-check the C oracle on tiny inputs: it is
written separately (vectorised numpy, float64 where the reference accumulates in f64), so a
dropped term, wrong index or transposed operand in either one shows up as a mismatch.

References (relative to the reference repository root):
  quantize   src/backend/bindless/test_int4_parity.rs:56-75 (round half away from zero is
             computed in float64 on the exact f32 quotient, not with np.round, which rounds
             half to even)
  dequantize src/backend/bindless/test_int4_parity.rs:78-87
  rotation   src/ops/reference/rope.rs:180-197
  attention  src/ops/reference/attention.rs:236-313, matmul.rs:91-104, softmax.rs:91-129
"""
from __future__ import annotations

import numpy as np


def quantize(x: np.ndarray):
    """x: [..., hd] float32 -> (scale [...] f32, words [..., hd/8] u32)."""
    x = np.asarray(x, np.float32)
    with np.errstate(invalid="ignore"):
        max_abs = np.fmax.reduce(np.abs(x), axis=-1, initial=np.float32(0.0)).astype(np.float32)
    scale = np.where(max_abs == 0, np.float32(1.0), max_abs / np.float32(7.0)).astype(np.float32)
    with np.errstate(invalid="ignore", divide="ignore"):
        quot = (x / scale[..., None]).astype(np.float32).astype(np.float64)
    r = np.sign(quot) * np.floor(np.abs(quot) + 0.5)
    r = np.where(np.isnan(r), 0.0, r)
    q = np.clip(r + 8, 1, 15).astype(np.uint32)
    q = q.reshape(*x.shape[:-1], x.shape[-1] // 8, 8)
    shifts = (np.arange(8, dtype=np.uint32) * 4)
    words = np.bitwise_or.reduce(q << shifts, axis=-1).astype(np.uint32)
    return scale, words


def dequantize(words: np.ndarray, scale: np.ndarray) -> np.ndarray:
    words = np.asarray(words, np.uint32)
    nib = (words[..., None] >> (np.arange(8, dtype=np.uint32) * 4)) & 0xF
    nib = nib.reshape(*words.shape[:-1], words.shape[-1] * 8)
    return ((nib.astype(np.float32) - np.float32(8.0)) * np.asarray(scale, np.float32)[..., None]).astype(np.float32)


def rotate(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """x [..., hd] f32; cos/sin [..., rope_dim/2] f32 broadcastable."""
    x = np.asarray(x, np.float32).copy()
    n = cos.shape[-1]
    a = x[..., 0:2 * n:2].copy()
    b = x[..., 1:2 * n:2].copy()
    x[..., 0:2 * n:2] = (a * cos).astype(np.float32) - (b * sin).astype(np.float32)
    x[..., 1:2 * n:2] = (a * sin).astype(np.float32) + (b * cos).astype(np.float32)
    return x


def attend(q: np.ndarray, k: np.ndarray, v: np.ndarray, q_pos0: int, softcap: float = 0.0):
    """One sequence.  q: [T, n_head, hd] (already rotated), k/v: [key_len, n_kv, hd]
    (dequantized).  Query t sits at absolute position q_pos0+t and sees keys 0..q_pos0+t."""
    T, n_head, hd = q.shape
    key_len, n_kv, _ = k.shape
    group = n_head // n_kv
    out = np.zeros((T, n_head, hd), np.float32)
    scl = np.float32(np.float32(1.0) / np.sqrt(np.float32(hd)))
    for h in range(n_head):
        kv = h // group
        prod = (q[:, h, None, :] * k[None, :, kv, :]).astype(np.float32)  # [T, L, hd] f32 products
        s = prod.astype(np.float64).sum(-1).astype(np.float32) * scl
        if softcap > 0:
            s = (np.tanh(s / np.float32(softcap)) * np.float32(softcap)).astype(np.float32)
        qpos = q_pos0 + np.arange(T)[:, None]
        s = np.where(np.arange(key_len)[None, :] > qpos, -np.inf, s).astype(np.float32)
        e = np.exp(s - s.max(-1, keepdims=True)).astype(np.float32)
        tot = e.astype(np.float64).sum(-1, keepdims=True)
        p = (e * (1.0 / tot).astype(np.float32)).astype(np.float32)
        pv = (p[:, :, None] * v[None, :, kv, :]).astype(np.float32)
        out[:, h, :] = pv.astype(np.float64).sum(1).astype(np.float32)
    return out
