"""Independent float64 restatement of the token mixers (brute force, numpy).

Written in a different formulation from the C oracle (vectorised, one-pass
delta rule o = decay*S^T q + (q.k) delta, softmax via numpy), so that a
dropped term, wrong sign or transposed index in either one shows up as a
disagreement far above fp32 rounding.  The reference's semantic quirks that
change results (piecewise softplus, conv tap orders, RoPE before the
(1+w) q/k norm, plain-w gated norm, interleaved q|gate, head repeat
vh -> vh // repeat) are reproduced; its fp32 rounding and lane orders are not.
"""
from __future__ import annotations

import ctypes

import numpy as np

_libm = ctypes.CDLL("libm.so.6")
_libm.powf.restype = ctypes.c_float
_libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]


def rope_freqs(half: int, base: float) -> np.ndarray:
    """1/base^(i/half) in fp32 with libm powf, as MathF.Pow computes it
    (Ops.cs:140-142).  A 1-ulp change of a frequency moves the angle at
    position 8192 by ~5e-4 rad, so the frequency must come from powf."""
    return np.array([np.float32(1.0) / np.float32(_libm.powf(np.float32(base),
                                                             np.float32(i) / np.float32(half)))
                     for i in range(half)], np.float32)


def softplus_ref(x):
    """Qwen35Ops.SoftplusScalar (Qwen35Ops.cs:121-142) in float64."""
    x = np.asarray(x, np.float64)
    ex = np.exp(x)
    series = ex - ex ** 2 / 2 + ex ** 3 / 3 - ex ** 4 / 4
    mid = np.where(ex < 0.5, series, np.log1p(ex))
    return np.where(x > 20, x, np.where(x < -10, ex, mid))


def silu(x):
    return x / (1.0 + np.exp(-x))


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def delta_rule(q, k, v, g, beta, state, eps):
    """q,k,v [T][H][D]; g, beta [T][H]; state [H][dk][dv].  l2norm on."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    S = np.array(state, np.float64)
    T, H, D = q.shape
    out = np.zeros((T, H, v.shape[2]))
    for t in range(T):
        qh = q[t] / np.sqrt((q[t] ** 2).sum(-1, keepdims=True) + eps) / np.sqrt(D)
        kh = k[t] / np.sqrt((k[t] ** 2).sum(-1, keepdims=True) + eps)
        dec = np.exp(np.asarray(g[t], np.float64))
        kv = np.einsum("had,ha->hd", S, kh) * dec[:, None]
        delta = np.asarray(beta[t], np.float64)[:, None] * (v[t] - kv)
        sq = np.einsum("had,ha->hd", S, qh) * dec[:, None]
        qk = (qh * kh).sum(-1)
        out[t] = sq + qk[:, None] * delta
        S = S * dec[:, None, None] + kh[:, :, None] * delta[:, None, :]
    return out, S


def gated_norm(x, w, z, eps):
    x = np.asarray(x, np.float64)
    r = 1.0 / np.sqrt((x ** 2).mean(-1, keepdims=True) + eps)
    return x * r * np.asarray(w, np.float64) * silu(np.asarray(z, np.float64))


def split_heads(conv_out, nk, nv, hd):
    """conv_out [..., conv_dim] -> q, k [..., nv, hd] (repeated), v [..., nv, hd]."""
    rep = nv // nk
    key_dim = nk * hd
    q = conv_out[..., :key_dim].reshape(*conv_out.shape[:-1], nk, hd)
    k = conv_out[..., key_dim:2 * key_dim].reshape(*conv_out.shape[:-1], nk, hd)
    v = conv_out[..., 2 * key_dim:].reshape(*conv_out.shape[:-1], nv, hd)
    return np.repeat(q, rep, axis=-2), np.repeat(k, rep, axis=-2), v


def deltanet_decode(qkv, z, b, a, w, conv_state, state, nk, nv, hd, eps=1e-6):
    W = np.asarray(w["conv_w"], np.float64).reshape(4, -1)
    cs = np.asarray(conv_state, np.float64)              # [C][3], index 0 oldest
    x = np.asarray(qkv, np.float64)
    window = np.concatenate([cs, x[:, None]], axis=1)    # [C][4]: tap j <-> window[j]
    conv = silu((W.T * window).sum(1))
    new_cs = window[:, 1:]
    q, k, v = split_heads(conv, nk, nv, hd)
    beta = sigmoid(np.asarray(b, np.float64))
    g = np.asarray(w["ssm_a"], np.float64) * softplus_ref(np.asarray(a, np.float64) +
                                                          np.asarray(w["dt_bias"], np.float64))
    o, S = delta_rule(q[None], k[None], v[None], g[None], beta[None], state, eps)
    y = gated_norm(o[0], w["ssm_norm"], np.asarray(z, np.float64).reshape(nv, hd), eps)
    return y.reshape(-1), new_cs, S, o[0].reshape(-1)


def deltanet_prefill(qkv, z, b, a, w, state, nk, nv, hd, eps=1e-6):
    """T >= 3.  Tap j <-> x[t-j], zero left pad; conv state = last 3 raw rows."""
    W = np.asarray(w["conv_w"], np.float64).reshape(4, -1)
    x = np.asarray(qkv, np.float64)
    T = x.shape[0]
    acc = np.zeros_like(x)
    for j in range(4):
        acc[j:] += W[j][None, :] * x[:T - j]
    conv = silu(acc)
    q, k, v = split_heads(conv, nk, nv, hd)
    beta = sigmoid(np.asarray(b, np.float64))
    g = np.asarray(w["ssm_a"], np.float64)[None] * softplus_ref(
        np.asarray(a, np.float64) + np.asarray(w["dt_bias"], np.float64)[None])
    o, S = delta_rule(q, k, v, g, beta, state, eps)
    y = gated_norm(o, w["ssm_norm"], np.asarray(z, np.float64).reshape(T, nv, hd), eps)
    return y.reshape(T, -1), np.ascontiguousarray(x[T - 3:].T), S, o.reshape(T, -1)


def rope_f64(x, pos, rope_dim, base):
    """x [..., hd] at positions pos (array broadcastable to x[..., 0]).  The
    angle is formed in fp32 as the reference does (Ops.cs:141-152) and the
    rotation in float64."""
    half = rope_dim // 2
    freq = rope_freqs(half, base)
    ang = (np.asarray(pos, np.float32)[..., None] * freq).astype(np.float32).astype(np.float64)
    c, s = np.cos(ang), np.sin(ang)
    y = np.array(x, np.float64)
    x0, x1 = y[..., :half].copy(), y[..., half:2 * half].copy()
    y[..., :half] = x0 * c - x1 * s
    y[..., half:2 * half] = x0 * s + x1 * c
    return y


def rms_zc(x, w, eps):
    x = np.asarray(x, np.float64)
    r = 1.0 / np.sqrt((x ** 2).mean(-1, keepdims=True) + eps)
    return x * r * (1.0 + np.asarray(w, np.float64))


def attn(start, q_gate, k, v, w, cache_k, cache_v, n_heads, n_kv, hd, rope_dim=64, base=1e7,
         eps=1e-6):
    """Returns (out [T][n_heads*hd], K rows, V rows written at start..)."""
    qg = np.asarray(q_gate, np.float64)
    T = qg.shape[0]
    qg = qg.reshape(T, n_heads, 2, hd)
    q, gate = qg[:, :, 0], qg[:, :, 1]
    pos = start + np.arange(T)
    q = rms_zc(rope_f64(q, pos[:, None], rope_dim, base), w["q_norm"], eps)
    kn = rms_zc(rope_f64(np.asarray(k, np.float64).reshape(T, n_kv, hd), pos[:, None],
                         rope_dim, base), w["k_norm"], eps)
    K = np.array(cache_k, np.float64)[:start + T].reshape(start + T, n_kv, hd)
    V = np.array(cache_v, np.float64)[:start + T].reshape(start + T, n_kv, hd)
    K[start:] = kn
    V[start:] = np.asarray(v, np.float64).reshape(T, n_kv, hd)
    group = n_heads // n_kv
    out = np.zeros((T, n_heads, hd))
    for h in range(n_heads):
        kvh = h // group
        s = q[:, h] @ K[:, kvh].T / np.sqrt(hd)           # [T][kvLen]
        mask = np.arange(start + T)[None, :] <= pos[:, None]
        s = np.where(mask, s, -np.inf)
        p = np.exp(s - s.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        out[:, h] = p @ V[:, kvh]
    out = out * sigmoid(gate)
    return out.reshape(T, -1), K.reshape(start + T, -1)[start:], V.reshape(start + T, -1)[start:]
