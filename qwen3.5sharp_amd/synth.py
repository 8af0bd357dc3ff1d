"""Seeded synthetic inputs for the token-mixer workloads.

One generator serves every consumer (parity tests, fixtures, bench): the
splitmix64 sequence seeded with ``0x51355000 + tensor_id``, 24-bit uniforms,
and Box-Muller normals.  Element i of a stream is the (i+1)-th splitmix64
output, so the generator is counter-based and vectorises in numpy.

The tensor ids and distributions below describe the workloads:

* Gated-DeltaNet layer: 16 k-heads, 32 v-heads, dk = dv = 128, conv kernel 4,
  conv_dim = 8192.  qkv ~N(0,1); conv weights ~N(0,0.5); conv state ~N(0,1)
  drawn as [3][conv_dim] and stored channel-major (cs[c*3+j]); b, a ~N(0,1);
  dt_bias ~N(0,0.1); A_log ~U(0,2.3) passed as ssm_a = -exp(A_log); z ~N(0,1);
  ssm_norm = 1+N(0,0.02); prior state ~N(0,0.1).
* Gated GQA layer: 16 q heads, 4 KV heads, head_dim 256, partial RoPE over 64
  dims (base 1e7); q|gate, k, v ~N(0,1); q_norm, k_norm = 1+N(0,0.02);
  pre-filled KV rows ~N(0,1).
"""
from __future__ import annotations

import numpy as np

SEED_BASE = 0x51355000
_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """Outputs offset+1 .. offset+n of splitmix64 started at ``seed``."""
    with np.errstate(over="ignore"):
        i = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + i * _GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        z = z ^ (z >> np.uint64(31))
    return z


def uniform(tensor_id: int, n: int, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
    """fp32 uniforms on [lo, hi) from the top 24 bits of each output."""
    u = (splitmix64(SEED_BASE + tensor_id, n) >> np.uint64(40)).astype(np.float64)
    u *= 1.0 / (1 << 24)
    return (lo + (hi - lo) * u).astype(np.float32)


def normal(tensor_id: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """fp32 normals by Box-Muller over consecutive uniform pairs (u1 in (0,1])."""
    pairs = (n + 1) // 2
    z = splitmix64(SEED_BASE + tensor_id, 2 * pairs) >> np.uint64(40)
    u1 = (z[0::2].astype(np.float64) + 1.0) * (1.0 / (1 << 24))
    u2 = z[1::2].astype(np.float64) * (1.0 / (1 << 24))
    r = np.sqrt(-2.0 * np.log(u1))
    out = np.empty(2 * pairs, dtype=np.float64)
    out[0::2] = r * np.cos(2.0 * np.pi * u2)
    out[1::2] = r * np.sin(2.0 * np.pi * u2)
    return (mean + std * out[:n]).astype(np.float32)


# Tensor ids (stable: fixtures and bench lines record them).
ID_QKV, ID_CONV_W, ID_CONV_STATE, ID_B, ID_A, ID_DT_BIAS, ID_A_LOG, ID_Z, ID_SSM_NORM, \
    ID_STATE = range(1, 11)
ID_QGATE, ID_K, ID_V, ID_Q_NORM, ID_K_NORM, ID_CACHE_K, ID_CACHE_V = range(11, 18)


def deltanet_weights(n_k_heads: int, n_v_heads: int, hd: int, conv_kernel: int = 4,
                     salt: int = 0) -> dict:
    """conv_w [K][conv_dim], ssm_a = -exp(A_log), dt_bias, ssm_norm."""
    conv_dim = 2 * n_k_heads * hd + n_v_heads * hd
    s = salt * 1000
    a_log = uniform(ID_A_LOG + s, n_v_heads, 0.0, 2.3)
    return {
        "conv_w": normal(ID_CONV_W + s, conv_kernel * conv_dim, 0.0, 0.5),
        "ssm_a": (-np.exp(a_log.astype(np.float64))).astype(np.float32),
        "dt_bias": normal(ID_DT_BIAS + s, n_v_heads, 0.0, 0.1),
        "ssm_norm": normal(ID_SSM_NORM + s, hd, 1.0, 0.02),
    }


def deltanet_inputs(T: int, n_k_heads: int, n_v_heads: int, hd: int, salt: int = 0) -> dict:
    """Projection outputs for T tokens: qkv [T][conv_dim], z, b, a."""
    conv_dim = 2 * n_k_heads * hd + n_v_heads * hd
    s = salt * 1000
    return {
        "qkv": normal(ID_QKV + s, T * conv_dim).reshape(T, conv_dim),
        "z": normal(ID_Z + s, T * n_v_heads * hd).reshape(T, n_v_heads * hd),
        "b": normal(ID_B + s, T * n_v_heads).reshape(T, n_v_heads),
        "a": normal(ID_A + s, T * n_v_heads).reshape(T, n_v_heads),
    }


def deltanet_state(n_k_heads: int, n_v_heads: int, hd: int, conv_kernel: int = 4,
                   salt: int = 0) -> dict:
    """Prior recurrent state [H][dk][dv] ~N(0,0.1) and conv state [conv_dim][K-1]."""
    conv_dim = 2 * n_k_heads * hd + n_v_heads * hd
    s = salt * 1000
    logical = normal(ID_CONV_STATE + s, (conv_kernel - 1) * conv_dim).reshape(conv_kernel - 1,
                                                                              conv_dim)
    return {
        "state": normal(ID_STATE + s, n_v_heads * hd * hd, 0.0, 0.1).reshape(n_v_heads, hd, hd),
        "conv_state": np.ascontiguousarray(logical.T),
    }


def attn_weights(head_dim: int, salt: int = 0) -> dict:
    s = salt * 1000
    return {
        "q_norm": normal(ID_Q_NORM + s, head_dim, 1.0, 0.02),
        "k_norm": normal(ID_K_NORM + s, head_dim, 1.0, 0.02),
    }


def attn_inputs(T: int, n_heads: int, n_kv_heads: int, head_dim: int, salt: int = 0) -> dict:
    """q|gate [T][2*n_heads*head_dim] (interleaved per head), k, v [T][kv_dim]."""
    s = salt * 1000
    kv_dim = n_kv_heads * head_dim
    return {
        "q_gate": normal(ID_QGATE + s, T * 2 * n_heads * head_dim).reshape(T, -1),
        "k": normal(ID_K + s, T * kv_dim).reshape(T, kv_dim),
        "v": normal(ID_V + s, T * kv_dim).reshape(T, kv_dim),
    }


def kv_prefill(n_pos: int, kv_dim: int, salt: int = 0) -> tuple:
    """Cache rows 0..n_pos-1 ~N(0,1) for K and V (treated as already RoPE'd/normed)."""
    s = salt * 1000
    k = normal(ID_CACHE_K + s, n_pos * kv_dim).reshape(n_pos, kv_dim)
    v = normal(ID_CACHE_V + s, n_pos * kv_dim).reshape(n_pos, kv_dim)
    return k, v


QBLOCK_BYTES = {1: 42, 2: 130, 4: 144, 5: 176, 6: 210, 14: 136}
QBLOCK_VALUES = {1: 256, 2: 512, 4: 256, 5: 256, 6: 256, 14: 256}


def quant_weights(qtype: int, n_out: int, n_in: int, salt: int = 0) -> np.ndarray:
    """GGUF STQ1_0 (qtype 1), Q2_0C (2), Q4_K (4), Q5_K (5), Q6_K (6) or
    IQ4_XS (14) rows [n_out][n_in / block values] as bytes: every quant byte
    uniform, the fp16 block scales in [0.004, 0.02] (finite, the size trained
    weights have; for IQ4_XS a twentieth of that, its sub-block scales
    reaching 31)."""
    nblk = n_out * (n_in // QBLOCK_VALUES[qtype])
    nb = QBLOCK_BYTES[qtype]
    raw = splitmix64(SEED_BASE + 300 + 10 * qtype + salt, (nblk * nb + 7) // 8)
    b = raw.view(np.uint8)[:nblk * nb].reshape(nblk, nb).copy()
    d = uniform(301 + 10 * qtype + salt, nblk, 0.004, 0.02).astype(np.float16)
    if qtype in (4, 5):
        b[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
        b[:, 2:4] = uniform(302 + 10 * qtype + salt, nblk, 0.004, 0.02).astype(np.float16) \
            .view(np.uint8).reshape(-1, 2)
    elif qtype == 14:
        b[:, 0:2] = (d * np.float16(0.05)).view(np.uint8).reshape(-1, 2)
    elif qtype == 2:
        b[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    elif qtype == 1:
        b[:, 40:42] = d.view(np.uint8).reshape(-1, 2)
    else:
        b[:, 208:210] = d.view(np.uint8).reshape(-1, 2)
    return b.ravel()
