"""numpy front end of the CPU oracle (libq35oracle.so).

TEST INFRASTRUCTURE ONLY: tests/ use it as the parity checker and bench.py's
cpu_baseline leg times it.  The product library never imports it.  Each
function forwards to the C restatement in q35_oracle.c, which cites the
reference file:line it follows.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libq35oracle.so")
_lib = None

F = ctypes.POINTER(ctypes.c_float)


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
    return _lib


class Dims(ctypes.Structure):
    _fields_ = [("n_k_heads", ctypes.c_int), ("n_v_heads", ctypes.c_int),
                ("head_k_dim", ctypes.c_int), ("conv_kernel", ctypes.c_int),
                ("n_heads", ctypes.c_int), ("n_kv_heads", ctypes.c_int),
                ("head_dim", ctypes.c_int), ("rope_dim", ctypes.c_int),
                ("rope_base", ctypes.c_float), ("eps", ctypes.c_float)]


def dims(n_k_heads=16, n_v_heads=32, head_k_dim=128, conv_kernel=4, n_heads=16, n_kv_heads=4,
         head_dim=256, rope_dim=64, rope_base=1e7, eps=1e-6) -> Dims:
    return Dims(n_k_heads, n_v_heads, head_k_dim, conv_kernel, n_heads, n_kv_heads, head_dim,
                rope_dim, rope_base, eps)


def _p(a: np.ndarray):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags.c_contiguous, (a.dtype, a.flags)
    return a.ctypes.data_as(F)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


# ---- scalar helpers ------------------------------------------------------

def silu(x: float) -> float:
    lib().q35o_silu.restype = ctypes.c_float
    return lib().q35o_silu(ctypes.c_float(x))


def softplus(x: float) -> float:
    lib().q35o_softplus.restype = ctypes.c_float
    return lib().q35o_softplus(ctypes.c_float(x))


def log1p_safe(x: float) -> float:
    lib().q35o_log1p_safe.restype = ctypes.c_float
    return lib().q35o_log1p_safe(ctypes.c_float(x))


def fast_exp(x) -> np.ndarray:
    x = _f32(x)
    y = np.empty_like(x)
    lib().q35o_fast_exp_n(_p(x), _p(y), x.size)
    return y


def sigmoid(x) -> np.ndarray:
    x = _f32(x)
    y = np.empty_like(x)
    lib().q35o_sigmoid(_p(x), _p(y), x.size)
    return y


# ---- DeltaNet ops --------------------------------------------------------

def causal_conv1d(inp, kernel, kernel_size, channels, seq):
    inp, kernel = _f32(inp), _f32(kernel)
    out = np.empty(channels * seq, np.float32)
    lib().q35o_causal_conv1d(_p(inp), _p(kernel), kernel_size, channels, seq, _p(out))
    return out.reshape(channels, seq)


def causal_conv1d_update(inp, kernel, kernel_size, channels, conv_state):
    """Returns (out, new_conv_state); conv_state is not modified."""
    inp, kernel = _f32(inp), _f32(kernel)
    cs = _f32(conv_state).copy()
    out = np.empty(channels, np.float32)
    lib().q35o_causal_conv1d_update(_p(inp), _p(kernel), kernel_size, channels, _p(cs), _p(out))
    return out, cs


def recurrent_gated_delta_rule(q, k, v, g, beta, state, tokens, n_heads, head_dim, v_head_dim,
                               eps, l2norm_qk=True):
    """Returns (out [tokens][n_heads][v_head_dim], new_state)."""
    q, k, v, g, beta = map(_f32, (q, k, v, g, beta))
    st = _f32(state).copy()
    out = np.empty(tokens * n_heads * v_head_dim, np.float32)
    lib().q35o_recurrent_gated_delta_rule(_p(q), _p(k), _p(v), _p(g), _p(beta), _p(st), tokens,
                                          n_heads, head_dim, v_head_dim, ctypes.c_float(eps),
                                          _p(out), int(l2norm_qk))
    return out.reshape(tokens, n_heads, v_head_dim), st


# ---- norms ---------------------------------------------------------------

def rms_norm_zero_centered(x, weight, rows, dim, eps):
    x = _f32(x)
    y = np.empty_like(x)
    w = None if weight is None else _f32(weight)
    lib().q35o_rms_norm_zero_centered(_p(x), _p(w), _p(y), rows, dim, ctypes.c_float(eps))
    return y


def gated_rms_norm(x, weight, gate, rows, dim, eps):
    x, gate = _f32(x), _f32(gate)
    y = np.empty_like(x)
    w = None if weight is None else _f32(weight)
    lib().q35o_gated_rms_norm(_p(x), _p(w), _p(gate), _p(y), rows, dim, ctypes.c_float(eps))
    return y


# ---- attention -----------------------------------------------------------

def rope_table(cap, half, base):
    c = np.empty(cap * half, np.float32)
    s = np.empty(cap * half, np.float32)
    lib().q35o_rope_table(cap, half, ctypes.c_float(base), _p(c), _p(s))
    return c.reshape(cap, half), s.reshape(cap, half)


def neox_rope(x, tokens, heads, head_dim, rope_dim, start_pos, base):
    y = _f32(x).copy()
    lib().q35o_neox_rope(_p(y), tokens, heads, head_dim, rope_dim, start_pos, ctypes.c_float(base))
    return y


def attention_scores(q, cache_k, heads, kv_heads, head_dim, q_len, kv_len, q_dim, kv_stride,
                     scale, start_pos, n_threads=1):
    q, cache_k = _f32(q), _f32(cache_k)
    sc = np.zeros(heads * q_len * kv_len, np.float32)
    lib().q35o_attention_scores(_p(q), _p(cache_k), _p(sc), heads, kv_heads, head_dim, q_len,
                                kv_len, q_dim, kv_stride, ctypes.c_float(scale), start_pos,
                                n_threads)
    return sc.reshape(heads, q_len, kv_len)


def softmax_causal(scores, heads, q_len, kv_len, start_pos, n_threads=1):
    sc = _f32(scores).copy()
    lib().q35o_softmax_causal(_p(sc), heads, q_len, kv_len, start_pos, n_threads)
    return sc


def attention_combine(cache_v, scores, heads, kv_heads, head_dim, q_len, kv_len, q_dim,
                      kv_stride, start_pos, n_threads=1):
    cache_v, scores = _f32(cache_v), _f32(scores)
    out = np.zeros(q_len * q_dim, np.float32)
    lib().q35o_attention_combine(_p(cache_v), _p(scores), _p(out), heads, kv_heads, head_dim,
                                 q_len, kv_len, q_dim, kv_stride, start_pos, n_threads)
    return out.reshape(q_len, q_dim)


# ---- mixers --------------------------------------------------------------

def deltanet_decode(d: Dims, qkv, z, b, a, w: dict, conv_state, state):
    """One token.  Returns (out, new_conv_state, new_state, core_out)."""
    qkv, z, b, a = map(_f32, (qkv, z, b, a))
    cs, st = _f32(conv_state).copy(), _f32(state).copy()
    nv, hd = d.n_v_heads, d.head_k_dim
    out = np.empty(nv * hd, np.float32)
    core = np.empty(nv * hd, np.float32)
    lib().q35o_deltanet_decode(ctypes.byref(d), _p(qkv), _p(z), _p(b), _p(a),
                               _p(_f32(w["conv_w"])), _p(_f32(w["ssm_a"])),
                               _p(_f32(w["dt_bias"])), _p(_f32(w["ssm_norm"])), _p(cs), _p(st),
                               _p(out), _p(core))
    return out, cs, st, core


def deltanet_prefill(d: Dims, T, qkv, z, b, a, w: dict, state, conv_state=None):
    """T tokens.  Returns (out [T][nv*hd], new_conv_state, new_state, core_out)."""
    qkv, z, b, a = map(_f32, (qkv, z, b, a))
    nv, nk, hd = d.n_v_heads, d.n_k_heads, d.head_k_dim
    conv_dim = 2 * nk * hd + nv * hd
    cs = np.zeros((conv_dim, d.conv_kernel - 1), np.float32) if conv_state is None \
        else _f32(conv_state).copy()
    st = _f32(state).copy()
    out = np.empty((T, nv * hd), np.float32)
    core = np.empty((T, nv * hd), np.float32)
    lib().q35o_deltanet_prefill(ctypes.byref(d), T, _p(qkv), _p(z), _p(b), _p(a),
                                _p(_f32(w["conv_w"])), _p(_f32(w["ssm_a"])),
                                _p(_f32(w["dt_bias"])), _p(_f32(w["ssm_norm"])), _p(cs), _p(st),
                                _p(out), _p(core))
    return out, cs, st, core


def attn_decode(d: Dims, start, q_gate, k, v, w: dict, cache_k, cache_v, n_threads=1, inplace=False):
    """Returns (out [n_heads*head_dim], cache_k', cache_v') with row `start` written.
    inplace: write the row into cache_k / cache_v themselves (contiguous fp32
    arrays) instead of into copies, for caches of many rows."""
    if inplace:
        assert all(a.dtype == np.float32 and a.flags.c_contiguous for a in (cache_k, cache_v))
        ck, cv = cache_k, cache_v
    else:
        ck, cv = _f32(cache_k).copy(), _f32(cache_v).copy()
    out = np.empty(d.n_heads * d.head_dim, np.float32)
    lib().q35o_attn_decode(ctypes.byref(d), start, _p(_f32(q_gate)), _p(_f32(k)), _p(_f32(v)),
                           _p(_f32(w["q_norm"])), _p(_f32(w["k_norm"])), _p(ck), _p(cv),
                           _p(out), n_threads)
    return out, ck, cv


def attn_prefill(d: Dims, start, T, q_gate, k, v, w: dict, cache_k, cache_v, n_threads=1):
    """Returns (out [T][n_heads*head_dim], cache_k', cache_v') with rows start.. written."""
    ck, cv = _f32(cache_k).copy(), _f32(cache_v).copy()
    out = np.empty((T, d.n_heads * d.head_dim), np.float32)
    lib().q35o_attn_prefill(ctypes.byref(d), start, T, _p(_f32(q_gate)), _p(_f32(k)),
                            _p(_f32(v)), _p(_f32(w["q_norm"])), _p(_f32(w["k_norm"])), _p(ck),
                            _p(cv), _p(out), n_threads)
    return out, ck, cv


# ---- quantized projections (q35_oracle_quant.c) --------------------------

QK = 256
Q4K_BYTES, Q6K_BYTES, Q8K_BYTES = 144, 210, 292
Q5K_BYTES, IQ4XS_BYTES = 176, 136
Q2_0C_BYTES, STQ1_0_BYTES = 130, 42     # Q2_0C blocks hold 512 values
# Projection type codes of q35o_linear_q (and of the library's linear entry
# points): 1 = STQ1_0, 2 = Q2_0C, 4 = Q4_K, 5 = Q5_K, 6 = Q6_K, 14 = IQ4_XS.
QT_STQ1_0, QT_Q2_0C, QT_Q4K, QT_Q5K, QT_Q6K, QT_IQ4XS = 1, 2, 4, 5, 6, 14
_U8 = ctypes.POINTER(ctypes.c_uint8)


def _bytes(a) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.uint8)
    return a


def half_to_float(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16).ravel()
    f = lib().q35o_half_to_float
    f.restype = ctypes.c_float
    f.argtypes = [ctypes.c_uint16]
    return np.array([f(int(v)) for v in h], dtype=np.float32)


def q8k_quantize(x) -> np.ndarray:
    """Q8_K blocks (292 bytes each) of a row of n floats, n a multiple of 256."""
    x = _f32(x).ravel()
    out = np.zeros(x.size // QK * Q8K_BYTES, dtype=np.uint8)
    lib().q35o_q8k_quantize_row(_p(x), out.ctypes.data_as(_U8), ctypes.c_int(x.size))
    return out


def q4k_dot(w, q8, n) -> float:
    f = lib().q35o_q4k_dot
    f.restype = ctypes.c_float
    w, q8 = _bytes(w), _bytes(q8)
    return f(w.ctypes.data_as(_U8), q8.ctypes.data_as(_U8), ctypes.c_int(n))


def q6k_dot(w, q8, n) -> float:
    f = lib().q35o_q6k_dot
    f.restype = ctypes.c_float
    w, q8 = _bytes(w), _bytes(q8)
    return f(w.ctypes.data_as(_U8), q8.ctypes.data_as(_U8), ctypes.c_int(n))


def q5k_dot(w, q8, n) -> float:
    f = lib().q35o_q5k_dot
    f.restype = ctypes.c_float
    w, q8 = _bytes(w), _bytes(q8)
    return f(w.ctypes.data_as(_U8), q8.ctypes.data_as(_U8), ctypes.c_int(n))


def iq4xs_dot(w, q8, n) -> float:
    f = lib().q35o_iq4xs_dot
    f.restype = ctypes.c_float
    w, q8 = _bytes(w), _bytes(q8)
    return f(w.ctypes.data_as(_U8), q8.ctypes.data_as(_U8), ctypes.c_int(n))


def q2_0c_dot(w, q8, n) -> float:
    """Q2_0C.DotAvx2, the raw-row order (rows outside the eight-row panels)."""
    f = lib().q35o_q2_0c_dot
    f.restype = ctypes.c_float
    w, q8 = _bytes(w), _bytes(q8)
    return f(w.ctypes.data_as(_U8), q8.ctypes.data_as(_U8), ctypes.c_int(n))


def stq1_0_dot(w, q8, n) -> float:
    """STQ1_0.DotAvx2, the raw-row order (rows outside the eight-row panels)."""
    f = lib().q35o_stq1_0_dot
    f.restype = ctypes.c_float
    w, q8 = _bytes(w), _bytes(q8)
    return f(w.ctypes.data_as(_U8), q8.ctypes.data_as(_U8), ctypes.c_int(n))


def dot(qtype: int, w, q8, n) -> float:
    return {QT_Q4K: q4k_dot, QT_Q5K: q5k_dot, QT_Q6K: q6k_dot, QT_IQ4XS: iq4xs_dot,
            QT_Q2_0C: q2_0c_dot, QT_STQ1_0: stq1_0_dot}[qtype](w, q8, n)


def dequantize(qtype: int, w, k) -> np.ndarray:
    w = _bytes(w)
    y = np.empty(k, dtype=np.float32)
    fn = {QT_Q4K: lib().q35o_q4k_dequantize_row, QT_Q5K: lib().q35o_q5k_dequantize_row,
          QT_Q6K: lib().q35o_q6k_dequantize_row, QT_IQ4XS: lib().q35o_iq4xs_dequantize_row,
          QT_Q2_0C: lib().q35o_q2_0c_dequantize_row, QT_STQ1_0: lib().q35o_stq1_0_dequantize_row}[qtype]
    fn(w.ctypes.data_as(_U8), _p(y), ctypes.c_int(k))
    return y


def linear_q(qtype: int, w, x, n_in, n_out) -> np.ndarray:
    """y[t] = W x[t] with W given as GGUF rows of qtype 1 (STQ1_0), 2 (Q2_0C),
    4 (Q4_K), 5 (Q5_K), 6 (Q6_K) or 14 (IQ4_XS) blocks; every row of x is one
    token of the same call (the STQ1_0 order depends on the token count)."""
    w = _bytes(w)
    x = _f32(x).reshape(-1, n_in)
    y = np.empty((x.shape[0], n_out), dtype=np.float32)
    lib().q35o_linear_q(ctypes.c_int(qtype), w.ctypes.data_as(_U8), _p(x), _p(y),
                        ctypes.c_int(n_in), ctypes.c_int(n_out), ctypes.c_int(x.shape[0]))
    return y


def linear_f32(w, x, n_in, n_out) -> np.ndarray:
    """Qwen35Model.F32Gemm: y[t][o] = Ops.DotF32(x[t], w[o]), w [n_out][n_in]."""
    w = _f32(w).reshape(n_out, n_in)
    x = _f32(x).reshape(-1, n_in)
    y = np.empty((x.shape[0], n_out), dtype=np.float32)
    lib().q35o_linear_f32(_p(w), _p(x), _p(y), ctypes.c_int(n_in), ctypes.c_int(n_out), ctypes.c_int(x.shape[0]))
    return y


def add_rmsnorm(hidden, delta, w, dim, eps=1e-6):
    """Ops.AddInPlace then Qwen35Ops.RmsNormZeroCentered over rows of dim:
    returns (hidden after the add, y).  delta / w may be None."""
    h = _f32(hidden).reshape(-1, dim).copy()
    rows = h.shape[0]
    d = None if delta is None else _f32(delta).reshape(rows, dim).copy()
    ww = None if w is None else _f32(w).ravel().copy()
    y = np.empty_like(h)
    lib().q35o_add_rmsnorm(_p(h), None if d is None else _p(d), None if ww is None else _p(ww), _p(y),
                           ctypes.c_int(dim), ctypes.c_int(rows), ctypes.c_float(eps))
    return h, y
