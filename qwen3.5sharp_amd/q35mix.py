"""ctypes front end of libq35mix.so (include/q35mix.h).

This is the Python view of the C ABI that tests and bench.py drive.  It
loads the in-tree libq35mix.so and raises if it is missing: there is no
CPU fallback.  Device memory is the library's own (q35m_malloc); the HIP
runtime it links is used directly only for event timing on the context
stream.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libq35mix.so")

OK = 0
ERR_INVALID, ERR_UNSUPPORTED, ERR_CAPACITY, ERR_NO_DEVICE, ERR_HIP, ERR_OOM, ERR_RANGE = \
    -1, -2, -3, -4, -5, -6, -7
STATE_RECURRENT, STATE_CONV, STATE_KEYS, STATE_VALUES = 0, 1, 2, 3
PROJ_REFERENCE, PROJ_BLOCK = 0, 1

_lib = None
_hip = None


class Q35Error(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"q35mix error {code}: {msg}")
        self.code = code


def build() -> None:
    subprocess.run(["make", "-s", "-j8", "-C", HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(f"{LIB_PATH} is not built (run __graft_entry__.build())")
        _lib = ctypes.CDLL(LIB_PATH)
        _lib.q35m_last_error.restype = ctypes.c_char_p
        _lib.q35m_stream.restype = ctypes.c_void_p
        _lib.q35m_stream.argtypes = [ctypes.c_void_p]
        for name in ("q35m_malloc",):
            getattr(_lib, name).argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
        _lib.q35m_free.argtypes = [ctypes.c_void_p]
        for name in ("q35m_copy_h2d", "q35m_copy_d2h"):
            getattr(_lib, name).argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                            ctypes.c_size_t]
        for name in ("q35m_state_read", "q35m_state_write"):
            getattr(_lib, name).argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                            ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t]
        _lib.q35m_profile_kernel_name.restype = ctypes.c_char_p
        _lib.q35m_profile.argtypes = [ctypes.c_void_p, ctypes.c_int]
        _lib.q35m_profile_read.argtypes = [ctypes.c_void_p, ctypes.c_int,
                                           ctypes.POINTER(ctypes.c_double),
                                           ctypes.POINTER(ctypes.c_long)]
        _lib.q35m_state_device_ptr.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                               ctypes.c_int, ctypes.POINTER(ctypes.c_void_p),
                                               ctypes.POINTER(ctypes.c_size_t)]
        for name in ("q35m_linear_q4k", "q35m_linear_q6k", "q35m_linear_q4k_prequant",
                     "q35m_linear_q6k_prequant", "q35m_linear_q5k", "q35m_linear_iq4xs",
                     "q35m_linear_q5k_prequant", "q35m_linear_iq4xs_prequant", "q35m_linear_q2_0c",
                     "q35m_linear_stq1_0", "q35m_linear_q2_0c_prequant", "q35m_linear_stq1_0_prequant"):
            getattr(_lib, name).argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                            ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                            ctypes.c_int]
        _lib.q35m_grow.argtypes = [ctypes.c_void_p, ctypes.c_int]
        _lib.q35m_gguf_open.argtypes = [ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p)]
        _lib.q35m_gguf_close.argtypes = [ctypes.c_void_p]
        _lib.q35m_gguf_tensor.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int),
                                          ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int),
                                          ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_size_t)]
        _lib.q35m_gguf_int.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64)]
        _lib.q35m_gguf_float.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_double)]
        _lib.q35m_gguf_string.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p)]
        _lib.q35m_load_mixer_weights.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_char_p,
                                                 ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        _lib.q35m_snapshot_bytes.restype = ctypes.c_size_t
        _lib.q35m_snapshot_bytes.argtypes = [ctypes.c_void_p]
        for name in ("q35m_snapshot_save", "q35m_snapshot_restore"):
            getattr(_lib, name).argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t,
                                            ctypes.POINTER(SnapshotInfo)]
        _lib.q35m_add_rmsnorm.argtypes = [ctypes.c_void_p] * 6 + [ctypes.c_int, ctypes.c_int, ctypes.c_float]
        _lib.q35m_add_rmsnorm.restype = ctypes.c_int
        _lib.q35m_quantize_q8k.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                           ctypes.c_int, ctypes.c_int]
        _lib.q35m_q8k_bytes.restype = ctypes.c_size_t
        _lib.q35m_q8k_bytes.argtypes = [ctypes.c_int, ctypes.c_int]
        _lib.q35m_reuse_plan.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                                         ctypes.c_void_p, ctypes.c_int] + [ctypes.POINTER(ctypes.c_int)] * 3
        _lib.q35m_decode_graph_create.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                                                  ctypes.POINTER(DecodeIO), ctypes.c_int,
                                                  ctypes.POINTER(ctypes.c_void_p)]
        _lib.q35m_decode_graph_run.argtypes = [ctypes.c_void_p, ctypes.c_int]
        _lib.q35m_decode_graph_destroy.argtypes = [ctypes.c_void_p]
    return _lib


def reuse_plan(cached, prompt, snap_lens=()):
    """(truncate_to, suffix_start, snapshot index or -1) of q35m_reuse_plan
    (KvCacheAlign.Plan, extended to the caller's snapshot lengths)."""
    arrs = [np.ascontiguousarray(np.asarray(a, dtype=np.int32)) for a in (cached, prompt, snap_lens)]
    ptr = lambda a: ctypes.c_void_p(a.ctypes.data) if a.size else None  # noqa: E731
    out = [ctypes.c_int(-7) for _ in range(3)]
    check(lib().q35m_reuse_plan(ptr(arrs[0]), arrs[0].size, ptr(arrs[1]), arrs[1].size, ptr(arrs[2]),
                                arrs[2].size, *[ctypes.byref(o) for o in out]))
    return tuple(o.value for o in out)


def check(code: int) -> None:
    if code != OK:
        raise Q35Error(code, lib().q35m_last_error().decode())


def device_count() -> int:
    n = ctypes.c_int(0)
    r = lib().q35m_device_count(ctypes.byref(n))
    return n.value if r == OK else 0


class Config(ctypes.Structure):
    _fields_ = [("num_layers", ctypes.c_int), ("num_heads", ctypes.c_int),
                ("num_kv_heads", ctypes.c_int), ("head_dim", ctypes.c_int),
                ("rope_dim", ctypes.c_int), ("rope_base", ctypes.c_float),
                ("ssm_conv_kernel", ctypes.c_int), ("ssm_inner_size", ctypes.c_int),
                ("ssm_state_size", ctypes.c_int), ("ssm_time_step_rank", ctypes.c_int),
                ("ssm_group_count", ctypes.c_int), ("eps", ctypes.c_float),
                ("full_attention_interval", ctypes.c_int),
                ("is_recurrent", ctypes.POINTER(ctypes.c_ubyte))]


def qwen35_config(num_layers=32, num_heads=16, num_kv_heads=4, n_k_heads=16, n_v_heads=32,
                  interval=4, is_recurrent=None) -> Config:
    """Mixer dims of the 4B-class family member: hd 256, rope 64 (base 1e7),
    dk = dv = 128, conv 4, eps 1e-6; GQA at (i+1) % 4 == 0."""
    c = Config(num_layers, num_heads, num_kv_heads, 256, 64, 1e7, 4, n_v_heads * 128, 128,
               n_v_heads, n_k_heads, 1e-6, interval, None)
    if is_recurrent is not None:
        arr = (ctypes.c_ubyte * num_layers)(*[1 if x else 0 for x in is_recurrent])
        c.is_recurrent = ctypes.cast(arr, ctypes.POINTER(ctypes.c_ubyte))
        c._keep = arr
    return c


class DeviceArray:
    """fp32 device buffer owned by the library allocator."""

    def __init__(self, ctx: "Context", shape, data: np.ndarray | None = None):
        self.ctx = ctx
        self.shape = tuple(int(s) for s in np.atleast_1d(shape)) if not isinstance(shape, tuple) \
            else shape
        self.nbytes = int(np.prod(self.shape)) * 4
        p = ctypes.c_void_p()
        check(lib().q35m_malloc(ctypes.byref(p), max(self.nbytes, 4)))
        self.ptr = p.value
        if data is not None:
            self.upload(data)

    def upload(self, data: np.ndarray) -> None:
        a = np.ascontiguousarray(data, dtype=np.float32)
        assert a.nbytes == self.nbytes, (a.shape, self.shape)
        check(lib().q35m_copy_h2d(self.ctx.handle, self.ptr, a.ctypes.data, a.nbytes))

    def download(self) -> np.ndarray:
        a = np.empty(self.shape, np.float32)
        check(lib().q35m_copy_d2h(self.ctx.handle, a.ctypes.data, self.ptr, a.nbytes))
        return a

    def free(self) -> None:
        if self.ptr:
            lib().q35m_free(self.ptr)
            self.ptr = None


class DeviceView(DeviceArray):
    """fp32 window [offset, offset + prod(shape)) of another device buffer
    (shares its memory; frees nothing)."""

    def __init__(self, base: DeviceArray, offset: int, shape):
        self.ctx = base.ctx
        self.shape = tuple(int(s) for s in np.atleast_1d(shape))
        self.nbytes = int(np.prod(self.shape)) * 4
        assert 0 <= offset and offset * 4 + self.nbytes <= base.nbytes
        self.ptr = base.ptr + 4 * offset
        self._base = base

    def free(self) -> None:
        self.ptr = None


class Gguf:
    """A GGUF file opened by the library (q35m_gguf_open); tensors are views
    of the read-only mapping."""

    def __init__(self, path: str):
        h = ctypes.c_void_p()
        check(lib().q35m_gguf_open(str(path).encode(), ctypes.byref(h)))
        self.handle = h.value

    def close(self) -> None:
        if self.handle:
            check(lib().q35m_gguf_close(ctypes.c_void_p(self.handle)))
            self.handle = None

    def tensor(self, name: str):
        """(ggml type, dims innermost first, raw bytes)."""
        t, nd, p, nb = ctypes.c_int(), ctypes.c_int(), ctypes.c_void_p(), ctypes.c_size_t()
        dims = (ctypes.c_int64 * 4)()
        check(lib().q35m_gguf_tensor(ctypes.c_void_p(self.handle), name.encode(), ctypes.byref(t), dims,
                                     ctypes.byref(nd), ctypes.byref(p), ctypes.byref(nb)))
        raw = ctypes.string_at(p.value, nb.value) if nb.value else b""
        return t.value, tuple(dims[:nd.value]), raw

    def int(self, key: str) -> int:
        v = ctypes.c_int64()
        check(lib().q35m_gguf_int(ctypes.c_void_p(self.handle), key.encode(), ctypes.byref(v)))
        return v.value

    def float(self, key: str) -> float:
        v = ctypes.c_double()
        check(lib().q35m_gguf_float(ctypes.c_void_p(self.handle), key.encode(), ctypes.byref(v)))
        return v.value

    def string(self, key: str) -> str:
        v = ctypes.c_char_p()
        check(lib().q35m_gguf_string(ctypes.c_void_p(self.handle), key.encode(), ctypes.byref(v)))
        return v.value.decode()


class DecodeIO(ctypes.Structure):
    """q35m_decode_io: one layer's activations in a decode graph (DeltaNet:
    qkv, z, b, a, out; full attention: q_gate, k, v, unused, out)."""
    _fields_ = [("in0", ctypes.c_void_p), ("in1", ctypes.c_void_p), ("in2", ctypes.c_void_p),
                ("in3", ctypes.c_void_p), ("out", ctypes.c_void_p)]


class DecodeGraph:
    """q35m_decode_graph: one decode step of every layer for a fixed batch,
    captured once (q35m_decode_graph_create) and run per token.  `io` holds,
    per layer, the device arrays (in0, in1, in2, in3, out) of that layer's
    mixer (in3 None for full-attention layers)."""

    def __init__(self, ctx: "Context", seqs, io, max_len: int):
        self.ctx = ctx
        arr = (DecodeIO * len(io))()
        for l, bufs in enumerate(io):
            arr[l] = DecodeIO(*[None if b is None else b.ptr for b in bufs])
        h = ctypes.c_void_p()
        check(lib().q35m_decode_graph_create(ctypes.c_void_p(ctx.handle), len(seqs), _seqs(seqs), arr, max_len,
                                             ctypes.byref(h)))
        self.handle = h.value
        self._io = io

    def run(self, replay: bool = True) -> None:
        check(lib().q35m_decode_graph_run(ctypes.c_void_p(self.handle), int(replay)))

    def try_run(self, replay: bool = True) -> int:
        return lib().q35m_decode_graph_run(ctypes.c_void_p(self.handle), int(replay))

    def close(self) -> None:
        if self.handle:
            check(lib().q35m_decode_graph_destroy(ctypes.c_void_p(self.handle)))
            self.handle = None


class SnapshotInfo(ctypes.Structure):
    """q35m_snapshot_info: the length and epoch a snapshot was taken at."""
    _fields_ = [("kv_len", ctypes.c_int), ("epoch", ctypes.c_uint)]


class DeviceBytes(DeviceArray):
    """Raw byte buffer in device memory (quantized weight blocks)."""

    def __init__(self, ctx: "Context", data: np.ndarray):
        a = np.ascontiguousarray(data, dtype=np.uint8).ravel()
        self.ctx = ctx
        self.shape = a.shape
        self.nbytes = a.nbytes
        p = ctypes.c_void_p()
        check(lib().q35m_malloc(ctypes.byref(p), max(self.nbytes, 4)))
        self.ptr = p.value
        check(lib().q35m_copy_h2d(self.ctx.handle, self.ptr, a.ctypes.data, a.nbytes))

    def download(self) -> np.ndarray:
        a = np.empty(self.nbytes, np.uint8)
        check(lib().q35m_copy_d2h(self.ctx.handle, a.ctypes.data, self.ptr, a.nbytes))
        return a

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _seqs(seqs):
    arr = (ctypes.c_int * len(seqs))(*seqs)
    return arr


class Context:
    """One q35m_ctx: the mixer state of every layer for n_seqs sequences."""

    def __init__(self, cfg: Config, n_seqs: int = 1, kv_capacity: int = 4096):
        self.cfg = cfg
        h = ctypes.c_void_p()
        check(lib().q35m_create(ctypes.byref(cfg), n_seqs, kv_capacity, ctypes.byref(h)))
        self.handle = h.value
        self.n_seqs = n_seqs
        self.kv_capacity = kv_capacity
        nv, nk = cfg.ssm_time_step_rank, cfg.ssm_group_count
        self.conv_dim = 2 * nk * 128 + nv * 128
        self.value_dim = nv * 128
        self.q_dim = cfg.num_heads * 256
        self.kv_dim = cfg.num_kv_heads * 256

    def close(self) -> None:
        if self.handle:
            check(lib().q35m_destroy(ctypes.c_void_p(self.handle)))
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def array(self, shape, data=None) -> DeviceArray:
        return DeviceArray(self, shape, data)

    @property
    def stream(self) -> int:
        return lib().q35m_stream(self.handle)

    def sync(self) -> None:
        check(lib().q35m_sync(ctypes.c_void_p(self.handle)))

    # ---- lifecycle (Qwen35Model.ResetCache / TruncateCache / Forward) ----
    def reset(self, seq: int) -> None:
        check(lib().q35m_reset(ctypes.c_void_p(self.handle), seq))

    def truncate(self, seq: int, length: int) -> None:
        check(lib().q35m_truncate(ctypes.c_void_p(self.handle), seq, length))

    def advance(self, seq: int, n: int) -> None:
        check(lib().q35m_advance(ctypes.c_void_p(self.handle), seq, n))

    def kv_len(self, seq: int) -> int:
        n = ctypes.c_int()
        check(lib().q35m_kv_len(ctypes.c_void_p(self.handle), seq, ctypes.byref(n)))
        return n.value

    # ---- weights -----------------------------------------------------------
    def set_deltanet_weights(self, layer: int, w: dict) -> None:
        arrs = [np.ascontiguousarray(w[k], np.float32) for k in
                ("conv_w", "ssm_a", "dt_bias", "ssm_norm")]
        check(lib().q35m_set_deltanet_weights(ctypes.c_void_p(self.handle), layer,
                                              *[a.ctypes.data_as(ctypes.c_void_p) for a in arrs]))

    def set_attn_weights(self, layer: int, w: dict) -> None:
        arrs = [np.ascontiguousarray(w[k], np.float32) for k in ("q_norm", "k_norm")]
        check(lib().q35m_set_attn_weights(ctypes.c_void_p(self.handle), layer,
                                          *[a.ctypes.data_as(ctypes.c_void_p) for a in arrs]))

    # ---- mixers (device arrays) -----------------------------------------
    def deltanet_decode(self, layer, seqs, qkv, z, b, a, out) -> None:
        check(lib().q35m_deltanet_decode(ctypes.c_void_p(self.handle), layer, len(seqs),
                                         _seqs(seqs), *[ctypes.c_void_p(x.ptr) for x in
                                                        (qkv, z, b, a, out)]))

    def deltanet_prefill(self, layer, seq, T, qkv, z, b, a, out) -> None:
        check(lib().q35m_deltanet_prefill(ctypes.c_void_p(self.handle), layer, seq, T,
                                          *[ctypes.c_void_p(x.ptr) for x in (qkv, z, b, a, out)]))

    def attn_decode(self, layer, seqs, q_gate, k, v, out) -> None:
        check(lib().q35m_attn_decode(ctypes.c_void_p(self.handle), layer, len(seqs),
                                     _seqs(seqs), *[ctypes.c_void_p(x.ptr) for x in
                                                    (q_gate, k, v, out)]))

    def attn_decode_noalloc(self, layer, seqs, q_gate, k, v, out) -> None:
        """q35m_attn_decode with the split-K partials in the library's fixed
        device scratch (no allocation)."""
        check(lib().q35m_attn_decode_noalloc(ctypes.c_void_p(self.handle), layer, len(seqs),
                                             _seqs(seqs), *[ctypes.c_void_p(x.ptr) for x in
                                                            (q_gate, k, v, out)]))

    def attn_prefill(self, layer, seq, T, q_gate, k, v, out) -> None:
        check(lib().q35m_attn_prefill(ctypes.c_void_p(self.handle), layer, seq, T,
                                      *[ctypes.c_void_p(x.ptr) for x in (q_gate, k, v, out)]))

    def bytes_array(self, data) -> DeviceBytes:
        return DeviceBytes(self, data)

    def quantize_q8k(self, x, n_in, tokens) -> "DeviceBytes":
        """Q8_K blocks of x [tokens][n_in] in a new device buffer."""
        q8 = DeviceBytes(self, np.zeros(lib().q35m_q8k_bytes(n_in, tokens), np.uint8))
        check(lib().q35m_quantize_q8k(ctypes.c_void_p(self.handle), ctypes.c_void_p(x.ptr),
                                      ctypes.c_void_p(q8.ptr), n_in, tokens))
        return q8

    def load_mixer_weights(self, gguf: "Gguf") -> None:
        """The mixers' F32 tensors of every layer from a GGUF file."""
        c = self.cfg
        if c.is_recurrent:
            rec = bytes(int(bool(c.is_recurrent[i])) for i in range(c.num_layers))
        else:
            rec = bytes(int((i + 1) % c.full_attention_interval != 0) for i in range(c.num_layers))
        check(lib().q35m_load_mixer_weights(ctypes.c_void_p(self.handle), ctypes.c_void_p(gguf.handle),
                                            c.num_layers, rec, self.conv_dim, c.ssm_time_step_rank,
                                            c.ssm_state_size, c.head_dim))

    def grow(self, kv_capacity: int) -> None:
        check(lib().q35m_grow(ctypes.c_void_p(self.handle), kv_capacity))

    def snapshot_save(self, seq: int):
        """(device buffer, SnapshotInfo) of seq's linear state."""
        n = lib().q35m_snapshot_bytes(ctypes.c_void_p(self.handle))
        buf = DeviceBytes(self, np.zeros(max(n, 1), np.uint8))
        info = SnapshotInfo()
        check(lib().q35m_snapshot_save(ctypes.c_void_p(self.handle), seq, ctypes.c_void_p(buf.ptr), n,
                                       ctypes.byref(info)))
        return buf, info

    def snapshot_restore(self, seq: int, buf, info) -> None:
        check(lib().q35m_snapshot_restore(ctypes.c_void_p(self.handle), seq, ctypes.c_void_p(buf.ptr),
                                          buf.nbytes, ctypes.byref(info)))

    def add_rmsnorm(self, hidden, delta, w, y, q8, dim, tokens, eps=1e-6) -> None:
        """hidden += delta (delta may be None), y = RmsNormZeroCentered(hidden, w)
        (w may be None), optionally also as Q8_K blocks into q8 (may be None)."""
        ptr = lambda a: None if a is None else ctypes.c_void_p(a.ptr)  # noqa: E731
        check(lib().q35m_add_rmsnorm(ctypes.c_void_p(self.handle), ctypes.c_void_p(hidden.ptr), ptr(delta),
                                     ptr(w), ptr(y), ptr(q8), dim, tokens, eps))

    _LINEAR = {1: "stq1_0", 2: "q2_0c", 4: "q4k", 5: "q5k", 6: "q6k", 14: "iq4xs"}

    def linear_q_prequant(self, qtype: int, w, q8, y, n_in, n_out, tokens) -> None:
        fn = getattr(lib(), f"q35m_linear_{self._LINEAR[qtype]}_prequant")
        check(fn(ctypes.c_void_p(self.handle), ctypes.c_void_p(w.ptr), ctypes.c_void_p(q8.ptr),
                 ctypes.c_void_p(y.ptr), n_in, n_out, tokens))

    def linear_q(self, qtype: int, w, x, y, n_in, n_out, tokens) -> None:
        """y[tokens][n_out] = W x for GGUF weight rows of qtype 1 (STQ1_0),
        2 (Q2_0C), 4 (Q4_K), 5 (Q5_K), 6 (Q6_K) or 14 (IQ4_XS)."""
        fn = getattr(lib(), f"q35m_linear_{self._LINEAR[qtype]}")
        check(fn(ctypes.c_void_p(self.handle), ctypes.c_void_p(w.ptr), ctypes.c_void_p(x.ptr),
                 ctypes.c_void_p(y.ptr), n_in, n_out, tokens))

    def set_projection_order(self, order: int) -> None:
        """PROJ_REFERENCE (0, default) or PROJ_BLOCK (1): q35m_set_projection_order."""
        check(lib().q35m_set_projection_order(ctypes.c_void_p(self.handle), order))

    def linear_f32(self, w, x, y, n_in, n_out, tokens) -> None:
        """y[tokens][n_out] = W x for F32 weights W [n_out][n_in] (Ops.DotF32 order)."""
        check(lib().q35m_linear_f32(ctypes.c_void_p(self.handle), ctypes.c_void_p(w.ptr), ctypes.c_void_p(x.ptr),
                                    ctypes.c_void_p(y.ptr), n_in, n_out, tokens))

    # ---- per-kernel event timers -----------------------------------------
    def profile(self, enable: bool) -> None:
        check(lib().q35m_profile(self.handle, int(enable)))

    def profile_read(self) -> dict:
        """{kernel name: (total ms, launches)} for kernels launched since profile(True)."""
        res = {}
        k = 0
        while True:
            name = lib().q35m_profile_kernel_name(k)
            if not name:
                break
            ms, n = ctypes.c_double(), ctypes.c_long()
            check(lib().q35m_profile_read(self.handle, k, ctypes.byref(ms), ctypes.byref(n)))
            if n.value:
                res[name.decode()] = (ms.value, n.value)
            k += 1
        return res

    # ---- state I/O -----------------------------------------------------------
    def _state_shape(self, kind: int, rows: int | None):
        cfg = self.cfg
        if kind == STATE_RECURRENT:
            return (cfg.ssm_time_step_rank, 128, 128)
        if kind == STATE_CONV:
            return (self.conv_dim, 3)
        return (self.kv_capacity if rows is None else rows, self.kv_dim)

    def state_read(self, layer: int, seq: int, kind: int, rows: int | None = None) -> np.ndarray:
        a = np.empty(self._state_shape(kind, rows), np.float32)
        check(lib().q35m_state_read(self.handle, layer, seq, kind, a.ctypes.data, a.nbytes))
        return a

    def state_write(self, layer: int, seq: int, kind: int, data: np.ndarray) -> None:
        a = np.ascontiguousarray(data, np.float32)
        check(lib().q35m_state_write(self.handle, layer, seq, kind, a.ctypes.data, a.nbytes))

    def state_device_ptr(self, layer: int, seq: int, kind: int):
        p = ctypes.c_void_p()
        n = ctypes.c_size_t()
        check(lib().q35m_state_device_ptr(self.handle, layer, seq, kind, ctypes.byref(p),
                                          ctypes.byref(n)))
        return p.value, n.value


# ---- HIP event timing on the context stream ------------------------------

def hip() -> ctypes.CDLL:
    """The HIP runtime libq35mix.so itself links (same process-wide instance)."""
    global _hip
    if _hip is None:
        lib()
        _hip = ctypes.CDLL("libamdhip64.so.7")
        _hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        _hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        _hip.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        _hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                             ctypes.c_void_p]
        _hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
    return _hip


HIP_ATTR_MULTIPROCESSOR_COUNT = 63   # hipDeviceAttributeMultiprocessorCount


def cu_count(device: int = 0) -> int:
    """Compute units of a device (the decode-attention split is sized by it)."""
    n = ctypes.c_int(0)
    h = hip()
    h.hipDeviceGetAttribute.argtypes = [ctypes.POINTER(ctypes.c_int), ctypes.c_int, ctypes.c_int]
    r = h.hipDeviceGetAttribute(ctypes.byref(n), HIP_ATTR_MULTIPROCESSOR_COUNT, device)
    if r != 0:
        raise RuntimeError(f"hipDeviceGetAttribute failed: {r}")
    return n.value


def attn_decode_variant(n_seqs: int, n_kv_heads: int, lengths, n_cu: int, q_per_kv: int = 4) -> str:
    """Split the decode attention picks for a batch whose sequences hold
    `lengths` cached rows, as its per-kernel timer names it: one 64-row
    sub-chunk per workgroup ("1") while there are fewer than n_cu of them;
    else 16-row sub-chunks over one round of 2 workgroups per CU, 4 ("4,16")
    or 8 ("8,16") per workgroup, when 8 cover the rows; else 4 or 8 sub-chunks
    of 64 rows ("4", "8"), the fewest that keep one round.  A workgroup takes
    the q heads of one kv head, at most 8 (q_per_kv / 8 workgroups a kv head
    beyond); with 8 the one-sub-chunk split goes as 4 of 16 rows."""
    hpw = min(q_per_kv, 8)
    ng = n_seqs * n_kv_heads * (q_per_kv // hpw)
    max_cached = max(int(x) for x in lengths)
    max64, max16 = -(-max_cached // 64), -(-max_cached // 16)
    slots = 2 * n_cu
    if ng * max64 < n_cu:
        return "4,16" if hpw >= 8 else "1"
    nch = max(1, slots // ng)
    need = -(-max16 // nch)
    if need <= 4:
        return "4,16"
    if need <= 8:
        return "8,16"
    return "4" if ng * -(-max64 // 4) <= slots else "8"


class Event:
    def __init__(self):
        self.h = ctypes.c_void_p()
        r = hip().hipEventCreate(ctypes.byref(self.h))
        if r != 0:
            raise RuntimeError(f"hipEventCreate failed: {r}")

    def record(self, stream: int) -> None:
        r = hip().hipEventRecord(self.h, ctypes.c_void_p(stream))
        if r != 0:
            raise RuntimeError(f"hipEventRecord failed: {r}")

    def synchronize(self) -> None:
        hip().hipEventSynchronize(self.h)

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        end.synchronize()
        r = hip().hipEventElapsedTime(ctypes.byref(ms), self.h, end.h)
        if r != 0:
            raise RuntimeError(f"hipEventElapsedTime failed: {r}")
        return ms.value
