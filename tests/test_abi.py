"""C ABI checks that need no GPU: the library loads, exports every entry point
include/q35mix.h declares, and rejects bad arguments before touching a device."""
import ctypes
import os
import re

import pytest

import q35mix

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    for fn in os.listdir(os.path.join(ROOT, "include")):
        if fn.endswith(".h"):
            text = open(os.path.join(ROOT, "include", fn)).read()
            names |= set(re.findall(r"^\s*(?:int|void\*|const char\*|void|size_t)\s+(q35m_\w+)\s*\(",
                                    text, re.M))
    return sorted(names)


def test_header_declares_entry_points():
    names = declared_symbols()
    for must in ("q35m_create", "q35m_destroy", "q35m_deltanet_decode", "q35m_deltanet_prefill",
                 "q35m_attn_decode", "q35m_attn_prefill", "q35m_state_read", "q35m_last_error"):
        assert must in names


@pytest.mark.parametrize("name", declared_symbols())
def test_library_exports(name):
    assert hasattr(q35mix.lib(), name), name


def _cfg(**kw):
    c = q35mix.qwen35_config(num_layers=4)
    for k, v in kw.items():
        setattr(c, k, v)
    return c


def _create(cfg, n_seqs=1, cap=16):
    h = ctypes.c_void_p()
    r = q35mix.lib().q35m_create(ctypes.byref(cfg) if cfg is not None else None, n_seqs, cap,
                                 ctypes.byref(h))
    return r, h


def test_create_rejects_bad_config():
    assert _create(None)[0] == q35mix.ERR_INVALID
    assert _create(_cfg(), n_seqs=0)[0] == q35mix.ERR_INVALID
    assert _create(_cfg(), cap=0)[0] == q35mix.ERR_INVALID
    assert _create(_cfg(ssm_state_size=64, ssm_inner_size=32 * 64))[0] == q35mix.ERR_UNSUPPORTED
    assert _create(_cfg(head_dim=128))[0] == q35mix.ERR_UNSUPPORTED
    assert _create(_cfg(num_heads=12))[0] == q35mix.ERR_UNSUPPORTED
    assert _create(_cfg(ssm_time_step_rank=24, ssm_inner_size=24 * 128))[0] == q35mix.ERR_INVALID
    assert _create(_cfg(ssm_inner_size=1000))[0] == q35mix.ERR_INVALID
    assert _create(_cfg(eps=0.0))[0] == q35mix.ERR_INVALID
    msg = q35mix.lib().q35m_last_error().decode()
    assert "eps" in msg


def test_null_context_is_rejected():
    L = q35mix.lib()
    assert L.q35m_reset(None, 0) == q35mix.ERR_INVALID
    assert L.q35m_truncate(None, 0, 0) == q35mix.ERR_INVALID
    assert L.q35m_sync(None) == q35mix.ERR_INVALID
    assert L.q35m_destroy(None) == q35mix.ERR_INVALID
    assert L.q35m_stream(None) is None
    n = ctypes.c_int()
    assert L.q35m_kv_len(None, 0, ctypes.byref(n)) == q35mix.ERR_INVALID
    assert L.q35m_linear_q4k(None, None, None, None, 256, 1, 1) == q35mix.ERR_INVALID
    assert L.q35m_linear_q6k(None, None, None, None, 256, 1, 1) == q35mix.ERR_INVALID
    assert L.q35m_quantize_q8k(None, None, None, 256, 1) == q35mix.ERR_INVALID
    assert L.q35m_linear_q4k_prequant(None, None, None, None, 256, 1, 1) == q35mix.ERR_INVALID
    assert L.q35m_q8k_bytes(2560, 3) == 3 * 10 * 304
    assert L.q35m_add_rmsnorm(None, None, None, None, None, None, 2560, 1, 1e-6) == q35mix.ERR_INVALID
    assert L.q35m_grow(None, 64) == q35mix.ERR_INVALID
    assert L.q35m_load_mixer_weights(None, None, 1, b"\x01", 1, 1, 1, 1) == q35mix.ERR_INVALID
    assert L.q35m_gguf_close(None) == q35mix.ERR_INVALID
    assert L.q35m_snapshot_bytes(None) == 0
    info = q35mix.SnapshotInfo()
    assert L.q35m_snapshot_save(None, 0, None, 0, ctypes.byref(info)) == q35mix.ERR_INVALID
    assert L.q35m_snapshot_restore(None, 0, None, 0, ctypes.byref(info)) == q35mix.ERR_INVALID


def test_null_handles_of_decode_graph_and_settings_are_rejected():
    """The decode-graph, projection-order, snapshot-check, no-alloc and
    profiling entry points refuse a null context or graph before any device
    work, with a message in q35m_last_error."""
    L = q35mix.lib()
    seqs = (ctypes.c_int * 1)(0)
    io = (q35mix.DecodeIO * 4)()
    g = ctypes.c_void_p(1234)
    assert L.q35m_decode_graph_create(None, 1, seqs, io, 16, ctypes.byref(g)) == q35mix.ERR_INVALID
    assert g.value is None                       # *out cleared before the checks
    assert "context" in L.q35m_last_error().decode()
    assert L.q35m_decode_graph_create(None, 1, seqs, io, 16, None) == q35mix.ERR_INVALID
    assert L.q35m_decode_graph_run(None, 1) == q35mix.ERR_INVALID
    assert "graph" in L.q35m_last_error().decode()
    assert L.q35m_decode_graph_destroy(None) == q35mix.OK
    assert L.q35m_set_projection_order(None, q35mix.PROJ_BLOCK) == q35mix.ERR_INVALID
    info = q35mix.SnapshotInfo()
    assert L.q35m_snapshot_valid(None, 0, ctypes.byref(info)) == q35mix.ERR_INVALID
    assert L.q35m_attn_decode_noalloc(None, 3, 1, seqs, None, None, None, None) == q35mix.ERR_INVALID
    assert L.q35m_deltanet_decode(None, 0, 1, seqs, None, None, None, None, None) == q35mix.ERR_INVALID
    assert L.q35m_attn_decode(None, 3, 1, seqs, None, None, None, None) == q35mix.ERR_INVALID
    assert L.q35m_profile(None, 1) == q35mix.ERR_INVALID
    ms, n = ctypes.c_double(), ctypes.c_long()
    assert L.q35m_profile_read(None, 0, ctypes.byref(ms), ctypes.byref(n)) == q35mix.ERR_INVALID


def test_profile_kernel_names_end_with_null():
    L = q35mix.lib()
    names = []
    k = 0
    while L.q35m_profile_kernel_name(k) is not None:
        names.append(L.q35m_profile_kernel_name(k).decode())
        k += 1
    assert L.q35m_profile_kernel_name(-1) is None
    assert len(names) == len(set(names))
    for must in ("deltanet_decode_kernel", "dn_chunk_prep", "dn_chunk_scan", "dn_chunk_out",
                 "attn_decode_merge", "q4k_gemm", "q6k_gemm", "q6k_gemm_blk"):
        assert must in names, must


def test_no_device_here_is_an_error_not_a_fallback():
    if q35mix.device_count() > 0:
        pytest.skip("a HIP device is present")
    r, h = _create(_cfg())
    assert r == q35mix.ERR_NO_DEVICE
    assert h.value is None
    p = ctypes.c_void_p()
    assert q35mix.lib().q35m_malloc(ctypes.byref(p), 64) == q35mix.ERR_NO_DEVICE


def test_probe_library_exports():
    """bench.py's device-ceiling probes (a separate library, not the mixer ABI)."""
    lib = ctypes.CDLL(os.path.join(ROOT, "qwen3.5sharp_amd", "libq35probe.so"))
    for name in ("q35p_hbm_read_gbs", "q35p_hbm_copy_gbs", "q35p_mfma_f32_tflops"):
        assert hasattr(lib, name), name
    v = ctypes.c_double(0.0)
    assert lib.q35p_mfma_f32_tflops(0, ctypes.byref(v)) == -1      # rejected before any device call
