"""q35m_attn_decode_noalloc (decode attention whose split-K partials live in
the library's fixed device scratch instead of an allocated workspace)
against q35m_attn_decode on the same state, through the C ABI: bit-identical
outputs and new cache rows on two calls in a row, the second with a smaller
batch and shorter contexts; both also within 1e-4 of the oracle; a batch
whose partials would not fit the scratch is refused with Q35M_ERR_CAPACITY;
and the entry point captured into a HIP graph replays bit-identically to the
eager call."""
import ctypes
import sys

import numpy as np
import pytest

import oracle
import q35mix
import synth

pytestmark = pytest.mark.gpu

NH, NKV, HD = 16, 4, 256
KV_DIM = NKV * HD


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def bits_equal(a, b):
    return np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))


def test_noalloc_matches_allocating_entry_point():
    n, cap = 8, 8200
    lens = [8192, 7001, 5000, 4096, 3000, 700, 64, 0]
    with q35mix.Context(q35mix.qwen35_config(num_layers=1, is_recurrent=[0]), n_seqs=n, kv_capacity=cap) as c:
        wts = synth.attn_weights(HD, salt=5)
        c.set_attn_weights(0, wts)
        caches = []
        for s, L in enumerate(lens):
            k, v = synth.kv_prefill(L + 1, KV_DIM, salt=150 + s)
            if L:
                c.state_write(0, s, q35mix.STATE_KEYS, k[:L])
                c.state_write(0, s, q35mix.STATE_VALUES, v[:L])
                c.advance(s, L)
            caches.append((k, v))
        for call, (seqs, salt) in enumerate(((list(range(n)), 61), ([6, 1], 62))):
            if call == 1:
                c.truncate(1, 1000)                 # shorter context for the second call
            m = len(seqs)
            x = synth.attn_inputs(m, NH, NKV, HD, salt=salt)
            qg, kk, vv = c.array((m, 2 * c.q_dim), x["q_gate"]), c.array((m, c.kv_dim), x["k"]), \
                c.array((m, c.kv_dim), x["v"])
            out_a, out_b = c.array((m, c.q_dim)), c.array((m, c.q_dim))
            say(f"call {call}: {m} sequences, lengths {[c.kv_len(s) for s in seqs]}")
            c.attn_decode(0, seqs, qg, kk, vv, out_a)
            rows_a = [(c.state_read(0, s, q35mix.STATE_KEYS, c.kv_len(s) + 1)[-1],
                       c.state_read(0, s, q35mix.STATE_VALUES, c.kv_len(s) + 1)[-1]) for s in seqs]
            c.attn_decode_noalloc(0, seqs, qg, kk, vv, out_b)
            a, b = out_a.download(), out_b.download()
            assert bits_equal(a, b)
            for j, s in enumerate(seqs):
                L = c.kv_len(s)
                kr = c.state_read(0, s, q35mix.STATE_KEYS, L + 1)[-1]
                vr = c.state_read(0, s, q35mix.STATE_VALUES, L + 1)[-1]
                assert bits_equal(kr, rows_a[j][0]) and bits_equal(vr, rows_a[j][1])
                k, v = caches[s]
                ck = np.zeros((L + 1, KV_DIM), np.float32)
                cv = np.zeros_like(ck)
                ck[:L], cv[:L] = k[:L], v[:L]
                ref, _, _ = oracle.attn_decode(oracle.dims(), L, x["q_gate"][j], x["k"][j], x["v"][j], wts,
                                               ck, cv, n_threads=8)
                e = float(np.max(np.abs(b[j].astype(np.float64) - ref)) / np.max(np.abs(ref)))
                say(f"  seq {s} len {L}: noalloc == allocating, rel err vs oracle {e:.2e}")
                assert e <= 1e-4


def test_noalloc_refuses_batches_beyond_the_scratch():
    """64 sequences at 8192 cached rows need ~17 MB of partials (> 16 MiB):
    refused before any launch; the allocating entry point still serves it."""
    n, L = 64, 8192
    with q35mix.Context(q35mix.qwen35_config(num_layers=1, is_recurrent=[0]), n_seqs=n, kv_capacity=L + 1) as c:
        c.set_attn_weights(0, synth.attn_weights(HD, salt=6))
        for s in range(n):
            c.advance(s, L)
        x = synth.attn_inputs(n, NH, NKV, HD, salt=63)
        qg, kk, vv = c.array((n, 2 * c.q_dim), x["q_gate"]), c.array((n, c.kv_dim), x["k"]), \
            c.array((n, c.kv_dim), x["v"])
        out = c.array((n, c.q_dim))
        with pytest.raises(q35mix.Q35Error) as e:
            c.attn_decode_noalloc(0, list(range(n)), qg, kk, vv, out)
        assert e.value.code == q35mix.ERR_CAPACITY
        say(f"refused: {e.value}")
        c.attn_decode(0, list(range(n)), qg, kk, vv, out)
        assert np.isfinite(out.download()).all()


def test_noalloc_under_graph_capture():
    """The no-allocation entry point captured into a HIP graph on the
    context's stream: three replays, with eager copies and synchronisations
    between them, each equal bit for bit to the eager call (same inputs, same
    position: the same new cache row and output)."""
    hip = q35mix.hip()
    L = 3000
    with q35mix.Context(q35mix.qwen35_config(num_layers=1, is_recurrent=[0]), n_seqs=1, kv_capacity=L + 1) as c:
        c.set_attn_weights(0, synth.attn_weights(HD, salt=8))
        k, v = synth.kv_prefill(L, KV_DIM, salt=9)
        c.state_write(0, 0, q35mix.STATE_KEYS, k)
        c.state_write(0, 0, q35mix.STATE_VALUES, v)
        c.advance(0, L)
        x = synth.attn_inputs(1, NH, NKV, HD, salt=10)
        qg, kk, vv = c.array((1, 2 * c.q_dim), x["q_gate"]), c.array((1, c.kv_dim), x["k"]), \
            c.array((1, c.kv_dim), x["v"])
        out = c.array((1, c.q_dim))
        c.attn_decode_noalloc(0, [0], qg, kk, vv, out)
        c.sync()
        ref = out.download()
        stream = ctypes.c_void_p(c.stream)
        graph, exe = ctypes.c_void_p(), ctypes.c_void_p()
        assert hip.hipStreamBeginCapture(stream, 0) == 0          # hipStreamCaptureModeGlobal
        try:
            c.attn_decode_noalloc(0, [0], qg, kk, vv, out)
        finally:
            r_end = hip.hipStreamEndCapture(stream, ctypes.byref(graph))
        assert r_end == 0
        assert hip.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, ctypes.c_size_t(0)) == 0
        try:
            for rep in range(3):
                out.upload(np.zeros((1, c.q_dim), np.float32))    # eager work between replays
                c.sync()
                assert hip.hipGraphLaunch(exe, stream) == 0
                c.sync()
                got = out.download()
                assert bits_equal(got, ref), rep
        finally:
            hip.hipGraphExecDestroy(exe)
            hip.hipGraphDestroy(graph)
