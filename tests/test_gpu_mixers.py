"""Parity of the HIP mixers (through the C ABI) with the CPU oracle.

Tolerance: max|gpu - oracle| / max|oracle| <= 1e-4 per tensor for fp32
outputs and states (the stated fp32 gate); conv windows and V rows are pure
copies and must match bit for bit.
"""
import sys

import numpy as np
import pytest

import oracle
import q35mix
import synth

pytestmark = pytest.mark.gpu

TOL = 1e-4
NK, NV = 16, 32
NH, NKV, HD = 16, 4, 256


def rel(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    # Layers 0-2 Gated-DeltaNet, layer 3 GQA; 4 sequences; 8200 KV rows.
    c = q35mix.Context(q35mix.qwen35_config(num_layers=4), n_seqs=4, kv_capacity=8200)
    for layer in range(3):
        c.set_deltanet_weights(layer, synth.deltanet_weights(NK, NV, 128, salt=layer))
    c.set_attn_weights(3, synth.attn_weights(HD))
    yield c
    c.close()


DIMS = oracle.dims()


# --------------------------------------------------------------------------
# Gated-DeltaNet decode
# --------------------------------------------------------------------------

def _dn_decode_case(ctx, layer, seqs, salt0, steps=1):
    w = synth.deltanet_weights(NK, NV, 128, salt=layer)
    states = {}
    for j, s in enumerate(seqs):
        st = synth.deltanet_state(NK, NV, 128, salt=salt0 + j)
        ctx.state_write(layer, s, q35mix.STATE_RECURRENT, st["state"])
        ctx.state_write(layer, s, q35mix.STATE_CONV, st["conv_state"])
        states[s] = (st["conv_state"], st["state"])
    n = len(seqs)
    for step in range(steps):
        x = synth.deltanet_inputs(n, NK, NV, 128, salt=salt0 + 100 + step)
        qkv, z = ctx.array((n, ctx.conv_dim), x["qkv"]), ctx.array((n, ctx.value_dim), x["z"])
        b, a = ctx.array((n, NV), x["b"]), ctx.array((n, NV), x["a"])
        out = ctx.array((n, ctx.value_dim))
        ctx.deltanet_decode(layer, seqs, qkv, z, b, a, out)
        got = out.download()
        for j, s in enumerate(seqs):
            cs, st = states[s]
            o_ref, cs_ref, st_ref, _ = oracle.deltanet_decode(DIMS, x["qkv"][j], x["z"][j],
                                                              x["b"][j], x["a"][j], w, cs, st)
            states[s] = (cs_ref, st_ref)
            e = rel(got[j], o_ref)
            say(f"deltanet_decode step {step} seq {s}: out rel err {e:.2e}")
            assert e <= TOL
    for s in seqs:
        cs_ref, st_ref = states[s]
        st_gpu = ctx.state_read(layer, s, q35mix.STATE_RECURRENT)
        cs_gpu = ctx.state_read(layer, s, q35mix.STATE_CONV)
        e = rel(st_gpu, st_ref)
        say(f"deltanet_decode seq {s}: state rel err {e:.2e}")
        assert e <= TOL
        np.testing.assert_array_equal(cs_gpu, cs_ref)


def test_deltanet_decode_single(ctx):
    """One token, one sequence at the full layer shape (16 k / 32 v heads)."""
    _dn_decode_case(ctx, 0, [0], salt0=1)


def test_deltanet_decode_batch_and_steps(ctx):
    """Three sequences batched in one launch, four chained tokens."""
    _dn_decode_case(ctx, 1, [2, 0, 3], salt0=10, steps=4)


# --------------------------------------------------------------------------
# Gated-DeltaNet prefill
# --------------------------------------------------------------------------

def _dn_prefill_case(ctx, layer, seq, T, salt, zero_state=True):
    w = synth.deltanet_weights(NK, NV, 128, salt=layer)
    st = synth.deltanet_state(NK, NV, 128, salt=salt)
    state0 = np.zeros_like(st["state"]) if zero_state else st["state"]
    ctx.state_write(layer, seq, q35mix.STATE_RECURRENT, state0)
    ctx.state_write(layer, seq, q35mix.STATE_CONV, st["conv_state"])
    x = synth.deltanet_inputs(T, NK, NV, 128, salt=salt + 50)
    qkv, z = ctx.array((T, ctx.conv_dim), x["qkv"]), ctx.array((T, ctx.value_dim), x["z"])
    b, a = ctx.array((T, NV), x["b"]), ctx.array((T, NV), x["a"])
    out = ctx.array((T, ctx.value_dim))
    ctx.deltanet_prefill(layer, seq, T, qkv, z, b, a, out)
    got = out.download()
    o_ref, cs_ref, st_ref, _ = oracle.deltanet_prefill(DIMS, T, x["qkv"], x["z"], x["b"], x["a"],
                                                       w, state0, st["conv_state"])
    e_out = rel(got, o_ref)
    e_st = rel(ctx.state_read(layer, seq, q35mix.STATE_RECURRENT), st_ref)
    say(f"deltanet_prefill T={T}: out rel err {e_out:.2e}, state rel err {e_st:.2e}")
    assert e_out <= TOL
    assert e_st <= TOL
    np.testing.assert_array_equal(ctx.state_read(layer, seq, q35mix.STATE_CONV), cs_ref)


@pytest.mark.parametrize("T", [1, 2, 3, 17, 64, 130])
def test_deltanet_prefill_small(ctx, T):
    _dn_prefill_case(ctx, 2, 1, T, salt=200 + T)


def test_deltanet_prefill_continues_state(ctx):
    """Prefill from a non-zero recurrent state (continuation prefill)."""
    _dn_prefill_case(ctx, 2, 3, 77, salt=300, zero_state=False)


def test_deltanet_prefill_2048(ctx):
    """T = 2048 from a zero state, full layer shape."""
    _dn_prefill_case(ctx, 0, 2, 2048, salt=400)


# --------------------------------------------------------------------------
# GQA attention decode / prefill
# --------------------------------------------------------------------------

def _fill_kv(ctx, seq, n_rows, salt):
    k, v = synth.kv_prefill(n_rows, ctx.kv_dim, salt=salt)
    ctx.state_write(3, seq, q35mix.STATE_KEYS, k)
    ctx.state_write(3, seq, q35mix.STATE_VALUES, v)
    ctx.truncate(seq, 0)
    ctx.advance(seq, n_rows)
    return k, v


def test_attn_decode_8192(ctx):
    """One token at position 8192 over a pre-filled 8192-row cache."""
    seq = 0
    ctx.reset(seq)
    k, v = _fill_kv(ctx, seq, 8192, salt=5)
    x = synth.attn_inputs(1, NH, NKV, HD, salt=6)
    wts = synth.attn_weights(HD)
    qg, kk, vv = ctx.array((1, 2 * ctx.q_dim), x["q_gate"]), ctx.array((1, ctx.kv_dim), x["k"]), \
        ctx.array((1, ctx.kv_dim), x["v"])
    out = ctx.array((1, ctx.q_dim))
    ctx.attn_decode(3, [seq], qg, kk, vv, out)
    got = out.download()[0]
    ck = np.zeros((8193, ctx.kv_dim), np.float32)
    cv = np.zeros_like(ck)
    ck[:8192], cv[:8192] = k, v
    o_ref, ck_ref, cv_ref = oracle.attn_decode(DIMS, 8192, x["q_gate"][0], x["k"][0], x["v"][0],
                                               wts, ck, cv, n_threads=8)
    e = rel(got, o_ref)
    say(f"attn_decode pos 8192: out rel err {e:.2e}")
    assert e <= TOL
    kr = ctx.state_read(3, seq, q35mix.STATE_KEYS, rows=8193)
    vr = ctx.state_read(3, seq, q35mix.STATE_VALUES, rows=8193)
    assert rel(kr[8192], ck_ref[8192]) <= TOL
    np.testing.assert_array_equal(vr[8192], cv_ref[8192])
    np.testing.assert_array_equal(kr[:8192], k)


def test_attn_decode_ragged_batch(ctx):
    """Three sequences at different lengths (1, 37, 700) in one launch."""
    seqs, lens = [1, 2, 3], [0, 37, 700]
    wts = synth.attn_weights(HD)
    caches = {}
    for s, L in zip(seqs, lens):
        ctx.reset(s)
        if L:
            caches[s] = _fill_kv(ctx, s, L, salt=20 + s)
        else:
            caches[s] = (np.zeros((0, ctx.kv_dim), np.float32),) * 2
    x = synth.attn_inputs(3, NH, NKV, HD, salt=7)
    qg, kk, vv = ctx.array((3, 2 * ctx.q_dim), x["q_gate"]), ctx.array((3, ctx.kv_dim), x["k"]), \
        ctx.array((3, ctx.kv_dim), x["v"])
    out = ctx.array((3, ctx.q_dim))
    ctx.attn_decode(3, seqs, qg, kk, vv, out)
    got = out.download()
    for j, (s, L) in enumerate(zip(seqs, lens)):
        ck = np.zeros((L + 1, ctx.kv_dim), np.float32)
        cv = np.zeros_like(ck)
        ck[:L], cv[:L] = caches[s]
        o_ref, _, _ = oracle.attn_decode(DIMS, L, x["q_gate"][j], x["k"][j], x["v"][j], wts, ck,
                                         cv, n_threads=8)
        e = rel(got[j], o_ref)
        say(f"attn_decode seq {s} len {L}: out rel err {e:.2e}")
        assert e <= TOL


@pytest.mark.parametrize("start,T", [(0, 5), (0, 64), (100, 37), (0, 2048)])
def test_attn_prefill(ctx, start, T):
    seq = 2
    ctx.reset(seq)
    k0 = v0 = None
    if start:
        k0, v0 = _fill_kv(ctx, seq, start, salt=40)
    wts = synth.attn_weights(HD)
    x = synth.attn_inputs(T, NH, NKV, HD, salt=8 + T)
    qg, kk, vv = ctx.array((T, 2 * ctx.q_dim), x["q_gate"]), ctx.array((T, ctx.kv_dim), x["k"]), \
        ctx.array((T, ctx.kv_dim), x["v"])
    out = ctx.array((T, ctx.q_dim))
    ctx.attn_prefill(3, seq, T, qg, kk, vv, out)
    got = out.download()
    ck = np.zeros((start + T, ctx.kv_dim), np.float32)
    cv = np.zeros_like(ck)
    if start:
        ck[:start], cv[:start] = k0, v0
    o_ref, ck_ref, cv_ref = oracle.attn_prefill(DIMS, start, T, x["q_gate"], x["k"], x["v"], wts,
                                                ck, cv, n_threads=8)
    e = rel(got, o_ref)
    say(f"attn_prefill start {start} T {T}: out rel err {e:.2e}")
    assert e <= TOL
    kr = ctx.state_read(3, seq, q35mix.STATE_KEYS, rows=start + T)
    vr = ctx.state_read(3, seq, q35mix.STATE_VALUES, rows=start + T)
    assert rel(kr[start:], ck_ref[start:]) <= TOL
    np.testing.assert_array_equal(vr[start:], x["v"])


def test_attn_prefill_then_decode_is_one_longer_prefill(ctx):
    """Attention has no conv quirk: prefill(T) + decode(1) == prefill(T+1)."""
    wts = synth.attn_weights(HD)
    T = 50
    x = synth.attn_inputs(T + 1, NH, NKV, HD, salt=60)
    full = ctx.array((T + 1, ctx.q_dim))
    ctx.reset(0)
    ctx.attn_prefill(3, 0, T + 1, ctx.array((T + 1, 2 * ctx.q_dim), x["q_gate"]),
                     ctx.array((T + 1, ctx.kv_dim), x["k"]), ctx.array((T + 1, ctx.kv_dim), x["v"]),
                     full)
    ctx.reset(1)
    part = ctx.array((T, ctx.q_dim))
    ctx.attn_prefill(3, 1, T, ctx.array((T, 2 * ctx.q_dim), x["q_gate"][:T]),
                     ctx.array((T, ctx.kv_dim), x["k"][:T]), ctx.array((T, ctx.kv_dim), x["v"][:T]),
                     part)
    ctx.advance(1, T)
    last = ctx.array((1, ctx.q_dim))
    ctx.attn_decode(3, [1], ctx.array((1, 2 * ctx.q_dim), x["q_gate"][T:]),
                    ctx.array((1, ctx.kv_dim), x["k"][T:]), ctx.array((1, ctx.kv_dim), x["v"][T:]),
                    last)
    f = full.download()
    assert rel(part.download(), f[:T]) <= 1e-5
    assert rel(last.download()[0], f[T]) <= 1e-5


# --------------------------------------------------------------------------
# lifecycle
# --------------------------------------------------------------------------

def test_state_roundtrip_and_reset(ctx):
    st = synth.deltanet_state(NK, NV, 128, salt=77)
    ctx.state_write(0, 3, q35mix.STATE_RECURRENT, st["state"])
    ctx.state_write(0, 3, q35mix.STATE_CONV, st["conv_state"])
    np.testing.assert_array_equal(ctx.state_read(0, 3, q35mix.STATE_RECURRENT), st["state"])
    np.testing.assert_array_equal(ctx.state_read(0, 3, q35mix.STATE_CONV), st["conv_state"])
    ctx.advance(3, 5)
    ctx.reset(3)
    assert ctx.kv_len(3) == 0
    assert not ctx.state_read(0, 3, q35mix.STATE_RECURRENT).any()
    assert not ctx.state_read(0, 3, q35mix.STATE_CONV).any()


def test_truncate_refuses_to_extend(ctx):
    ctx.reset(0)
    ctx.advance(0, 10)
    ctx.truncate(0, 4)
    assert ctx.kv_len(0) == 4
    with pytest.raises(q35mix.Q35Error) as ei:
        ctx.truncate(0, 5)
    assert ei.value.code == q35mix.ERR_RANGE
    with pytest.raises(q35mix.Q35Error) as ei:
        ctx.advance(0, 10 ** 6)
    assert ei.value.code == q35mix.ERR_CAPACITY
    with pytest.raises(q35mix.Q35Error) as ei:
        ctx.deltanet_decode(3, [0], *[ctx.array((1, 8))] * 5)   # layer 3 is full attention
    assert ei.value.code == q35mix.ERR_INVALID


@pytest.mark.parametrize("lens", [[16383, 9000, 100, 16000], [8192, 8000, 5000, 7000]])
def test_attn_decode_long_batch(lens):
    """Four sequences at long contexts: exercises the multi-sub-chunk partial
    kernel (4 and 2 sub-chunks of 64 rows per workgroup) and a long merge."""
    n = len(lens)
    with q35mix.Context(q35mix.qwen35_config(num_layers=1, is_recurrent=[0]), n_seqs=n,
                        kv_capacity=16400) as c:
        wts = synth.attn_weights(HD, salt=3)
        c.set_attn_weights(0, wts)
        caches = []
        for s, L in enumerate(lens):
            k, v = synth.kv_prefill(L, c.kv_dim, salt=70 + s)
            c.state_write(0, s, q35mix.STATE_KEYS, k)
            c.state_write(0, s, q35mix.STATE_VALUES, v)
            c.advance(s, L)
            caches.append((k, v))
        x = synth.attn_inputs(n, NH, NKV, HD, salt=9)
        qg, kk, vv = c.array((n, 2 * c.q_dim), x["q_gate"]), c.array((n, c.kv_dim), x["k"]), \
            c.array((n, c.kv_dim), x["v"])
        out = c.array((n, c.q_dim))
        c.attn_decode(0, list(range(n)), qg, kk, vv, out)
        got = out.download()
        for s, L in enumerate(lens):
            ck = np.zeros((L + 1, c.kv_dim), np.float32)
            cv = np.zeros_like(ck)
            ck[:L], cv[:L] = caches[s]
            o_ref, _, _ = oracle.attn_decode(DIMS, L, x["q_gate"][s], x["k"][s], x["v"][s], wts,
                                             ck, cv, n_threads=8)
            e = rel(got[s], o_ref)
            say(f"attn_decode long batch seq {s} len {L}: out rel err {e:.2e}")
            assert e <= TOL


@pytest.mark.parametrize("n", [16, 32])
def test_deltanet_decode_wide_batch(n):
    """16 and 32 sequences in one launch (512 and 1024 workgroups), three
    chained tokens, so the double-buffered conv windows flip three times."""
    with q35mix.Context(q35mix.qwen35_config(num_layers=1, is_recurrent=[1]), n_seqs=n,
                        kv_capacity=4) as c:
        c.set_deltanet_weights(0, synth.deltanet_weights(NK, NV, 128, salt=0))
        _dn_decode_case(c, 0, list(range(n))[::-1], salt0=300 + n, steps=3)


def test_deltanet_prefill_then_decode(ctx):
    """Prefill of 5 tokens, two decode steps, a second prefill (which ignores
    the stored window but rewrites it) and one more decode step, on one
    sequence: the window each step reads is the one the previous step left."""
    layer, s = 0, 2
    w = synth.deltanet_weights(NK, NV, 128, salt=layer)
    st = synth.deltanet_state(NK, NV, 128, salt=77)
    ctx.state_write(layer, s, q35mix.STATE_RECURRENT, st["state"])
    ctx.state_write(layer, s, q35mix.STATE_CONV, st["conv_state"])
    cs_ref, st_ref = st["conv_state"], st["state"]
    for step, T in enumerate([5, 1, 1, 3, 1]):
        x = synth.deltanet_inputs(T, NK, NV, 128, salt=900 + step)
        qkv, z = ctx.array((T, ctx.conv_dim), x["qkv"]), ctx.array((T, ctx.value_dim), x["z"])
        b, a = ctx.array((T, NV), x["b"]), ctx.array((T, NV), x["a"])
        out = ctx.array((T, ctx.value_dim))
        if step in (0, 3):
            ctx.deltanet_prefill(layer, s, T, qkv, z, b, a, out)
            o_ref, cs_ref, st_ref, _ = oracle.deltanet_prefill(DIMS, T, x["qkv"], x["z"], x["b"],
                                                               x["a"], w, st_ref, cs_ref)
        else:
            ctx.deltanet_decode(layer, [s], qkv, z, b, a, out)
            o_ref, cs_ref, st_ref, _ = oracle.deltanet_decode(DIMS, x["qkv"][0], x["z"][0],
                                                              x["b"][0], x["a"][0], w, cs_ref,
                                                              st_ref)
        e = rel(out.download().reshape(np.shape(o_ref)), o_ref)
        say(f"deltanet prefill/decode chain step {step} (T={T}): out rel err {e:.2e}")
        assert e <= TOL
        np.testing.assert_array_equal(ctx.state_read(layer, s, q35mix.STATE_CONV), cs_ref)
    assert rel(ctx.state_read(layer, s, q35mix.STATE_RECURRENT), st_ref) <= TOL
