"""Edge cases of the HIP mixers through the C ABI: chunk counts that exercise
every branch of the prefill scan's loop, the 64-sequence decode batch, the
last KV row and the limits the ABI enforces.  Parity gate as in
test_gpu_mixers.py: max|gpu - oracle| / max|oracle| <= 1e-4."""
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
NSEQ, CAP = 64, 256
DIMS = oracle.dims()


def rel(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    # Layer 0 Gated-DeltaNet, layer 1 GQA; 64 sequences (the batch limit); 256 KV rows.
    c = q35mix.Context(q35mix.qwen35_config(num_layers=2, is_recurrent=[1, 0]), n_seqs=NSEQ,
                       kv_capacity=CAP)
    c.set_deltanet_weights(0, synth.deltanet_weights(NK, NV, 128, salt=31))
    c.set_attn_weights(1, synth.attn_weights(HD, salt=31))
    yield c
    c.close()


@pytest.mark.parametrize("T", [200, 600, 1030, 2049])
def test_deltanet_prefill_chunk_counts(ctx, T):
    """4, 10, 17 and 33 chunks (whole pairs of the scan loop, or one chunk
    left over; ragged last chunk at 1030 and 2049), from a non-zero state."""
    w = synth.deltanet_weights(NK, NV, 128, salt=31)
    st = synth.deltanet_state(NK, NV, 128, salt=500 + T)
    ctx.state_write(0, 5, q35mix.STATE_RECURRENT, st["state"])
    ctx.state_write(0, 5, q35mix.STATE_CONV, st["conv_state"])
    x = synth.deltanet_inputs(T, NK, NV, 128, salt=600 + T)
    args = [ctx.array((T, ctx.conv_dim), x["qkv"]), ctx.array((T, ctx.value_dim), x["z"]),
            ctx.array((T, NV), x["b"]), ctx.array((T, NV), x["a"])]
    out = ctx.array((T, ctx.value_dim))
    ctx.deltanet_prefill(0, 5, T, *args, out)
    o_ref, cs_ref, st_ref, _ = oracle.deltanet_prefill(DIMS, T, x["qkv"], x["z"], x["b"], x["a"],
                                                       w, st["state"], st["conv_state"])
    e_out = rel(out.download(), o_ref)
    e_st = rel(ctx.state_read(0, 5, q35mix.STATE_RECURRENT), st_ref)
    say(f"deltanet_prefill T={T}: out rel err {e_out:.2e}, state rel err {e_st:.2e}")
    assert e_out <= TOL and e_st <= TOL
    np.testing.assert_array_equal(ctx.state_read(0, 5, q35mix.STATE_CONV), cs_ref)


@pytest.mark.parametrize("T", [63, 65, 66, 67, 129])
def test_deltanet_prefill_chunk_tails(ctx, T):
    """Last chunk holding 63, 1, 2, 3 and 1 tokens: the conv's zero padding
    past T, the conv-window write-back from the raw inputs T-3..T-1 when they
    straddle a chunk boundary, and the masked gates of the padded tokens."""
    w = synth.deltanet_weights(NK, NV, 128, salt=31)
    st = synth.deltanet_state(NK, NV, 128, salt=1500 + T)
    ctx.state_write(0, 9, q35mix.STATE_RECURRENT, st["state"])
    ctx.state_write(0, 9, q35mix.STATE_CONV, st["conv_state"])
    x = synth.deltanet_inputs(T, NK, NV, 128, salt=1600 + T)
    args = [ctx.array((T, ctx.conv_dim), x["qkv"]), ctx.array((T, ctx.value_dim), x["z"]),
            ctx.array((T, NV), x["b"]), ctx.array((T, NV), x["a"])]
    out = ctx.array((T, ctx.value_dim))
    ctx.deltanet_prefill(0, 9, T, *args, out)
    o_ref, cs_ref, st_ref, _ = oracle.deltanet_prefill(DIMS, T, x["qkv"], x["z"], x["b"], x["a"],
                                                       w, st["state"], st["conv_state"])
    e_out = rel(out.download(), o_ref)
    e_st = rel(ctx.state_read(0, 9, q35mix.STATE_RECURRENT), st_ref)
    say(f"deltanet_prefill tail T={T}: out rel err {e_out:.2e}, state rel err {e_st:.2e}")
    assert e_out <= TOL and e_st <= TOL
    np.testing.assert_array_equal(ctx.state_read(0, 9, q35mix.STATE_CONV), cs_ref)


def test_decode_batch_of_64(ctx):
    """Both decode mixers with the full 64-sequence batch, ragged KV lengths."""
    seqs = list(range(NSEQ))
    w = synth.deltanet_weights(NK, NV, 128, salt=31)
    states = []
    for s in seqs:
        st = synth.deltanet_state(NK, NV, 128, salt=700 + s)
        ctx.state_write(0, s, q35mix.STATE_RECURRENT, st["state"])
        ctx.state_write(0, s, q35mix.STATE_CONV, st["conv_state"])
        states.append(st)
    x = synth.deltanet_inputs(NSEQ, NK, NV, 128, salt=800)
    out = ctx.array((NSEQ, ctx.value_dim))
    ctx.deltanet_decode(0, seqs, ctx.array((NSEQ, ctx.conv_dim), x["qkv"]),
                        ctx.array((NSEQ, ctx.value_dim), x["z"]), ctx.array((NSEQ, NV), x["b"]),
                        ctx.array((NSEQ, NV), x["a"]), out)
    got = out.download()
    worst = 0.0
    for j, s in enumerate(seqs):
        o_ref, cs_ref, st_ref, _ = oracle.deltanet_decode(DIMS, x["qkv"][j], x["z"][j], x["b"][j],
                                                          x["a"][j], w, states[j]["conv_state"],
                                                          states[j]["state"])
        worst = max(worst, rel(got[j], o_ref))
        if j % 21 == 0:
            assert rel(ctx.state_read(0, s, q35mix.STATE_RECURRENT), st_ref) <= TOL
            np.testing.assert_array_equal(ctx.state_read(0, s, q35mix.STATE_CONV), cs_ref)
    say(f"deltanet_decode batch 64: worst out rel err {worst:.2e}")
    assert worst <= TOL

    wts = synth.attn_weights(HD, salt=31)
    rng = np.random.default_rng(5)
    lens = [int(v) for v in rng.integers(0, CAP - 1, NSEQ)]
    caches = []
    for s, L in zip(seqs, lens):
        ctx.reset(s)
        k, v = synth.kv_prefill(max(L, 1), ctx.kv_dim, salt=900 + s)
        k, v = k[:L], v[:L]
        if L:
            ctx.state_write(1, s, q35mix.STATE_KEYS, k)
            ctx.state_write(1, s, q35mix.STATE_VALUES, v)
            ctx.advance(s, L)
        caches.append((k, v))
    xa = synth.attn_inputs(NSEQ, NH, NKV, HD, salt=901)
    out = ctx.array((NSEQ, ctx.q_dim))
    ctx.attn_decode(1, seqs, ctx.array((NSEQ, 2 * ctx.q_dim), xa["q_gate"]),
                    ctx.array((NSEQ, ctx.kv_dim), xa["k"]), ctx.array((NSEQ, ctx.kv_dim), xa["v"]),
                    out)
    got = out.download()
    worst = 0.0
    for j, L in enumerate(lens):
        ck = np.zeros((L + 1, ctx.kv_dim), np.float32)
        cv = np.zeros_like(ck)
        ck[:L], cv[:L] = caches[j]
        o_ref, _, _ = oracle.attn_decode(DIMS, L, xa["q_gate"][j], xa["k"][j], xa["v"][j], wts, ck,
                                         cv, n_threads=8)
        worst = max(worst, rel(got[j], o_ref))
    say(f"attn_decode batch 64: worst out rel err {worst:.2e}")
    assert worst <= TOL


def test_attn_decode_last_row_then_full(ctx):
    """The decode that writes the last KV row works; the next one reports a
    full cache (Q35M_ERR_CAPACITY) instead of writing past it."""
    s = 7
    ctx.reset(s)
    L = CAP - 1
    k, v = synth.kv_prefill(L, ctx.kv_dim, salt=950)
    ctx.state_write(1, s, q35mix.STATE_KEYS, k)
    ctx.state_write(1, s, q35mix.STATE_VALUES, v)
    ctx.advance(s, L)
    wts = synth.attn_weights(HD, salt=31)
    xa = synth.attn_inputs(1, NH, NKV, HD, salt=951)
    args = [ctx.array((1, 2 * ctx.q_dim), xa["q_gate"]), ctx.array((1, ctx.kv_dim), xa["k"]),
            ctx.array((1, ctx.kv_dim), xa["v"])]
    out = ctx.array((1, ctx.q_dim))
    ctx.attn_decode(1, [s], *args, out)
    ck = np.zeros((CAP, ctx.kv_dim), np.float32)
    cv = np.zeros_like(ck)
    ck[:L], cv[:L] = k, v
    o_ref, ck_ref, _ = oracle.attn_decode(DIMS, L, xa["q_gate"][0], xa["k"][0], xa["v"][0], wts,
                                          ck, cv, n_threads=8)
    assert rel(out.download()[0], o_ref) <= TOL
    assert rel(ctx.state_read(1, s, q35mix.STATE_KEYS)[L], ck_ref[L]) <= TOL
    ctx.advance(s, 1)
    with pytest.raises(q35mix.Q35Error) as ei:
        ctx.attn_decode(1, [s], *args, out)
    assert ei.value.code == q35mix.ERR_CAPACITY


def test_abi_limits(ctx):
    """Batch limit, repeated sequence ids, partial K/V rows, bad state kind."""
    a = ctx.array((1, 8))
    with pytest.raises(q35mix.Q35Error) as ei:
        ctx.deltanet_decode(0, list(range(NSEQ)) + [0], a, a, a, a, a)
    assert ei.value.code == q35mix.ERR_CAPACITY
    with pytest.raises(q35mix.Q35Error) as ei:
        ctx.deltanet_decode(0, [3, 3], a, a, a, a, a)
    assert ei.value.code == q35mix.ERR_INVALID
    with pytest.raises(q35mix.Q35Error) as ei:
        ctx.state_write(1, 0, q35mix.STATE_KEYS, np.zeros((3, 100), np.float32))
    assert ei.value.code == q35mix.ERR_INVALID
    with pytest.raises(q35mix.Q35Error) as ei:
        ctx.state_read(1, 0, 9)
    assert ei.value.code == q35mix.ERR_INVALID


def test_attn_prefill_row_limit():
    """The prefill flash kernel addresses a kv head's rows through a buffer
    descriptor (32-bit offsets): a prefill that would reach past 2^21 cached
    rows is refused with ERR_UNSUPPORTED before any work (the capacity check
    comes first, so the context holds 2^21 + 1 rows: 8 GiB of K/V)."""
    rows = (1 << 21) + 1
    c = q35mix.Context(q35mix.qwen35_config(num_layers=1, is_recurrent=[0]), n_seqs=1, kv_capacity=rows)
    try:
        c.set_attn_weights(0, synth.attn_weights(256))
        a = c.array((1, 8))
        with pytest.raises(q35mix.Q35Error) as ei:
            c.attn_prefill(0, 0, rows, a, a, a, a)
        assert ei.value.code == q35mix.ERR_UNSUPPORTED
    finally:
        c.close()


def test_deltanet_prefill_long_context():
    """T = 16421 (257 chunks: an odd count, the last holding 37 tokens) in a
    2 k-head / 4 v-head geometry, from a non-zero state: the chunk scan's
    recurrence over a long chain and the workspace offsets at large chunk
    counts, outputs of every token and the final state against the oracle."""
    nk, nv, T = 2, 4, 16421
    d = oracle.dims(n_k_heads=nk, n_v_heads=nv)
    cfg = q35mix.qwen35_config(num_layers=1, n_k_heads=nk, n_v_heads=nv, is_recurrent=[1])
    with q35mix.Context(cfg, n_seqs=1, kv_capacity=4) as c:
        w = synth.deltanet_weights(nk, nv, 128, salt=77)
        c.set_deltanet_weights(0, w)
        st = synth.deltanet_state(nk, nv, 128, salt=78)
        c.state_write(0, 0, q35mix.STATE_RECURRENT, st["state"])
        c.state_write(0, 0, q35mix.STATE_CONV, st["conv_state"])
        x = synth.deltanet_inputs(T, nk, nv, 128, salt=79)
        out = c.array((T, c.value_dim))
        say(f"deltanet_prefill long T={T}: launching")
        c.deltanet_prefill(0, 0, T, c.array((T, c.conv_dim), x["qkv"]), c.array((T, c.value_dim), x["z"]),
                           c.array((T, nv), x["b"]), c.array((T, nv), x["a"]), out)
        got = out.download()
        o_ref, cs_ref, st_ref, _ = oracle.deltanet_prefill(d, T, x["qkv"], x["z"], x["b"], x["a"], w,
                                                           st["state"], st["conv_state"])
        e_out = rel(got, o_ref)
        e_last = rel(got[-64:], o_ref[-64:])
        e_st = rel(c.state_read(0, 0, q35mix.STATE_RECURRENT), st_ref)
        say(f"  out rel err {e_out:.2e} (last chunk {e_last:.2e}), state rel err {e_st:.2e}")
        assert e_out <= TOL and e_last <= TOL and e_st <= TOL
        np.testing.assert_array_equal(c.state_read(0, 0, q35mix.STATE_CONV), cs_ref)
