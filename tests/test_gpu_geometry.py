"""Mixer geometries of other Qwen3.5-family sizes, through the C ABI against
the oracle: the gated GQA layer with 1, 2, 8, 16 and 24 q heads per kv head
(ModelConfig.NumHeads / NumKvHeads, ModelConfig.cs:19-31, are free in the
reference; the 4B shape has 4), decode over every split of the cached rows
(batch 1 at 8192 rows included) and prefill with a continuation; and the
Gated-DeltaNet layer with 1, 3 and 4 v-heads per k-head (SsmTimeStepRank /
SsmGroupCount), decode, prefill, and decode after the prefill.

Tolerance: max|gpu - oracle| / max|oracle| <= 1e-4 per tensor (fp32); V rows
and conv windows are copies and must match bit for bit.
"""
import sys

import numpy as np
import pytest

import oracle
import q35mix
import synth

pytestmark = pytest.mark.gpu

TOL = 1e-4
HD = 256


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def rel(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


GQA_SHAPES = [(4, 4), (8, 4), (16, 2), (32, 2), (24, 1), (48, 2)]


@pytest.mark.parametrize("nh,nkv", GQA_SHAPES)
def test_attention_group_sizes(nh, nkv):
    """Decode for 3 sequences with 0, 700 and 9000 cached rows (the 1- and
    multi-sub-chunk splits), then a 70-token prefill of a fresh sequence and a
    33-token continuation, each against the oracle; K rows within tolerance,
    V rows bit-exact."""
    g = nh // nkv
    say(f"GQA geometry: {nh} q heads, {nkv} kv heads (group {g})")
    d = oracle.dims(n_heads=nh, n_kv_heads=nkv)
    kv_dim = nkv * HD
    cfg = q35mix.qwen35_config(num_layers=1, num_heads=nh, num_kv_heads=nkv, is_recurrent=[0])
    lens = [0, 700, 9000]
    with q35mix.Context(cfg, n_seqs=4, kv_capacity=9100) as c:
        w = synth.attn_weights(HD, salt=g)
        c.set_attn_weights(0, w)
        caches = []
        for s, L in enumerate(lens):
            k, v = synth.kv_prefill(L + 1, kv_dim, salt=200 + 10 * g + s)
            if L:
                c.state_write(0, s, q35mix.STATE_KEYS, k[:L])
                c.state_write(0, s, q35mix.STATE_VALUES, v[:L])
                c.advance(s, L)
            caches.append((k, v))
        n = len(lens)
        x = synth.attn_inputs(n, nh, nkv, HD, salt=300 + g)
        out = c.array((n, nh * HD))
        c.attn_decode(0, list(range(n)), c.array((n, 2 * nh * HD), x["q_gate"]), c.array((n, kv_dim), x["k"]),
                      c.array((n, kv_dim), x["v"]), out)
        got = out.download()
        for s, L in enumerate(lens):
            ck = np.zeros((L + 1, kv_dim), np.float32)
            cv = np.zeros_like(ck)
            ck[:L], cv[:L] = caches[s][0][:L], caches[s][1][:L]
            ref, ck2, cv2 = oracle.attn_decode(d, L, x["q_gate"][s], x["k"][s], x["v"][s], w, ck, cv, n_threads=8)
            e = rel(got[s], ref)
            say(f"  decode seq {s} len {L}: out rel err {e:.2e}")
            assert e <= TOL
            assert rel(c.state_read(0, s, q35mix.STATE_KEYS, L + 1)[L], ck2[L]) <= TOL
            np.testing.assert_array_equal(c.state_read(0, s, q35mix.STATE_VALUES, L + 1)[L], cv2[L])
        # prefill of 70 tokens on sequence 3, then 33 more
        ck = np.zeros((103, kv_dim), np.float32)
        cv = np.zeros_like(ck)
        start = 0
        for T, salt in ((70, 400), (33, 401)):
            xp = synth.attn_inputs(T, nh, nkv, HD, salt=salt + g)
            outp = c.array((T, nh * HD))
            c.attn_prefill(0, 3, T, c.array((T, 2 * nh * HD), xp["q_gate"]), c.array((T, kv_dim), xp["k"]),
                           c.array((T, kv_dim), xp["v"]), outp)
            ref, ck, cv = oracle.attn_prefill(d, start, T, xp["q_gate"], xp["k"], xp["v"], w, ck, cv, n_threads=8)
            e = rel(outp.download(), ref)
            say(f"  prefill start {start} T {T}: out rel err {e:.2e}")
            assert e <= TOL
            c.advance(3, T)
            start += T
        assert rel(c.state_read(0, 3, q35mix.STATE_KEYS, start), ck[:start]) <= TOL
        np.testing.assert_array_equal(c.state_read(0, 3, q35mix.STATE_VALUES, start), cv[:start])


@pytest.mark.parametrize("nh,nkv", GQA_SHAPES)
def test_attention_group_sizes_batch1_long(nh, nkv):
    """Batch-1 decode at 8192 cached rows in each geometry: a split of
    pipelined 16-row sub-chunks (asserted through the kernel timers against
    the selection rule), for 1, 2 and 8 q heads a workgroup and groups of 16
    and 24 taken as two and three head groups of 8; output, new K row and V
    row against the oracle."""
    g = nh // nkv
    say(f"GQA geometry batch 1 long: {nh} q heads, {nkv} kv heads (group {g})")
    d = oracle.dims(n_heads=nh, n_kv_heads=nkv)
    kv_dim = nkv * HD
    cfg = q35mix.qwen35_config(num_layers=1, num_heads=nh, num_kv_heads=nkv, is_recurrent=[0])
    L = 8192
    with q35mix.Context(cfg, n_seqs=1, kv_capacity=L + 1) as c:
        w = synth.attn_weights(HD, salt=50 + g)
        c.set_attn_weights(0, w)
        k, v = synth.kv_prefill(L + 1, kv_dim, salt=500 + g)
        c.state_write(0, 0, q35mix.STATE_KEYS, k[:L])
        c.state_write(0, 0, q35mix.STATE_VALUES, v[:L])
        c.advance(0, L)
        x = synth.attn_inputs(1, nh, nkv, HD, salt=600 + g)
        out = c.array((1, nh * HD))
        c.profile(True)
        c.attn_decode(0, [0], c.array((1, 2 * nh * HD), x["q_gate"]), c.array((1, kv_dim), x["k"]),
                      c.array((1, kv_dim), x["v"]), out)
        ran = [n for n in c.profile_read() if n.startswith("attn_decode_partial<")]
        c.profile(False)
        want = q35mix.attn_decode_variant(1, nkv, [L], q35mix.cu_count(), q_per_kv=g)
        assert want in ("4,16", "8,16") and ran == [f"attn_decode_partial<{want}>"], (ran, want)
        ck = np.zeros((L + 1, kv_dim), np.float32)
        cv = np.zeros_like(ck)
        ck[:L], cv[:L] = k[:L], v[:L]
        ref, ck2, cv2 = oracle.attn_decode(d, L, x["q_gate"][0], x["k"][0], x["v"][0], w, ck, cv, n_threads=8)
        e = rel(out.download()[0], ref)
        say(f"  decode len {L}: out rel err {e:.2e}")
        assert e <= TOL
        assert rel(c.state_read(0, 0, q35mix.STATE_KEYS, L + 1)[L], ck2[L]) <= TOL
        np.testing.assert_array_equal(c.state_read(0, 0, q35mix.STATE_VALUES, L + 1)[L], cv2[L])


@pytest.mark.parametrize("nh,nkv", [(16, 2), (24, 1)])
def test_attention_group8_short_context(nh, nkv):
    """Groups of 8 q heads a workgroup at short contexts: the rows go as 4
    sub-chunks of 16 a workgroup (the one-sub-chunk kernel would need more
    than 256 VGPRs with 8 heads), asserted through the kernel timers; two
    sequences with 1 and 300 cached rows against the oracle."""
    g = nh // nkv
    d = oracle.dims(n_heads=nh, n_kv_heads=nkv)
    kv_dim = nkv * HD
    cfg = q35mix.qwen35_config(num_layers=1, num_heads=nh, num_kv_heads=nkv, is_recurrent=[0])
    lens = [1, 300]
    with q35mix.Context(cfg, n_seqs=2, kv_capacity=301) as c:
        w = synth.attn_weights(HD, salt=70 + g)
        c.set_attn_weights(0, w)
        caches = []
        for s, L in enumerate(lens):
            k, v = synth.kv_prefill(L + 1, kv_dim, salt=700 + 10 * g + s)
            c.state_write(0, s, q35mix.STATE_KEYS, k[:L])
            c.state_write(0, s, q35mix.STATE_VALUES, v[:L])
            c.advance(s, L)
            caches.append((k, v))
        x = synth.attn_inputs(2, nh, nkv, HD, salt=710 + g)
        out = c.array((2, nh * HD))
        c.profile(True)
        c.attn_decode(0, [0, 1], c.array((2, 2 * nh * HD), x["q_gate"]), c.array((2, kv_dim), x["k"]),
                      c.array((2, kv_dim), x["v"]), out)
        ran = [n for n in c.profile_read() if n.startswith("attn_decode_partial<")]
        c.profile(False)
        assert ran == ["attn_decode_partial<4,16>"], ran
        assert q35mix.attn_decode_variant(2, nkv, lens, q35mix.cu_count(), q_per_kv=g) == "4,16"
        got = out.download()
        for s, L in enumerate(lens):
            ck = np.zeros((L + 1, kv_dim), np.float32)
            cv = np.zeros_like(ck)
            ck[:L], cv[:L] = caches[s][0][:L], caches[s][1][:L]
            ref, _, _ = oracle.attn_decode(d, L, x["q_gate"][s], x["k"][s], x["v"][s], w, ck, cv, n_threads=8)
            e = rel(got[s], ref)
            say(f"  group {g} decode len {L}: out rel err {e:.2e}")
            assert e <= TOL


@pytest.mark.parametrize("nk,nv", [(16, 16), (8, 24), (8, 32)])
def test_deltanet_v_heads_per_k_head(nk, nv):
    """1, 3 and 4 v-heads per k-head: two chained decode steps of 2 sequences
    from random states, then a 130-token prefill (3 chunks, the last partial)
    continuing one of them, then a decode step after the prefill (every
    v-head reads the conv windows the prefill left); outputs and states within
    tolerance, conv windows bit-exact."""
    say(f"DeltaNet geometry: {nk} k heads, {nv} v heads")
    d = oracle.dims(n_k_heads=nk, n_v_heads=nv)
    cfg = q35mix.qwen35_config(num_layers=1, n_k_heads=nk, n_v_heads=nv, is_recurrent=[1])
    with q35mix.Context(cfg, n_seqs=2, kv_capacity=4) as c:
        w = synth.deltanet_weights(nk, nv, 128, salt=nk + nv)
        c.set_deltanet_weights(0, w)
        states = []
        for s in range(2):
            st = synth.deltanet_state(nk, nv, 128, salt=500 + s + nv)
            c.state_write(0, s, q35mix.STATE_RECURRENT, st["state"])
            c.state_write(0, s, q35mix.STATE_CONV, st["conv_state"])
            states.append((st["conv_state"], st["state"]))
        for step in range(2):
            x = synth.deltanet_inputs(2, nk, nv, 128, salt=600 + step + nv)
            out = c.array((2, c.value_dim))
            c.deltanet_decode(0, [0, 1], c.array((2, c.conv_dim), x["qkv"]), c.array((2, c.value_dim), x["z"]),
                              c.array((2, nv), x["b"]), c.array((2, nv), x["a"]), out)
            got = out.download()
            for s in range(2):
                ref, cs, st, _ = oracle.deltanet_decode(d, x["qkv"][s], x["z"][s], x["b"][s], x["a"][s], w,
                                                        *states[s])
                states[s] = (cs, st)
                e = rel(got[s], ref)
                say(f"  decode step {step} seq {s}: out rel err {e:.2e}")
                assert e <= TOL
        for s in range(2):
            assert rel(c.state_read(0, s, q35mix.STATE_RECURRENT), states[s][1]) <= TOL
            np.testing.assert_array_equal(c.state_read(0, s, q35mix.STATE_CONV), states[s][0])
        T = 130
        x = synth.deltanet_inputs(T, nk, nv, 128, salt=700 + nv)
        out = c.array((T, c.value_dim))
        c.deltanet_prefill(0, 1, T, c.array((T, c.conv_dim), x["qkv"]), c.array((T, c.value_dim), x["z"]),
                           c.array((T, nv), x["b"]), c.array((T, nv), x["a"]), out)
        ref, cs, st, _ = oracle.deltanet_prefill(d, T, x["qkv"], x["z"], x["b"], x["a"], w, states[1][1],
                                                 states[1][0])
        e_out, e_st = rel(out.download(), ref), rel(c.state_read(0, 1, q35mix.STATE_RECURRENT), st)
        say(f"  prefill T={T}: out rel err {e_out:.2e}, state rel err {e_st:.2e}")
        assert e_out <= TOL and e_st <= TOL
        np.testing.assert_array_equal(c.state_read(0, 1, q35mix.STATE_CONV), cs)
        x = synth.deltanet_inputs(1, nk, nv, 128, salt=800 + nv)
        out = c.array((1, c.value_dim))
        c.deltanet_decode(0, [1], c.array((1, c.conv_dim), x["qkv"]), c.array((1, c.value_dim), x["z"]),
                          c.array((1, nv), x["b"]), c.array((1, nv), x["a"]), out)
        ref, cs, st, _ = oracle.deltanet_decode(d, x["qkv"][0], x["z"][0], x["b"][0], x["a"][0], w, cs, st)
        e = rel(out.download()[0], ref)
        say(f"  decode after the prefill: out rel err {e:.2e}")
        assert e <= TOL
        assert rel(c.state_read(0, 1, q35mix.STATE_RECURRENT), st) <= TOL
        np.testing.assert_array_equal(c.state_read(0, 1, q35mix.STATE_CONV), cs)
