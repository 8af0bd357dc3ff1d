"""Parity at the decode shapes of the 32-layer mixer stack (8 sequences at
context ~32K) and at every split the decode attention picks.

- The decode attention at 8 sequences x up to 32767 cached rows runs
  attn_decode_partial<8> (asserted through the per-kernel timers) and matches
  the oracle for every sequence, a ragged batch with a 1-row sequence included.
- Each split variant (1, 4 or 8 sub-chunks of 64 rows per workgroup, and 4
  or up to 8 sub-chunks of 16 rows for small batches at long contexts) is
  selected by a shape that
  the selection rule maps to it, asserted the same way, and matches the
  oracle, ragged batches with 0- and 1-row sequences included; sequences
  with no cached rows take only the new row.
- A reduced stack (3 Gated-DeltaNet layers + 1 GQA layer, 8 sequences, KV
  pre-filled to ~32,700 rows, 3 batched decode steps) matches the oracle in
  every layer's output after every step and in the final recurrent states,
  conv windows and K/V rows.

Tolerance: max|gpu - oracle| / max|oracle| <= 1e-4 per tensor (fp32); conv
windows and V rows are copies and must match bit for bit.  Cache rows are
N(0,1) values tiled from one seeded block of normals at per-sequence
offsets (drawing 33 M fresh normals per sequence would dominate the test).
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
KV_DIM = NKV * HD
DIMS = oracle.dims()
_BLOCK = []


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def rel(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def fill_rows(dst, off):
    """dst [rows][KV_DIM] <- the seeded block of normals, tiled from offset off
    (the block length is not a multiple of a row, so rows do not repeat)."""
    if not _BLOCK:
        _BLOCK.append(synth.normal(4321, 4_000_037))
    b = _BLOCK[0]
    flat = dst.reshape(-1)
    o, p = 0, off % b.size
    while o < flat.size:
        n = min(b.size - p, flat.size - o)
        flat[o:o + n] = b[p:p + n]
        o += n
        p = 0


def variant_ran(c):
    names = [k for k in c.profile_read() if k.startswith("attn_decode_partial<")]
    assert len(names) == 1, names
    return names[0][len("attn_decode_partial<"):-1]


def attn_batch_case(lens, salt, cap=None):
    """One batched decode-attention call over sequences holding `lens` cached
    rows; returns the split variant that ran."""
    n = len(lens)
    cap = cap or max(lens) + 1
    with q35mix.Context(q35mix.qwen35_config(num_layers=1, is_recurrent=[0]), n_seqs=n,
                        kv_capacity=cap) as c:
        wts = synth.attn_weights(HD, salt=salt)
        c.set_attn_weights(0, wts)
        caches = []
        for s, L in enumerate(lens):
            ck = np.empty((L + 1, KV_DIM), np.float32)
            cv = np.empty_like(ck)
            fill_rows(ck, 7919 * (2 * s) + salt)
            fill_rows(cv, 7919 * (2 * s + 1) + salt)
            if L:
                c.state_write(0, s, q35mix.STATE_KEYS, ck[:L])
                c.state_write(0, s, q35mix.STATE_VALUES, cv[:L])
                c.advance(s, L)
            caches.append((ck, cv))
        x = synth.attn_inputs(n, NH, NKV, HD, salt=salt)
        qg, kk, vv = c.array((n, 2 * c.q_dim), x["q_gate"]), c.array((n, c.kv_dim), x["k"]), \
            c.array((n, c.kv_dim), x["v"])
        out = c.array((n, c.q_dim))
        say(f"attn_decode batch lens {lens}: launching")
        c.profile(True)
        c.attn_decode(0, list(range(n)), qg, kk, vv, out)
        ran = variant_ran(c)
        c.profile(False)
        got = out.download()
        for s, L in enumerate(lens):
            ck, cv = caches[s]
            o_ref, _, _ = oracle.attn_decode(DIMS, L, x["q_gate"][s], x["k"][s], x["v"][s], wts,
                                             ck, cv, n_threads=8, inplace=True)
            e = rel(got[s], o_ref)
            say(f"  seq {s} len {L}: out rel err {e:.2e} (split {ran})")
            assert e <= TOL
            if L < 64:
                # new row written into the cache (whole rows, so read 1..L+1)
                kr = c.state_read(0, s, q35mix.STATE_KEYS, L + 1)[L]
                vr = c.state_read(0, s, q35mix.STATE_VALUES, L + 1)[L]
                assert rel(kr, ck[L]) <= TOL
                np.testing.assert_array_equal(vr, cv[L])
    return ran


def test_attn_decode_long_context_split8():
    """8 sequences up to 32767 cached rows (the stack's shape, ragged, with a
    1-row sequence): the 8-sub-chunk split, checked per sequence."""
    lens = [32700, 30011, 28417, 24576, 20480, 16384, 32767, 1]
    ran = attn_batch_case(lens, salt=11, cap=32768)
    assert ran == "8"
    assert q35mix.attn_decode_variant(8, NKV, lens, q35mix.cu_count()) == "8"


SPLIT_SHAPES = [[8192], [8193], [8320], [16384], [8192, 8192], [8000, 7000, 8000, 6000], [0, 5, 4095],
                [0, 0], [1], [64, 65, 127, 128], [2000, 1999, 37], [4000, 0], [4000, 1], [32767]]


@pytest.mark.parametrize("lens", SPLIT_SHAPES)
def test_attn_decode_split_variants(lens):
    """Shapes whose selected split is 1 or 4 sub-chunks of 64 rows, or 4 or
    up to 8 of 16 rows per workgroup (the batch-1 8192-row shape and the
    lengths just past it among them), sequences with no cached rows, and
    cached lengths at and around sub-chunk boundaries."""
    want = q35mix.attn_decode_variant(len(lens), NKV, lens, q35mix.cu_count())
    ran = attn_batch_case(lens, salt=20 + len(lens))
    assert ran == want, (ran, want)


def test_attn_decode_variants_cover_all_splits():
    """The parametrized shapes above reach every split on this device."""
    cu = q35mix.cu_count()
    shapes = SPLIT_SHAPES + [[32700, 30011, 28417, 24576, 20480, 16384, 32767, 1]]
    got = {q35mix.attn_decode_variant(len(x), NKV, x, cu) for x in shapes}
    assert got == {"1", "4", "8", "4,16", "8,16"}, (cu, got)


def test_reduced_stack_long_context():
    """3 Gated-DeltaNet layers + 1 GQA layer, 8 sequences, KV pre-filled to
    ~32,700 rows (ragged), 3 decode steps with all 8 sequences in each
    layer's launch; every output, then the states, windows and K/V rows."""
    n = 8
    cap = 32768
    lens = [32700 - 13 * s for s in range(n)]
    steps = 3
    is_rec = [1, 1, 1, 0]
    c = q35mix.Context(q35mix.qwen35_config(num_layers=4, is_recurrent=is_rec), n_seqs=n, kv_capacity=cap)
    try:
        wd = [synth.deltanet_weights(NK, NV, 128, salt=60 + l) for l in range(3)]
        wa = synth.attn_weights(HD, salt=63)
        for l in range(3):
            c.set_deltanet_weights(l, wd[l])
        c.set_attn_weights(3, wa)
        dn = {}                       # (layer, seq) -> (conv window, state)
        for l in range(3):
            for s in range(n):
                st = synth.deltanet_state(NK, NV, 128, salt=100 * l + s)
                c.state_write(l, s, q35mix.STATE_RECURRENT, st["state"])
                c.state_write(l, s, q35mix.STATE_CONV, st["conv_state"])
                dn[l, s] = (st["conv_state"], st["state"])
        kv = []
        say("reduced stack: filling 8 KV caches")
        for s, L in enumerate(lens):
            ck = np.empty((L + steps, KV_DIM), np.float32)
            cv = np.empty_like(ck)
            fill_rows(ck, 104729 * s + 1)
            fill_rows(cv, 104729 * s + 2)
            c.state_write(3, s, q35mix.STATE_KEYS, ck[:L])
            c.state_write(3, s, q35mix.STATE_VALUES, cv[:L])
            c.advance(s, L)
            kv.append((ck, cv))
        seqs = list(range(n))
        for step in range(steps):
            xd = synth.deltanet_inputs(n, NK, NV, 128, salt=700 + step)
            xa = synth.attn_inputs(n, NH, NKV, HD, salt=800 + step)
            dargs = [c.array((n, c.conv_dim), xd["qkv"]), c.array((n, c.value_dim), xd["z"]),
                     c.array((n, NV), xd["b"]), c.array((n, NV), xd["a"])]
            aargs = [c.array((n, 2 * c.q_dim), xa["q_gate"]), c.array((n, c.kv_dim), xa["k"]),
                     c.array((n, c.kv_dim), xa["v"])]
            for l in range(4):
                say(f"reduced stack step {step} layer {l}: launching")
                if is_rec[l]:
                    out = c.array((n, c.value_dim))
                    c.deltanet_decode(l, seqs, *dargs, out)
                    got = out.download()
                    for s in seqs:
                        cs, st = dn[l, s]
                        o_ref, cs, st, _ = oracle.deltanet_decode(DIMS, xd["qkv"][s], xd["z"][s], xd["b"][s],
                                                                  xd["a"][s], wd[l], cs, st)
                        dn[l, s] = (cs, st)
                        e = rel(got[s], o_ref)
                        assert e <= TOL, (step, l, s, e)
                else:
                    out = c.array((n, c.q_dim))
                    c.profile(True)
                    c.attn_decode(l, seqs, *aargs, out)
                    ran = variant_ran(c)
                    c.profile(False)
                    got = out.download()
                    for s in seqs:
                        ck, cv = kv[s]
                        o_ref, _, _ = oracle.attn_decode(DIMS, lens[s] + step, xa["q_gate"][s], xa["k"][s],
                                                         xa["v"][s], wa, ck, cv, n_threads=8, inplace=True)
                        e = rel(got[s], o_ref)
                        assert e <= TOL, (step, l, s, e)
                    say(f"  GQA layer: split {ran}, all 8 sequences within {TOL}")
            for s in seqs:
                c.advance(s, 1)
        say("reduced stack: final states")
        for l in range(3):
            for s in seqs:
                cs, st = dn[l, s]
                assert rel(c.state_read(l, s, q35mix.STATE_RECURRENT), st) <= TOL
                np.testing.assert_array_equal(c.state_read(l, s, q35mix.STATE_CONV), cs)
        for s, L in enumerate(lens):
            ck, cv = kv[s]
            keys = c.state_read(3, s, q35mix.STATE_KEYS, L + steps)
            vals = c.state_read(3, s, q35mix.STATE_VALUES, L + steps)
            np.testing.assert_array_equal(keys[:L], ck[:L])
            assert rel(keys[L:], ck[L:L + steps]) <= TOL
            np.testing.assert_array_equal(vals, cv[:L + steps])
    finally:
        c.close()
