"""KV and state lifecycle through the C ABI, every decode step checked against
the oracle run from host copies of the same state: the linear-state snapshot
rolls a sequence back so that the same decode steps give bit-identical
outputs again (the reference's TruncateCache cannot roll the recurrent state
back); restore refuses after a truncate, and a snapshot taken at a longer
length is refused once a restore to a shorter length has let the rows above
it be written again; KV growth keeps every row and length (a context grown
from 16 to 64 rows decodes like one created with 64, and like the oracle),
also past the 4096 positions the RoPE table starts with."""
import sys

import numpy as np
import pytest

import oracle
import q35mix
import synth

pytestmark = pytest.mark.gpu

NK, NV = 16, 32
NH, NKV, HD = 16, 4, 256
TOL = 1e-4
DIMS = oracle.dims()
WD = synth.deltanet_weights(NK, NV, 128, salt=31)
WA = synth.attn_weights(HD, salt=31)


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def rel(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def make_ctx(cap, n_seqs=2):
    c = q35mix.Context(q35mix.qwen35_config(num_layers=2, is_recurrent=[1, 0]), n_seqs=n_seqs,
                       kv_capacity=cap)
    c.set_deltanet_weights(0, WD)
    c.set_attn_weights(1, WA)
    return c


class OracleSeq:
    """One sequence of the 2-layer (DeltaNet, GQA) model on the CPU oracle:
    the linear state, the conv window, the K/V rows and the length."""

    def __init__(self, cap, k=None, v=None):
        self.cs = np.zeros((2 * NK * 128 + NV * 128, 3), np.float32)
        self.st = np.zeros((NV, 128, 128), np.float32)
        self.ck = np.zeros((cap, NKV * HD), np.float32)
        self.cv = np.zeros((cap, NKV * HD), np.float32)
        self.len = 0
        if k is not None:
            self.ck[:len(k)], self.cv[:len(v)] = k, v
            self.len = len(k)

    def step(self, xd, xa, i):
        od, self.cs, self.st, _ = oracle.deltanet_decode(DIMS, xd["qkv"][i], xd["z"][i], xd["b"][i],
                                                         xd["a"][i], WD, self.cs, self.st)
        oa, self.ck, self.cv = oracle.attn_decode(DIMS, self.len, xa["q_gate"][i], xa["k"][i], xa["v"][i],
                                                  WA, self.ck, self.cv)
        self.len += 1
        return od, oa

    def save(self):
        return self.cs.copy(), self.st.copy(), self.len

    def restore(self, snap):
        cs, st, n = snap
        self.cs, self.st, self.len = cs.copy(), st.copy(), n


def step(c, seq, xd, xa, i, ref=None):
    """One decode step of both layers for one sequence; returns both outputs.
    With ref (an OracleSeq), the outputs are checked against the oracle's."""
    od, oa = c.array((1, c.value_dim)), c.array((1, c.q_dim))
    c.deltanet_decode(0, [seq], c.array((1, c.conv_dim), xd["qkv"][i:i + 1]),
                      c.array((1, c.value_dim), xd["z"][i:i + 1]), c.array((1, NV), xd["b"][i:i + 1]),
                      c.array((1, NV), xd["a"][i:i + 1]), od)
    c.attn_decode(1, [seq], c.array((1, 2 * c.q_dim), xa["q_gate"][i:i + 1]),
                  c.array((1, c.kv_dim), xa["k"][i:i + 1]), c.array((1, c.kv_dim), xa["v"][i:i + 1]), oa)
    c.advance(seq, 1)
    got = od.download(), oa.download()
    if ref is not None:
        assert c.kv_len(seq) == ref.len + 1
        rd, ra = ref.step(xd, xa, i)
        e1, e2 = rel(got[0][0], rd), rel(got[1][0], ra)
        assert e1 <= TOL and e2 <= TOL, (seq, i, e1, e2)
    return got


def bits_equal(a, b):
    return np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))


def test_snapshot_rolls_back_state():
    say("snapshot rollback (oracle-checked)")
    c = make_ctx(64)
    ref = OracleSeq(64)
    xd = synth.deltanet_inputs(12, NK, NV, 128, salt=71)
    xa = synth.attn_inputs(12, NH, NKV, HD, salt=72)
    for i in range(5):
        step(c, 1, xd, xa, i, ref)
    buf, info = c.snapshot_save(1)
    snap = ref.save()
    assert info.kv_len == 5
    first = [step(c, 1, xd, xa, i, ref) for i in range(5, 9)]
    assert c.kv_len(1) == 9
    c.snapshot_restore(1, buf, info)
    ref.restore(snap)
    assert c.kv_len(1) == 5
    # the restored state and window are the oracle's at length 5
    assert rel(c.state_read(0, 1, q35mix.STATE_RECURRENT), ref.st) <= TOL
    np.testing.assert_array_equal(c.state_read(0, 1, q35mix.STATE_CONV), ref.cs)
    again = [step(c, 1, xd, xa, i, ref) for i in range(5, 9)]
    for (d1, a1), (d2, a2) in zip(first, again):
        assert bits_equal(d1, d2) and bits_equal(a1, a2)
    # without the restore the continuation differs (the state really moved on)
    other = step(c, 1, xd, xa, 5, ref)
    assert not bits_equal(other[0], first[0][0])
    c.snapshot_restore(1, buf, info)            # still valid: the restore above cut the length only to its own
    c.truncate(1, 4)
    with pytest.raises(q35mix.Q35Error) as e:
        c.snapshot_restore(1, buf, info)
    assert e.value.code == q35mix.ERR_RANGE
    buf.free()
    c.close()


def test_restore_refuses_a_longer_snapshot_after_rewind():
    """Save A at length 5, step to 9, save B, restore A, step 4 other tokens to
    length 9: B's linear state belongs to rows 5-8 that were overwritten, so
    restoring B is refused; A stays restorable and decodes like the oracle."""
    say("snapshot A/B rewind")
    c = make_ctx(64)
    ref = OracleSeq(64)
    xd = synth.deltanet_inputs(9, NK, NV, 128, salt=75)
    xa = synth.attn_inputs(9, NH, NKV, HD, salt=76)
    xd2 = synth.deltanet_inputs(9, NK, NV, 128, salt=77)
    xa2 = synth.attn_inputs(9, NH, NKV, HD, salt=78)
    for i in range(5):
        step(c, 0, xd, xa, i, ref)
    buf_a, info_a = c.snapshot_save(0)
    snap_a = ref.save()
    for i in range(5, 9):
        step(c, 0, xd, xa, i, ref)
    buf_b, info_b = c.snapshot_save(0)
    c.snapshot_restore(0, buf_a, info_a)
    ref.restore(snap_a)
    for i in range(5, 9):
        step(c, 0, xd2, xa2, i, ref)
    assert c.kv_len(0) == 9
    with pytest.raises(q35mix.Q35Error) as e:
        c.snapshot_restore(0, buf_b, info_b)
    assert e.value.code == q35mix.ERR_RANGE
    c.snapshot_restore(0, buf_a, info_a)
    ref.restore(snap_a)
    step(c, 0, xd, xa, 5, ref)
    # a rejected K/V write leaves snapshots valid
    with pytest.raises(q35mix.Q35Error):
        c.state_write(1, 0, q35mix.STATE_KEYS, np.zeros((1, 7), np.float32))
    c.snapshot_restore(0, buf_a, info_a)
    buf_a.free()
    buf_b.free()
    c.close()


def test_grow_keeps_rows_and_lengths():
    say("grow 16 -> 64 (oracle-checked)")
    a, b = make_ctx(16), make_ctx(64)
    refs = [OracleSeq(64), OracleSeq(64)]
    xd = synth.deltanet_inputs(40, NK, NV, 128, salt=81)
    xa = synth.attn_inputs(40, NH, NKV, HD, salt=82)
    for i in range(12):
        for s in (0, 1):
            assert all(bits_equal(u, v) for u, v in zip(step(a, s, xd, xa, i, refs[s]), step(b, s, xd, xa, i)))
    with pytest.raises(q35mix.Q35Error):
        a.grow(8)
    a.grow(64)
    for i in range(12, 40):
        for s in (0, 1):
            assert all(bits_equal(u, v) for u, v in zip(step(a, s, xd, xa, i, refs[s]), step(b, s, xd, xa, i)))
    for s in (0, 1):
        assert a.kv_len(s) == b.kv_len(s) == 40
        keys = a.state_read(1, s, q35mix.STATE_KEYS, 40)
        assert bits_equal(keys, b.state_read(1, s, q35mix.STATE_KEYS, 40))
        assert rel(keys, refs[s].ck[:40]) <= TOL
        np.testing.assert_array_equal(a.state_read(1, s, q35mix.STATE_VALUES, 40), refs[s].cv[:40])
    a.close()
    b.close()


def test_grow_extends_rope_table():
    """Growing past the 4096 positions the RoPE table starts with rebuilds it:
    decodes at positions 4100 and 4101 match the oracle (which builds its own
    table) and a context created with 8192 rows."""
    say("grow 4096 -> 8192 (RoPE table rebuilt, oracle-checked)")
    a, b = make_ctx(4096, n_seqs=1), make_ctx(8192, n_seqs=1)
    a.grow(8192)
    k, v = synth.kv_prefill(4100, a.kv_dim, salt=91)
    ref = OracleSeq(8192, k, v)
    for c in (a, b):
        c.state_write(1, 0, q35mix.STATE_KEYS, k)
        c.state_write(1, 0, q35mix.STATE_VALUES, v)
        c.advance(0, 4100)
    xd = synth.deltanet_inputs(2, NK, NV, 128, salt=92)
    xa = synth.attn_inputs(2, NH, NKV, HD, salt=93)
    for i in range(2):
        assert all(bits_equal(u, w) for u, w in zip(step(a, 0, xd, xa, i, ref), step(b, 0, xd, xa, i)))
    # the new K rows carry the rotation of positions 4100 and 4101
    assert rel(a.state_read(1, 0, q35mix.STATE_KEYS, 4102)[4100:], ref.ck[4100:4102]) <= TOL
    a.close()
    b.close()


def test_prefix_reuse_plan_with_snapshots():
    """Prompt reuse as Qwen35Model.AlignPrompt does it (KvCacheAlign.Plan),
    with the linear state rolled back too: a sequence holding tokens 10..17
    (snapshots at lengths 3 and 6), then the prompt 10..14, 20, 21.  The
    reference's plan keeps 5 tokens; q35m_reuse_plan picks the snapshot at 3,
    and restoring it and decoding prompt[3:] matches the oracle run of the
    prompt from scratch at every step, while truncating to 5 alone (the
    reference's TruncateCache) would keep the state of all 8 cached tokens."""
    say("prefix reuse with snapshots")
    xd = synth.deltanet_inputs(16, NK, NV, 128, salt=91)
    xa = synth.attn_inputs(16, NH, NKV, HD, salt=92)
    row = lambda tok: tok - 10   # noqa: E731  (token id -> its input row)
    c = make_ctx(64)
    cached = list(range(10, 18))
    snaps = {}
    ref = OracleSeq(64)
    for i, tok in enumerate(cached):
        step(c, 0, xd, xa, row(tok), ref)
        if i + 1 in (3, 6):
            snaps[i + 1] = c.snapshot_save(0)
    st_after_cached = c.state_read(0, 0, q35mix.STATE_RECURRENT)
    prompt = [10, 11, 12, 13, 14, 20, 21]
    assert q35mix.reuse_plan(cached, prompt)[:2] == (5, 5)
    lens = sorted(snaps)
    keep, start, idx = q35mix.reuse_plan(cached, prompt, lens)
    assert (keep, start) == (3, 3) and lens[idx] == 3
    buf, info = snaps[lens[idx]]
    c.snapshot_restore(0, buf, info)
    assert c.kv_len(0) == 3
    # The oracle from scratch over the prompt: its first 3 tokens, then the rest.
    fresh = OracleSeq(64)
    for tok in prompt[:start]:
        fresh.step(xd, xa, row(tok))
    assert rel(c.state_read(0, 0, q35mix.STATE_RECURRENT), fresh.st) <= TOL
    assert not bits_equal(c.state_read(0, 0, q35mix.STATE_RECURRENT), st_after_cached)
    for tok in prompt[start:]:
        step(c, 0, xd, xa, row(tok), fresh)
    assert c.kv_len(0) == len(prompt)
    for b, _ in snaps.values():
        b.free()
    c.close()
