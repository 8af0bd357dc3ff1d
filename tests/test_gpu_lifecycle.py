"""KV and state lifecycle through the C ABI: the linear-state snapshot rolls a
sequence back so that the same decode steps give bit-identical outputs
again (the reference's TruncateCache cannot roll the recurrent state back),
restore refuses after a truncate, and KV growth keeps every row and length:
a context grown from 16 to 64 rows decodes bit-identically to one created
with 64."""
import sys

import numpy as np
import pytest

import q35mix
import synth

pytestmark = pytest.mark.gpu

NK, NV = 16, 32
NH, NKV, HD = 16, 4, 256


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def make_ctx(cap, n_seqs=2):
    c = q35mix.Context(q35mix.qwen35_config(num_layers=2, is_recurrent=[1, 0]), n_seqs=n_seqs,
                       kv_capacity=cap)
    c.set_deltanet_weights(0, synth.deltanet_weights(NK, NV, 128, salt=31))
    c.set_attn_weights(1, synth.attn_weights(HD, salt=31))
    return c


def step(c, seq, xd, xa, i):
    """One decode step of both layers for one sequence; returns both outputs."""
    od, oa = c.array((1, c.value_dim)), c.array((1, c.q_dim))
    c.deltanet_decode(0, [seq], c.array((1, c.conv_dim), xd["qkv"][i:i + 1]),
                      c.array((1, c.value_dim), xd["z"][i:i + 1]), c.array((1, NV), xd["b"][i:i + 1]),
                      c.array((1, NV), xd["a"][i:i + 1]), od)
    c.attn_decode(1, [seq], c.array((1, 2 * c.q_dim), xa["q_gate"][i:i + 1]),
                  c.array((1, c.kv_dim), xa["k"][i:i + 1]), c.array((1, c.kv_dim), xa["v"][i:i + 1]), oa)
    c.advance(seq, 1)
    return od.download(), oa.download()


def bits_equal(a, b):
    return np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))


def test_snapshot_rolls_back_state():
    say("snapshot rollback")
    c = make_ctx(64)
    xd = synth.deltanet_inputs(12, NK, NV, 128, salt=71)
    xa = synth.attn_inputs(12, NH, NKV, HD, salt=72)
    for i in range(5):
        step(c, 1, xd, xa, i)
    buf, info = c.snapshot_save(1)
    assert info.kv_len == 5
    first = [step(c, 1, xd, xa, i) for i in range(5, 9)]
    assert c.kv_len(1) == 9
    c.snapshot_restore(1, buf, info)
    assert c.kv_len(1) == 5
    again = [step(c, 1, xd, xa, i) for i in range(5, 9)]
    for (d1, a1), (d2, a2) in zip(first, again):
        assert bits_equal(d1, d2) and bits_equal(a1, a2)
    # without the restore the continuation differs (the state really moved on)
    other = step(c, 1, xd, xa, 5)
    assert not bits_equal(other[0], first[0][0])
    c.snapshot_restore(1, buf, info)            # still valid: no truncate since
    c.truncate(1, 4)
    with pytest.raises(q35mix.Q35Error) as e:
        c.snapshot_restore(1, buf, info)
    assert e.value.code == q35mix.ERR_RANGE
    buf.free()
    c.close()


def test_grow_keeps_rows_and_lengths():
    say("grow 16 -> 64")
    a, b = make_ctx(16), make_ctx(64)
    xd = synth.deltanet_inputs(40, NK, NV, 128, salt=81)
    xa = synth.attn_inputs(40, NH, NKV, HD, salt=82)
    for i in range(12):
        for s in (0, 1):
            assert all(bits_equal(u, v) for u, v in zip(step(a, s, xd, xa, i), step(b, s, xd, xa, i)))
    with pytest.raises(q35mix.Q35Error):
        a.grow(8)
    a.grow(64)
    for i in range(12, 40):
        for s in (0, 1):
            assert all(bits_equal(u, v) for u, v in zip(step(a, s, xd, xa, i), step(b, s, xd, xa, i)))
    for s in (0, 1):
        assert a.kv_len(s) == b.kv_len(s) == 40
        assert bits_equal(a.state_read(1, s, q35mix.STATE_KEYS, 40), b.state_read(1, s, q35mix.STATE_KEYS, 40))
    a.close()
    b.close()


def test_grow_extends_rope_table():
    """Growing past the 4096 positions the RoPE table starts with rebuilds it:
    a decode at position 4100 matches a context created with 8192 rows."""
    say("grow 4096 -> 8192 (RoPE table rebuilt)")
    a, b = make_ctx(4096, n_seqs=1), make_ctx(8192, n_seqs=1)
    a.grow(8192)
    k, v = synth.kv_prefill(4100, a.kv_dim, salt=91)
    for c in (a, b):
        c.state_write(1, 0, q35mix.STATE_KEYS, k)
        c.state_write(1, 0, q35mix.STATE_VALUES, v)
        c.advance(0, 4100)
    xd = synth.deltanet_inputs(2, NK, NV, 128, salt=92)
    xa = synth.attn_inputs(2, NH, NKV, HD, salt=93)
    for i in range(2):
        assert all(bits_equal(u, w) for u, w in zip(step(a, 0, xd, xa, i), step(b, 0, xd, xa, i)))
    a.close()
    b.close()
